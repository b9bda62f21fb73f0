"""The GEMM's LDS fragment reads are inline asm (k_gemm.hip,
DmaSlab::frag): the compiler does not know they are pending, so
nothing may read or overwrite their destination registers before the
kernel's own ``s_waitcnt lgkmcnt(N)`` has retired them.  This test compiles k_gemm.hip for gfx950 to
assembly and follows every control-flow path from each such read to the
wait.  CPU only (hipcc cross-compiles); about a minute."""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

from malus_amd import build as B

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def _regs(tok):
    m = re.match(r"v\[(\d+):(\d+)\]", tok.strip())
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)\b", tok.strip())
    return {int(m.group(1))} if m else set()


def _functions(asm):
    funcs, cur = [], None
    for line in asm.split("\n"):
        if re.match(r"^_Z\S+:", line):
            cur = (line.split(":")[0], [])
            funcs.append(cur)
        elif cur is not None:
            cur[1].append(line)
    return funcs


def _lgkm_wait(t):
    m = re.search(r"lgkmcnt\((\d+)\)", t)
    return int(m.group(1)) if m else None


def _hazards(name, body):
    """Walk every path from each inline-asm ds_read.  LDS operations retire
    in issue order, so ``s_waitcnt lgkmcnt(N)`` retires all but the last N
    outstanding ones; the read is done once it is retired.  Scalar memory
    loads also count against lgkmcnt but return out of order, so one issued
    while the read is outstanding is reported too."""
    insts, labels, in_asm = [], {}, False
    for line in body:
        t = line.strip()
        if t.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if t.startswith(";;#ASMEND"):
            in_asm = False
            continue
        m = re.match(r"^(\.LBB\w+):", line)
        if m:
            labels[m.group(1)] = len(insts)
            continue
        if not t or t.startswith(";") or t.startswith("."):
            continue
        insts.append((t, in_asm))
        if t.startswith("s_endpgm"):
            break
    # lgkmcnt is 4 bits: with 16 LDS operations issued after a read, any
    # lgkmcnt wait retires it, so counts past 16 are the same state (this
    # also bounds the walk around loops)
    cap = 16
    reads, found = 0, []
    for k, (t, a) in enumerate(insts):
        if not (a and t.startswith("ds_read")):
            continue
        reads += 1
        pend = _regs(t.split()[1].rstrip(","))
        # state: number of LDS operations issued after this read
        stack, seen = [(k + 1, 0)], set()
        while stack:
            j, after = stack.pop()
            while j < len(insts) and (j, after) not in seen:
                seen.add((j, after))
                tt, aa = insts[j]
                op = tt.split()[0]
                if op == "s_endpgm":
                    break
                if op == "s_waitcnt":
                    n = _lgkm_wait(tt)
                    if n is not None and after + 1 > n:  # this read is among the retired ones
                        break
                    j += 1
                    continue
                if op.startswith(("s_load", "s_buffer_load")):
                    found.append(f"{name}: scalar load while an LDS read is pending: {tt}")
                    break
                ops = [x for x in re.split(r",\s*", tt[len(op):].strip()) if x]
                used = set().union(*(_regs(x) for x in ops)) if ops else set()
                if op.startswith("ds_"):
                    if aa and op.startswith("ds_read") and not (used & pend):
                        after = min(after + 1, cap)
                        j += 1
                        continue
                    if not (used & pend):
                        after = min(after + 1, cap)
                        j += 1
                        continue
                if used & pend:
                    found.append(f"{name}: {tt}")
                    break
                if op == "s_branch":
                    j = labels[ops[0]]
                    continue
                if op.startswith("s_cbranch"):
                    stack.append((labels[ops[0]], after))
                j += 1
    return reads, found


def test_inline_asm_lds_reads_are_waited_for_before_use():
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    src = B.CSRC / "k_gemm.hip"
    with tempfile.TemporaryDirectory() as d:
        out = os.path.join(d, "k_gemm.s")
        cmd = [HIPCC, "-x", "hip", *B.COMMON, *B.DEVICE, "--cuda-device-only", "-S", "-I", str(B.CSRC), str(src),
               "-o", out]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        assert proc.returncode == 0, proc.stderr[-2000:]
        asm = open(out).read()
    total, bad = 0, []
    for name, body in _functions(asm):
        if "k_sgemm_dma" not in name:
            continue
        reads, found = _hazards(name, body)
        total += reads
        bad += found
    assert total > 100, "no inline-asm fragment reads found: the check is not looking at the right code"
    assert not bad, "registers of a pending LDS read used before its wait:\n" + "\n".join(bad[:10])
