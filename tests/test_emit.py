"""CPU tests of the HIP emitter (malus_compile_kernels): the emitted text,
the registry's id order, the kernel-language type rules, and hipRTC
compilation of every emitted kernel for gfx950 (no GPU needed).

The text checks follow the reference emitter's own unit tests
(crates/malus-codegen-gpu/src/tests.rs: builtin synthesis, id ordering,
uniforms struct, intrinsics injected only when used, shared memory,
barriers), restated for the HIP output.
"""
import ctypes as C
import glob
import os
import re

import pytest

import malus_amd as M
from tests.emit_programs import BUILTINS, PROGRAM, SIGMOID_BACKWARD

REF = "/root/reference"


def rtc(src):
    log = C.create_string_buffer(1 << 16)
    n = M.lib().malus_rtc_compile(src.encode(), b"gfx950", None, 0, log, len(log))
    assert n > 0, f"hipRTC rejected the emitted source:\n{src}\n{log.value.decode()}"
    return n


def emit_error(src, builtins=()):
    with pytest.raises(RuntimeError) as e:
        M.compile_kernels(src, builtins)
    return str(e.value)


def test_implicit_map_lowers_to_v1_out_tid():
    r = M.compile_kernels(SIGMOID_BACKWARD)
    (name, kid, src), = r.entries
    assert name == "sigmoid_backward"
    assert f"void malus_kernel_{kid}(const float* __restrict__ grad_out, const float* __restrict__ sig_z, " \
           "float* __restrict__ out, unsigned int n)" in src
    assert "if (tid >= n) return;" in src
    # binops fully parenthesized, left-associative order kept (lib.rs:540-546)
    assert "out[tid] = ((grad_out[tid] * sig_z[tid]) * (1.0f - sig_z[tid]));" in src
    rtc(src)


def test_ids_increase_user_kernels_first_then_builtins_in_reference_order():
    r = M.compile_kernels(PROGRAM + SIGMOID_BACKWARD, list(reversed(BUILTINS)))
    names = [n for n, _, _ in r.entries]
    ids = [i for _, i, _ in r.entries]
    assert ids == sorted(ids) and len(set(ids)) == len(ids)
    user = ["axpb", "nudge", "row_softmax", "bcast_sub", "transpose2", "gather_rows", "col_sum", "row_argmax",
            "math_mix", "sigmoid_backward"]
    assert names[:len(user)] == user
    # tensor-tensor in BinOp order, scalar in (op, scalar_on_right) order, unary by name
    assert names[len(user):] == ["malus_add", "malus_sub", "malus_mul", "malus_div", "malus_add_scalar",
                                 "malus_rsub_scalar", "malus_sub_scalar", "malus_mul_scalar", "malus_rdiv_scalar",
                                 "malus_div_scalar", "abs", "exp", "log", "relu", "sigmoid", "sqrt", "tanh"]
    # ids are process-global: a second compile never reuses one
    r2 = M.compile_kernels(SIGMOID_BACKWARD)
    assert r2.entries[0][1] > ids[-1]


def test_builtin_synthesis_text():
    r = M.compile_kernels("", BUILTINS)
    s = r.sources
    assert "out[tid] = (a[tid] / b[tid]);" in s["malus_div"]
    assert "out[tid] = (a[tid] - scalar_val[0]);" in s["malus_sub_scalar"]
    assert "out[tid] = (scalar_val[0] - a[tid]);" in s["malus_rsub_scalar"]
    assert "out[tid] = (scalar_val[0] / a[tid]);" in s["malus_rdiv_scalar"]
    assert s["malus_mul_scalar"].startswith("//@malus-v1-scalar-inputs 1\n")
    assert "out[tid] = fmaxf(0.0f, a[tid]);" in s["relu"]
    assert "1.0f / (1.0f + __malus_exp(-a[tid]))" in s["sigmoid"] and "(float)exp((double)x)" in s["sigmoid"]
    assert "__malus_tanh" not in s["exp"]  # only the helpers a kernel calls are emitted
    for src in s.values():
        rtc(src)


def test_explicit_kernel_abi_uniforms_meta_and_intrinsics():
    r = M.compile_kernels(PROGRAM)
    kid = r.ids["gather_rows"]
    src = r.sources["gather_rows"]
    assert src.startswith("//@malus-v2-uniform-bytes 8\n")
    # uniforms in declaration order, one 4-byte slot each
    assert re.search(r"struct Uniforms_%d \{\s*int dim;\s*int nrows;\s*\};" % kid, src)
    sig = src[src.index(f"malus_kernel_{kid}("):src.index(") {")]
    parts = [p.strip() for p in sig[sig.index("(") + 1:].split(",")]
    assert parts == ["const float* __restrict__ table", "const int* __restrict__ idx", "float* __restrict__ out",
                     f"Uniforms_{kid} u", "TensorMeta table_meta", "TensorMeta idx_meta", "TensorMeta out_meta"]
    assert "u.dim" in src and "u.nrows" in src
    # only the intrinsics a body uses are materialized
    assert "_tid = (int)(blockIdx.x * blockDim.x + threadIdx.x)" in src and "_tgid" not in src
    sm = r.sources["row_softmax"]
    assert "_tgid = (int)blockIdx.x" in sm and "_lid = (int)threadIdx.x" in sm and "_tgsize = (int)blockDim.x" in sm
    assert "_tid" not in sm
    assert "__shared__ float vals[1024];" in sm and "__syncthreads();" in sm and "while ((stride > 0)) {" in sm
    bs = r.sources["bcast_sub"]
    assert "(int)a_meta.ndim" in bs and "(int)a_meta.strides[d]" in bs and "(int)b_meta.shape[(d - lead)]" in bs
    assert "for (int d = 0; d < (int)a_meta.ndim; d++) {" in bs
    assert "x[(r) * (int)x_meta.strides[0] + (c) * (int)x_meta.strides[1]]" in r.sources["transpose2"]
    am = r.sources["row_argmax"]
    assert "int* __restrict__ out" in am and "int at = 0;" in am
    mm = r.sources["math_mix"]
    assert "__malus_pow(fabsf(b), 1.5f)" in mm and "__malus_rsqrt(" in mm and "__malus_sigmoid(b)" in mm
    assert "((!(a > 0.0f)) && (b < 0.0f))" in mm
    # no uniforms struct without scalar params
    assert "Uniforms_" not in r.sources["transpose2"] and "//@malus-v2-uniform-bytes 0" in r.sources["transpose2"]


def test_every_emitted_test_kernel_compiles_for_gfx950():
    r = M.compile_kernels(PROGRAM + SIGMOID_BACKWARD, BUILTINS)
    for name, _, src in r.entries:
        rtc(src)


def test_literals_keep_their_value():
    r = M.compile_kernels("""kernel lits(x: Tensor<f32>) -> Tensor<f32>:
    let i = thread_id()
    out[i] = x[i] * 0.7978845608028654 + 1e-5 - 2.5e10 + 3.0
""")
    src = r.sources["lits"]
    # the shortest digits that read back as the same double, then an f32 literal
    assert "0.7978845608028654f" in src and "1e-05f" in src and "2.5e+10f" in src and "3.0f" in src
    rtc(src)


def test_tags_mark_the_kernels_the_runtime_implements():
    r = M.compile_kernels("""kernel __softmax_kernel(x: Tensor<f32>, axis_size: i32, inner_u: i32) -> Tensor<f32>:
    let i = thread_id()
    out[i] = x[i]
kernel mine(x: Tensor<f32>) -> Tensor<f32>:
    let i = thread_id()
    out[i] = x[i]
""", ["malus_add", "relu"], tags=True)
    s = r.sources
    assert s["__softmax_kernel"].startswith("//@malus-builtin __softmax_kernel\n")
    assert s["malus_add"].startswith("//@malus-builtin malus_add\n")
    assert s["relu"].startswith("//@malus-builtin relu\n")
    assert "//@malus-builtin" not in s["mine"]
    untagged = M.compile_kernels("kernel __eq_kernel(a: Tensor<f32>) -> Tensor<f32>:\n    return a\n")
    assert "//@malus-builtin" not in untagged.sources["__eq_kernel"]


def test_form_selection_and_non_kernel_items_are_skipped():
    src = """struct S:
    a: i32

fn host(x: Tensor<f32>) -> Tensor<f32>:
    let y = x + x
    for i in range(3):
        println("{}", i)
    return y

kernel only(x: Tensor<f32>) -> Tensor<f32>:
    let a = x * 2.0
    return a

fn other():
    return 0
"""
    r = M.compile_kernels(src)
    assert list(r.ids) == ["only"]
    assert "(implicit map, v1 ABI)" in r.sources["only"]


@pytest.mark.parametrize("src,msg", [
    ("kernel k(x: Tensor<f32>) -> Tensor<f32>:\n    let i = thread_id()\n    out[i] = x[i] * 2\n", "type mismatch"),
    ("kernel k(x: Tensor<f32>) -> Tensor<f32>:\n    let i = thread_id()\n    let a = 1.0\n    a = 2.0\n    out[i] = a\n",
     "immutable"),
    ("kernel k(x: Tensor<f32>) -> Tensor<f32>:\n    let i = thread_id()\n    x[i] = 1.0\n    out[i] = 1.0\n", "immutable"),
    ("kernel k(x: Tensor<f32>) -> Tensor<f32>:\n    let i = thread_id()\n    out[i] = y[i]\n", "unknown identifier"),
    ("kernel k(x: Tensor<f32>) -> f32:\n    return x\n", "must return a tensor"),
    ("kernel k(x: Tensor<f32>) -> Tensor<f32>:\n    return exp(x)\n", "implicit-map"),
    ("kernel k(x: Tensor<f32>) -> Tensor<f32>:\n    let i = thread_id()\n    for j in range(3):\n        break\n"
     "    out[i] = x[i]\n", "not valid in explicit kernel body"),
    ("kernel k(x: Tensor<f32>) -> Tensor<f32>:\n    let i = thread_id()\n    out[i] = x.shape\n", "must be indexed"),
    ("kernel k(x: Tensor<f32>) -> Tensor<f32>:\n    let i = thread_id()\n    out[i] = frob(x[i])\n", "unsupported call"),
    ("kernel k(x: Tensor<f32>) -> Tensor<f32>:\n    let i = thread_id()\n    out[i] = x[i] ** x\n", "**"),
    ("kernel k(x: Tensor<f32>) -> Tensor<f32>:\n    let i = thread_id()\n    out[i] = x + x\n", "tensor operands"),
])
def test_type_and_form_errors(src, msg):
    assert msg in emit_error(src)


def test_unknown_builtin_is_an_error():
    assert "unknown builtin" in emit_error("", ["malus_pow"])


@pytest.mark.skipif(not os.path.isdir(REF), reason="the reference tree is only present in the build container")
def test_reference_kernel_corpus_lowers_and_compiles():
    """Every `kernel` item of the reference's stdlib and examples lowers and
    compiles with hipRTC for gfx950 (read from the reference tree at test
    time; nothing of it is kept in this repository)."""
    files = sorted(glob.glob(f"{REF}/crates/malus-stdlib/stdlib/**/*.ml", recursive=True))
    files += sorted(glob.glob(f"{REF}/examples/*.ml"))
    count = 0
    for f in files:
        text = open(f).read()
        if "\nkernel " not in "\n" + text:
            continue
        r = M.compile_kernels(text)
        for name, _, src in r.entries:
            rtc(src)
            count += 1
    assert count >= 36  # 30 stdlib kernels + the examples' user kernels


def test_mutated_programs_lower_or_fail_cleanly():
    """Malformed input: seeded truncations, deletions, insertions and byte
    substitutions of the test programs either lower to kernels or raise the
    emitter's error (a RuntimeError with the library's message); none ends
    the process, and the emitter keeps working afterwards."""
    import random

    rng = random.Random(2024)
    alphabet = " \n\t:()[]<>,.=+-*/%!&|^~#\"'abcxyz019_"
    bases = [PROGRAM, SIGMOID_BACKWARD]
    lowered = rejected = 0
    for _ in range(3000):
        q = rng.choice(bases)
        at = rng.randrange(len(q))
        kind = rng.randrange(4)
        if kind == 0:
            q = q[:at]
        elif kind == 1:
            q = q[:at] + rng.choice(alphabet) + q[at + 1:]
        elif kind == 2:
            q = q[:at] + q[at + 1 + rng.randrange(8):]
        else:
            q = q[:at] + rng.choice(alphabet) * (1 + rng.randrange(4)) + q[at:]
        try:
            r = M.compile_kernels(q, BUILTINS if rng.random() < 0.5 else ())
            assert all(src for _, _, src in r.entries)
            lowered += 1
        except RuntimeError as e:
            assert str(e), "an emitter error carries a message"
            rejected += 1
    assert lowered and rejected
    (name, _, _), = M.compile_kernels(SIGMOID_BACKWARD).entries
    assert name == "sigmoid_backward"


def test_implicit_kernels_declare_their_element_widths():
    # kernel_dispatch allocates the v1 output with input 0's dtype
    # (metal.rs:1878-1888); the emitted kernel states the widths it reads and
    # writes, and the runtime refuses a launch where they disagree (an f16
    # input 0 would give a 2-byte output that an f32 kernel overruns).
    prog = "kernel widen(a: Tensor<f16>, b: Tensor<f32>) -> Tensor<f32>:\n    return b\n"
    (name, kid, src), = M.compile_kernels(prog).entries
    assert "//@malus-v1-elem-bytes 4 2 4\n" in src
    rtc(src)
    (_, _, src), = M.compile_kernels(SIGMOID_BACKWARD).entries
    assert "//@malus-v1-elem-bytes 4 4 4\n" in src
    r = M.compile_kernels("", ["malus_add", "malus_mul_scalar", "exp"])
    for name, _, src in r.entries:
        want = "4 4" if name == "exp" else "4 4 4"
        assert f"//@malus-v1-elem-bytes {want}\n" in src, name
