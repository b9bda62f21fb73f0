"""CPU checks of the drop-in boundary: the C-ABI library builds, loads, and
exports every symbol include/malus_hip.h declares (no compute calls)."""
import ctypes as C
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "malus_hip.h")
LIB = os.path.join(ROOT, "malus_amd", "libmalus_hip.so")

# RuntimeSymbols (crates/malus-codegen-cpu/src/lib.rs:115-184) minus the
# string I/O group, which is host text I/O outside this backend.
RUNTIME_SYMBOLS = """tensor_alloc_gpu tensor_free tensor_print kernel_dispatch gpu_barrier tensor_alloc_zeros_gpu
tensor_alloc_ones_gpu tensor_matmul tensor_len tensor_retain tensor_release tape_record_binop tape_record_unary
tape_register_leaf tape_pause tape_resume tape_clear tape_get_grad backward tape_zero_grad tape_record_reduce
tensor_reshape tensor_permute tape_record_perm tensor_causal_mask tape_record_layernorm tape_record_cross_entropy
tensor_randn tape_record_embedding malus_rand_uniform malus_buffer_i32 malus_buffer_get_i32 malus_buffer_set_i32
malus_buffer_free malus_buffer_freeze_i32 malus_rand_int malus_tensor_get_f32 tensor_ndim tensor_dim
kernel_dispatch_v2 tape_register_backward_fn malus_record_diff bench_step_begin bench_step_end""".split()


def declared_functions():
    src = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    return sorted(set(re.findall(r"\b([a-z_][a-z0-9_]*)\s*\(", src)) - {"if", "for", "while", "sizeof"})


def exported_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


def test_header_compiles_as_c99(tmp_path):
    src = tmp_path / "h.c"
    src.write_text('#include "malus_hip.h"\nint main(void){return 0;}\n')
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.dirname(HEADER), "-c", str(src), "-o",
                    str(tmp_path / "h.o")], check=True)


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB), "build first: python -m malus_amd.build"
    missing = [n for n in declared_functions() if n not in exported_symbols()]
    assert not missing, f"declared but not exported: {missing}"


def test_runtime_symbols_of_the_jit_are_all_exported():
    missing = [n for n in RUNTIME_SYMBOLS if n not in exported_symbols()]
    assert not missing, missing
    assert set(RUNTIME_SYMBOLS) <= set(declared_functions())


def test_library_loads_and_ctypes_signatures_resolve():
    import malus_amd as M

    lib = M.lib()  # dlopen only: nothing here touches a device
    for name in M.SIGNATURES:
        assert getattr(lib, name) is not None


def test_library_carries_gfx950_code_objects():
    blob = open(LIB, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob  # offload bundle entry for the MI355X target


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is present; the no-device path cannot be exercised")
def test_no_device_fails_loudly_without_cpu_fallback():
    import malus_amd as M

    lib = M.lib()
    lib.malus_set_abort_on_error(0)
    try:
        lib.malus_init()
        assert b"no HIP device" in lib.malus_last_error()
        shape = (C.c_size_t * 1)(4)
        assert lib.tensor_alloc_zeros_gpu(shape, 1) == 0  # no silent host allocation either
    finally:
        lib.malus_set_abort_on_error(1)


FLOAT2_KERNEL = r"""
extern "C" __global__ void malus_kernel_7(const float2* a, const float2* b, float2* out, unsigned n) {
  unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float2 x = a[i], y = b[i];
  out[i] = make_float2(x.x * y.x + 1.0f, x.y * y.y + 1.0f);
}
"""


def rtc_compile(src, arch=b"gfx950"):
    import malus_amd as M

    lib = M.lib()
    log = C.create_string_buffer(1 << 16)
    n = lib.malus_rtc_compile(src.encode(), arch, None, 0, log, len(log))
    assert n > 0, log.value.decode()
    buf = C.create_string_buffer(n)
    assert lib.malus_rtc_compile(src.encode(), arch, buf, n, log, len(log)) == n
    return buf.raw


def test_runtime_compiled_kernels_use_no_packed_fp32(tmp_path):
    """User kernels go through hipRTC with the library's option list, which
    disables packed-FP32 instruction selection: a float2 multiply-add that
    would otherwise become v_pk_mul_f32 / v_pk_add_f32 must not (checked in
    the AMD disassembly of the code object compiled here)."""
    co = tmp_path / "k.co"
    co.write_bytes(rtc_compile(FLOAT2_KERNEL))
    objdump = "/opt/rocm/llvm/bin/llvm-objdump"
    if not os.path.exists(objdump):
        pytest.skip("llvm-objdump not available")
    asm = subprocess.run([objdump, "-d", str(co)], capture_output=True, text=True, check=True).stdout
    assert "v_mul_f32" in asm or "v_fma" in asm or "v_add_f32" in asm, "kernel body not found in the disassembly"
    assert not re.search(r"v_pk_(add|mul|fma)_f32", asm), "packed FP32 instructions in a runtime-compiled kernel"


def test_runtime_compile_reports_errors():
    import malus_amd as M

    log = C.create_string_buffer(1 << 14)
    n = M.lib().malus_rtc_compile(b"extern \"C\" __global__ void k() { undefined_name(); }", b"gfx950", None, 0, log,
                                  len(log))
    assert n == 0 and b"undefined_name" in log.value
