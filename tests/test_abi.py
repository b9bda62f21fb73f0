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
