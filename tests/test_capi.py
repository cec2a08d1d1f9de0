"""The C-ABI library without a GPU: it loads, exports every entry point that
include/spbitnet_amd.h declares, and rejects bad arguments on the host
before any launch (these calls return before touching the HIP runtime)."""
import ctypes
import os
import re
import subprocess

import pytest

from tests.conftest import ROOT

HEADER = os.path.join(ROOT, "include", "spbitnet_amd.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(spb_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from spbitnet_amd import _lib
    return _lib.load()


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert len(names) >= 13
    from spbitnet_amd import _lib
    for n in names:
        assert hasattr(lib, n), f"{n} declared in spbitnet_amd.h but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (spb_[a-z0-9_]+)", out))
    assert set(names) <= exported
    assert exported <= set(names), f"undeclared exports: {exported - set(names)}"


def test_library_is_gfx950_only():
    """The embedded device code targets gfx950 and nothing else."""
    from spbitnet_amd import _lib
    blob = open(_lib.LIB_PATH, "rb").read()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa-[a-z-]*-?(gfx[0-9a-z]+)", blob))
    assert targets == {b"gfx950"}, targets


def test_abi_version(lib):
    assert lib.spb_abi_version() == 100


def test_host_validation_without_gpu(lib):
    g = lib.spb_sparse_ternary_gemv
    fake = ctypes.c_void_p(0x1000)
    # cols not a multiple of 4
    assert g(fake, fake, fake, fake, 4, 6, 1, 1, None) == 1
    assert b"multiple of 4" in lib.spb_last_error_string()
    # strides smaller than the format needs
    assert g(fake, fake, fake, fake, 4, 256, 7, 4, None) == 1
    assert b"meta_row_stride" in lib.spb_last_error_string()
    assert g(fake, fake, fake, fake, 4, 256, 8, 3, None) == 1
    # negative shape
    assert g(fake, fake, fake, fake, -1, 256, 8, 4, None) == 1
    # null pointers
    assert g(None, fake, fake, fake, 4, 256, 8, 4, None) == 1
    assert g(fake, fake, None, fake, 4, 256, 8, 4, None) == 1
    # rows == 0 / cols == 0 are successful no-ops, as in the reference
    assert g(fake, fake, fake, fake, 0, 256, 8, 4, None) == 0
    assert g(fake, fake, fake, fake, 4, 0, 0, 0, None) == 0
    assert lib.spb_sparse_ternary_unpack(fake, fake, fake, 0, 8, 1, 1, None) == 0
    assert lib.spb_fused_sparse_bitlinear_bf16(fake, fake, fake, None, fake, ctypes.c_float(1.0),
                                               4, 256, 8, 4, None) == 1
    assert lib.spb_absmax_reduce_bf16(fake, None, 16, None) == 1
    assert lib.spb_absmax_quantize_f16(fake, fake, fake, -3, None) == 1
    assert lib.spb_dequantize_bf16(fake, fake, fake, ctypes.c_float(1.0), 0, None) == 0
    # one-call BitLinear: workspace = 256 bytes of absmax + the planes (cols bytes, 32-rounded)
    assert lib.spb_bitlinear_workspace_size(2560) == 256 + 2560
    assert lib.spb_bitlinear_workspace_size(100) == 256 + 128
    assert lib.spb_bitlinear_workspace_size(0) == 0
    bl = lib.spb_bitlinear_bf16
    ws = ctypes.c_void_p(0x20000)
    assert bl(fake, fake, fake, fake, ctypes.c_float(1.0), 4, 256, 8, 4, ws, 511, None) == 1
    assert b"workspace" in lib.spb_last_error_string()
    assert bl(fake, fake, fake, fake, ctypes.c_float(1.0), 4, 256, 8, 4, None, 512, None) == 1
    assert bl(fake, fake, fake, fake, ctypes.c_float(1.0), 4, 256, 8, 4,
              ctypes.c_void_p(0x20004), 512, None) == 1  # not 16-byte aligned
    assert bl(fake, fake, fake, fake, ctypes.c_float(1.0), 4, 256, 7, 4, ws, 512, None) == 1
    assert bl(fake, fake, fake, fake, ctypes.c_float(1.0), 0, 256, 8, 4, None, 0, None) == 0


def test_gemv_kernel_selection(lib):
    kid = lib.spb_sparse_ternary_gemv_kernel_id
    a16 = ctypes.c_void_p(0x10000)
    assert kid(a16, a16, 6912, 2560, 80, 40) == 1
    assert kid(a16, a16, 2560, 6912, 216, 108) == 1
    assert kid(a16, a16, 64, 256, 8, 4) == 1
    assert kid(a16, a16, 64, 100, 4, 2) == 0        # cols % 128
    assert kid(a16, a16, 64, 256, 9, 4) == 0        # meta rows not 16-byte aligned
    assert kid(a16, a16, 64, 256, 8, 5) == 0        # values rows not 8-byte aligned
    assert kid(ctypes.c_void_p(0x10004), a16, 64, 256, 8, 4) == 0
    assert kid(a16, a16, 4, 65536, 2048, 1024) == 0  # beyond the bit-plane column limit


def test_gemm_kernel_selection(lib):
    kid = lib.spb_sparse_ternary_gemm_kernel_id
    a16, a4 = ctypes.c_void_p(0x10000), ctypes.c_void_p(0x10004)
    assert kid(a16, a16, a16, 6912, 2560, 64, 80, 40) == 2       # staged
    assert kid(a16, a16, a16, 2560, 6912, 16, 216, 108) == 2
    assert kid(a16, a16, a16, 64, 384, 16, 12, 6) == 1           # cols % 256 != 0: direct
    assert kid(a16, a16, a16, 64, 2560, 16, 81, 40) == 1         # meta stride % 4 != 0
    assert kid(a16, a16, a16, 64, 2560, 16, 80, 42) == 1         # values stride % 4 != 0
    assert kid(a4, a16, a16, 64, 2560, 16, 80, 40) == 1          # meta base not 16-byte aligned
    assert kid(a16, a16, a4, 64, 2560, 16, 80, 40) == 0          # X not 16-byte aligned: general
    assert kid(a16, a16, a16, 64, 100, 16, 4, 2) == 0            # cols % 128 != 0: general


def test_cpp_mirror_header_compiles_links_and_runs_noops(tmp_path):
    """include/spbitnet/sparse_ternary_kernels.h (the reference's C++ names
    over the C ABI) builds into a host program (ROCm clang, as hipcc uses for host code) and
    links the library."""
    from spbitnet_amd import _lib
    exe = tmp_path / "mirror_api"
    libdir = os.path.dirname(_lib.LIB_PATH)
    cmd = ["/opt/rocm/llvm/bin/clang++", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
           "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "cpp", "mirror_api.cpp"),
           "-L", libdir, "-lspbitnet_amd", f"-Wl,-rpath,{libdir}", "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "mirror api ok (abi 100)" in r.stdout
