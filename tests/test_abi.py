"""CPU-side checks of the drop-in boundary: the library loads, exports every
symbol include/m4_mlx_bridge.h declares, reproduces the reference's registry
values, and validates arguments with the reference's codes and order
(core/bridge/m4_mlx_bridge.mm:201-230; tests/redteam_bridge.py:151-471).
No kernel is launched here."""
from __future__ import annotations

import ctypes
import re

import numpy as np
import pytest

import m4_bridge
from conftest import ROOT


@pytest.fixture(scope="module")
def lib(libpath):
    return m4_bridge.load_library(libpath)


def test_exports_every_declared_symbol(lib):
    header = (ROOT / "include" / "m4_mlx_bridge.h").read_text()
    names = set(re.findall(r"^[A-Za-z_][\w\s\*]*?\b(m4_\w+)\s*\(", header, re.M))
    assert len(names) >= 25
    for n in sorted(names):
        assert hasattr(lib, n), f"missing export {n}"
    assert names == set(m4_bridge.SIGNATURES), "bindings and header disagree"


def test_exports_every_gguf_symbol(lib):
    import gguf

    header = (ROOT / "include" / "m4_gguf.h").read_text()
    names = set(re.findall(r"^M4_API [\w\s\*]*?\b(m4_\w+)\s*\(", header, re.M))
    assert len(names) >= 20
    for n in sorted(names):
        assert hasattr(lib, n), f"missing export {n}"
    assert names == set(gguf.SIGNATURES), "bindings and header disagree"


def test_expected_weight_bytes(lib):
    # core/bridge/m4_mlx_bridge.mm:58-75
    K, N = 4096, 4096
    exp = {0: K // 32 * N * 18, 1: K // 32 * N * 20, 2: K // 256 * N * 144, 3: K // 32 * N * 12,
           4: K // 256 * N * 160, 5: K // 256 * N * 144}
    for f, v in exp.items():
        assert lib.m4_bridge_get_expected_weight_bytes(f, K, N) == v
    assert lib.m4_bridge_get_expected_weight_bytes(6, K, N) == 0
    assert lib.m4_bridge_get_expected_weight_bytes(-1, K, N) == 0


def test_registry_matches_reference(lib):
    # tests/test_quant_registry.mm:15-101 and quant_registry.mm:60-172
    rows = {
        0: ("Q4_0", 32, 18, 4.50, "q4_0"), 1: ("MLX_4BIT", 32, 20, 5.00, "mlx_4bit"),
        2: ("Q4_K", 256, 144, 4.50, "q4_k"), 3: ("TERNARY_1_58", 32, 12, 3.00, "ternary_1_58"),
        4: ("VAR_RATE_AFFINE", 256, 160, 5.00, "var_rate_affine"), 5: ("EXL3", 256, 144, 4.50, "exl3"),
        6: ("Q8_0", 32, 34, 8.50, "q8_0"), 7: ("PRISM_Q2_0", 128, 34, 2.125, "prism_q2_0"),
    }
    for f, (name, bs, ss, bpw, sym) in rows.items():
        info = m4_bridge.CodecInfo()
        assert lib.m4_registry_get(f, ctypes.byref(info)) == 0
        assert info.format == f and info.name.decode() == name
        assert info.block_size == bs and info.struct_size == ss and info.bits_per_weight == bpw
        assert info.gemm_kernel_name.decode() == f"quant_router_gemm_{sym}_64x64"
        assert info.head_gemm_kernel_name.decode() == f"quant_router_head_gemm_{sym}_64x64"
        assert lib.m4_registry_get_by_name(name.encode()) == f
        assert lib.m4_registry_has_format(f)
        assert lib.m4_registry_compute_weight_bytes(f, 4096 * 4096) == (4096 * 4096 + bs - 1) // bs * ss
    arr = (ctypes.c_int * 16)()
    n = lib.m4_registry_available_formats(arr, 16)
    assert n >= 8 and list(arr[:8]) == list(range(8))
    assert lib.m4_registry_get(42, ctypes.byref(m4_bridge.CodecInfo())) == -3
    assert lib.m4_registry_get_by_name(b"NOPE") == -3
    assert lib.m4_registry_compute_weight_bytes(42, 100) == 0


def test_registry_custom_codec(lib):
    # tests/test_quant_registry.mm:103-121: QUANT_CUSTOM = 99 registered at runtime
    info = m4_bridge.CodecInfo(99, b"CUSTOM_TEST", b"test codec", 64, 40, 5.0, b"k_custom", b"k_custom_head")
    assert lib.m4_registry_register_codec(ctypes.byref(info)) == 0
    assert lib.m4_registry_has_format(99)
    assert lib.m4_registry_get_by_name(b"CUSTOM_TEST") == 99
    assert lib.m4_registry_compute_weight_bytes(99, 128) == 80
    out = m4_bridge.CodecInfo()
    assert lib.m4_registry_get(99, ctypes.byref(out)) == 0 and out.gemm_kernel_name == b"k_custom"


def _validate(lib, X=0x1000, Xb=None, W=0x2000, Wb=None, Y=0x3000, Yb=None, fmt=0, M=64, K=128, N=64):
    Xb = M * K * 2 if Xb is None else Xb
    Yb = M * N * 2 if Yb is None else Yb
    Wb = lib.m4_bridge_get_expected_weight_bytes(fmt, K, N) if Wb is None else Wb
    return lib.m4_bridge_validate_gemm(X, Xb, W, Wb, Y, Yb, fmt, M, K, N)


def test_validation_codes_and_order(lib):
    assert _validate(lib) == 0
    # -2: null pointers, odd X/Y (tests/redteam_bridge.py:151-167), undersized buffers (:351-352)
    assert _validate(lib, X=None) == -2 and _validate(lib, W=None) == -2 and _validate(lib, Y=None) == -2
    assert _validate(lib, X=0x1001) == -2 and _validate(lib, Y=0x3001) == -2
    assert _validate(lib, W=0x2001) == 0  # W alignment is not part of the contract
    assert _validate(lib, Xb=64 * 128 * 2 - 1) == -2
    assert _validate(lib, Yb=64 * 64 * 2 - 1) == -2
    assert _validate(lib, Wb=128 // 32 * 64 * 18 - 1) == -2
    # -3: format outside 0..5 (redteam_bridge.py:274)
    for f in (-1, 6, 7, 99):
        assert _validate(lib, fmt=f, Wb=10 ** 6) == -3
    # -4: zero dims, K % 32, K % 256 for super-block formats (redteam_bridge.py:363-471)
    assert _validate(lib, M=0) == -4 and _validate(lib, K=0) == -4 and _validate(lib, N=0) == -4
    assert _validate(lib, K=48, Wb=10 ** 6) == -4
    for f in (2, 4, 5):
        assert _validate(lib, fmt=f, K=128, Wb=10 ** 6) == -4
    for f in (0, 1, 3):
        assert _validate(lib, fmt=f, K=128) == 0
    # order: -2 (pointer) before -3 (format) before -4 (dims) before -2 (sizes)
    assert _validate(lib, X=None, fmt=9, M=0) == -2
    assert _validate(lib, fmt=9, M=0) == -3
    assert _validate(lib, M=0, Xb=0) == -4


def test_uninitialized_bridge_refuses_work(lib):
    # On a host with no GPU init fails; every dispatch must then return -1
    # (m4_mlx_bridge.mm:201-203) before touching the buffers.
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present; covered by the gpu tests")
    assert lib.m4_bridge_init(None) is False
    assert lib.m4_bridge_is_initialized() is False
    x = np.zeros((64, 128), np.float16)
    w = np.zeros(128 // 32 * 64 * 18, np.uint8)
    y = np.zeros((64, 64), np.float16)
    assert lib.m4_bridge_dispatch_gemm(x.ctypes.data, x.nbytes, w.ctypes.data, w.nbytes, y.ctypes.data, y.nbytes,
                                       0, 64, 128, 64) == -1
    assert lib.m4_bridge_dispatch_gemv(x.ctypes.data, 256, w.ctypes.data, w.nbytes, y.ctypes.data, 128,
                                       0, 128, 64) == -1
    assert lib.m4_bridge_dispatch_router_gemm(x.ctypes.data, x.nbytes, w.ctypes.data, w.nbytes, y.ctypes.data,
                                              y.nbytes, 7, 64, 128, 64) == -1
    assert lib.m4_bridge_rmsnorm(x.ctypes.data, x.nbytes, w.ctypes.data, 256, x.ctypes.data, x.nbytes, 64, 128,
                                 1e-5, 1) == -1
    assert lib.m4_bridge_rope(x.ctypes.data, x.nbytes, 1, 64, 128, 1e4, 0, 0) == -1
    dims = (ctypes.c_uint32 * 3)(64, 64, 128)
    assert lib.m4_bridge_dispatch_router_kernel(b"quant_router_gemm_ternary_1_58_vec", x.ctypes.data, x.nbytes,
                                                w.ctypes.data, w.nbytes, y.ctypes.data, y.nbytes, dims, 3) == -1
    assert lib.m4_bridge_dispatch_flash_attn_q8_0_gqa(x.ctypes.data, x.nbytes, w.ctypes.data, w.nbytes,
                                                      w.ctypes.data, w.nbytes, y.ctypes.data, y.nbytes,
                                                      2, 1, 32, 64, 0.125, 0) == -1
    assert lib.m4_bridge_prefill_layer_ex(*([x.ctypes.data] * 11), 0, 64, 128, 2, 1, 64, 256, 0.125, 1, 1e-5, 1,
                                          1e4, 0, 0) == -1
    lib.m4_bridge_synchronize()
    lib.m4_bridge_shutdown()
    assert lib.m4_bridge_get_uma_footprint_mb() > 0.0


def test_python_bridge_maps_status_to_runtime_error(libpath):
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    b = m4_bridge.HIPBridge(libpath)
    with pytest.raises(RuntimeError, match="status code -1"):
        b.dispatch_gemm(np.zeros((4, 32), np.float16), np.zeros(18 * 4, np.uint8), np.zeros((4, 4), np.float16), 0)


def test_non_finite_tripwire_host_side():
    """tests/e2e/test_tier1_feature_coverage.mm:490-531: a clean buffer passes;
    a NaN or Inf anywhere (fp32 or fp16, numpy or torch) trips the check the
    bridge defers to synchronize."""
    import torch

    clean = np.full(1000, 1.234, np.float32)
    assert m4_bridge._all_finite(clean)
    for bad in (np.nan, np.inf):
        a = np.ones(1000, np.float32)
        a[42] = bad
        assert not m4_bridge._all_finite(a)
        h = np.full(100, 0.5, np.float16)
        h[77] = bad
        assert not m4_bridge._all_finite(h) and not m4_bridge._all_finite(h.view(np.uint16))
        assert not m4_bridge._all_finite(torch.from_numpy(h))


def test_c_caller_compiles_and_links(libpath, tmp_path):
    """The headers are plain C and the library links from a C program: build
    tests/c/abi_smoke.c with the host compiler against the shipped .so and run
    it (entry points that need no GPU)."""
    import shutil
    import subprocess

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    exe = tmp_path / "abi_smoke"
    r = subprocess.run([cc, "-std=c99", "-Wall", "-Werror", "-I", str(ROOT / "include"), str(ROOT / "tests" / "c" /
                        "abi_smoke.c"), "-o", str(exe), "-L", str(libpath.parent), "-lm4_bridge",
                        f"-Wl,-rpath,{libpath.parent}"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "abi_smoke: ok" in r.stdout


def test_extract_buffer_strided_and_offset_views(libpath):
    """tests/redteam_bridge.py:93-134: a strided view is made contiguous (its own
    byte size, retained until synchronize); a contiguous row slice keeps its
    byte offset into the parent buffer."""
    import torch

    import m4_bridge

    B = m4_bridge.HIPBridge
    for X in (np.ones((64, 64), np.float16), torch.ones((64, 64), dtype=torch.float16)):
        strided = X[:, ::2]
        ptr, nbytes = B.extract_buffer_address_and_size(strided)
        assert ptr != 0 and nbytes == 64 * 32 * 2
        base, _ = B.extract_buffer_address_and_size(X)
        sub, sub_bytes = B.extract_buffer_address_and_size(X[10:20, :])
        assert sub - base == 10 * 64 * 2 and sub_bytes == 10 * 64 * 2
    assert len(B._retained_contig) >= 2
    B._retained_contig.clear()
