"""GPU parity: the HIP kernels, called through the C-ABI, against the oracle.

Bars: dequantized weights and Q8_0 codes bit-exact;
projections, SwiGLU and attention within max |diff| <= 1/128 = 0.0078125 of
the double-precision CPU gold (tests/e2e/test_tier1_feature_coverage.mm:149;
core/metrology/bench_standards.h:28).
"""
from __future__ import annotations

import numpy as np
import pytest

import synth
import tolerance
from tolerance import TOL

pytestmark = pytest.mark.gpu


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.cpu().numpy()


def empty16(*shape):
    import torch

    return torch.empty(*shape, dtype=torch.float16, device="cuda")


def maxdiff(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    assert np.all(np.isfinite(a)), "non-finite GPU output"
    return float(np.max(np.abs(a - b))) if a.size else 0.0


def absxw(oracle, fmt, X, W, K, N):
    """sum_k |x_k w_k| with the exact weights (error-bound scale)."""
    return np.abs(X.astype(np.float64)) @ np.abs(oracle.dequantize_f64(fmt, W, K, N)).T


def weights(kind, fmt, N, K, seed):
    return synth.random_blocks(fmt, N, K, seed) if kind == "random" else synth.quantized_weights(fmt, N, K, seed)


# --------------------------------------------------------------------------
# Dequantization: bit-exact
# --------------------------------------------------------------------------

@pytest.mark.parametrize("fmt,K", [(0, 512), (0, 96), (1, 512), (1, 96), (2, 512), (3, 512), (3, 96), (4, 512),
                                   (5, 512), (6, 512), (6, 96), (7, 512), (7, 384), (8, 512), (8, 192)])
@pytest.mark.parametrize("kind", ["random", "quantized"])
def test_dequant_bit_exact(bridge, oracle, fmt, K, kind):
    N = 72
    if kind == "quantized" and fmt == 1 and K % 64:
        pytest.skip("MLX g64 quantizer needs K % 64 == 0")
    if kind == "quantized" and 4 <= fmt <= 7:
        pytest.skip("formats 4..7 come from random generators only (no BASELINE quantizer)")
    W = weights(kind, fmt, N, K, 100 + fmt)
    out = empty16(N, K)
    bridge.dequantize(dev(W), out, fmt, K, N)
    bridge.synchronize()
    np.testing.assert_array_equal(host(out).view(np.uint16), oracle.dequantize(fmt, W, K, N).view(np.uint16))


def test_dequant_ternary_code3_and_q4k_slow_path(bridge, oracle):
    W = synth.random_blocks(3, 40, 256, 7, code3=True)
    out = empty16(40, 256)
    bridge.dequantize(dev(W), out, 3, 256, 40)
    # Q4_K with d >> dmin (binade gap > 3): exact-sum path
    Wk = synth.random_blocks(2, 40, 512, 8).reshape(40, 2, 144).copy()
    rng = np.random.default_rng(9)
    Wk[..., 0:2] = np.float16(3.0).reshape(1).view(np.uint8)
    Wk[..., 2:4] = (rng.random((40, 2)) * 1e-4).astype(np.float16)[..., None].view(np.uint8)
    Wk = Wk.reshape(-1)
    outk = empty16(40, 512)
    bridge.dequantize(dev(Wk), outk, 2, 512, 40)
    bridge.synchronize()
    np.testing.assert_array_equal(host(out).view(np.uint16), oracle.dequantize(3, W, 256, 40).view(np.uint16))
    np.testing.assert_array_equal(host(outk).view(np.uint16), oracle.dequantize(2, Wk, 512, 40).view(np.uint16))


@pytest.mark.parametrize("fmt", [4, 5])
def test_dequant_double_rounding_formats_wide_scales(bridge, oracle, fmt):
    """VAR_RATE_AFFINE / EXL3 weights are formed in double by the CPU gold and
    rounded once to fp16: scales and biases spread over the whole binary16
    range exercise the round-to-odd narrowing (inexact double -> float) and
    subnormal / overflowing results; mixed depths and orders per lane."""
    N, K = 96, 512
    rng = np.random.default_rng(40 + fmt)
    W = synth.random_blocks(fmt, N, K, 41 + fmt).reshape(N, K // 256, -1).copy()
    mag = 2.0 ** rng.integers(-24, 12, (N, K // 256, 2))
    sign = np.where(rng.random((N, K // 256, 2)) < 0.5, -1.0, 1.0)
    hdr = (sign * mag * (1 + rng.random((N, K // 256, 2)))).astype(np.float16)
    W[..., 0:4] = hdr.view(np.uint8).reshape(N, K // 256, 4)
    if fmt == 4:  # random depths (including values that mean 4-bit) and orders per sub-block
        W[..., 20:28] = rng.integers(0, 32, (N, K // 256, 8)).astype(np.uint8)
    W = W.reshape(-1)
    out = empty16(N, K)
    bridge.dequantize(dev(W), out, fmt, K, N)
    bridge.synchronize()
    np.testing.assert_array_equal(host(out).view(np.uint16), oracle.dequantize(fmt, W, K, N).view(np.uint16))


@pytest.mark.parametrize("fmt", [4, 5])
@pytest.mark.parametrize("M,K,N", [(1, 512, 256), (33, 512, 256), (129, 512, 256), (128, 4096, 320)])
def test_gemm_var_rate_and_exl3(bridge, oracle, fmt, M, K, N):
    """tests/e2e/test_tier1_feature_coverage.mm:382-460 shapes plus a split-K
    shape; standard, residual and direct-head outputs."""
    X = synth.activations(M, K, 80 + M, std=0.35)
    W = synth.random_blocks(fmt, N, K, 81 + fmt)
    Y = empty16(M, N)
    bridge.dispatch_gemm(dev(X), dev(W), Y, fmt, M, K, N)
    R = synth.activations(M, N, 82)
    Yr = empty16(M, N)
    bridge.dispatch_gemm_residual(dev(X), dev(W), dev(R), Yr, fmt, M, K, N)
    H, D = N // 64, 64
    Yh = empty16(H, M, D)
    bridge.dispatch_head_gemm(dev(X), dev(W), Yh, fmt, M, H, D, K)
    bridge.synchronize()
    tolerance.check_ref(host(Y), oracle.gemm(fmt, X, W, N), what="standard")
    tolerance.check_ref(host(Yr), oracle.gemm(fmt, X, W, N, R=R), what="residual")
    tolerance.check_ref(host(Yh), oracle.gemm(fmt, X, W, N, head_D=D), what="direct-head")


def test_router_kernels_by_name(bridge, oracle):
    """Every router kernel name (quant_router_{,head_}gemm_<fmt>_64x64 from the
    registry, quant_router_kernels.metal:588-927) and the vector-ALU ternary
    names (:934-1201) with the kernels' constant slots give the same output as
    the format-id entry points; the ternary names also meet the oracle bound.
    Unknown names return -3, a wrong slot count -4."""
    M, K, N, D = 33, 512, 128, 64
    X = synth.activations(M, K, 91, std=0.35)
    for fmt, sym in [(0, "q4_0"), (1, "mlx_4bit"), (2, "q4_k"), (3, "ternary_1_58"), (4, "var_rate_affine"),
                     (5, "exl3"), (6, "q8_0"), (7, "prism_q2_0")]:
        W = dev(synth.random_blocks(fmt, N, K, 92 + fmt))
        names = [(f"quant_router_gemm_{sym}_64x64", False), (f"quant_router_head_gemm_{sym}_64x64", True)]
        if fmt == 3:
            names += [("quant_router_gemm_ternary_1_58_vec", False), ("quant_router_head_gemm_ternary_1_58_vec", True)]
        Yf = empty16(M, N)
        bridge.dispatch_router_gemm(dev(X), W, Yf, fmt, M, K, N)
        Yhf = empty16(N // D, M, D)
        bridge.dispatch_head_gemm(dev(X), W, Yhf, fmt, M, N // D, D, K)
        for name, head in names:
            if head:
                Y = empty16(N // D, M, D)
                bridge.dispatch_router_kernel(name, dev(X), W, Y, M, N // D, D, K)
                bridge.synchronize()
                assert np.array_equal(host(Y).view(np.uint16), host(Yhf).view(np.uint16)), name
            else:
                Y = empty16(M, N)
                bridge.dispatch_router_kernel(name, dev(X), W, Y, M, N, K)
                bridge.synchronize()
                assert np.array_equal(host(Y).view(np.uint16), host(Yf).view(np.uint16)), name
        if fmt == 3:
            Wh = host(W)
            tolerance.check_ref(host(Yf), oracle.gemm(3, X, Wh, N), what="ternary by name")
    W = dev(synth.random_blocks(0, N, K, 99))
    Y = empty16(M, N)
    with pytest.raises(RuntimeError, match="status code -3"):
        bridge.dispatch_router_kernel("quant_router_gemm_q5_0_64x64", dev(X), W, Y, M, N, K)
    with pytest.raises(RuntimeError, match="status code -4"):
        bridge.dispatch_router_kernel("quant_router_head_gemm_q4_0_64x64", dev(X), W, Y, M, N, K)


def test_host_range_into_protected_page_returns_minus_5(bridge):
    """tests/redteam_bridge.py:178-221: a host X running from a readable page
    into a PROT_NONE page gives -5 (no fault); the dispatch's staged host
    output is never written back, and the bridge keeps working."""
    import ctypes
    import mmap

    pg = mmap.PAGESIZE
    buf = mmap.mmap(-1, 2 * pg, mmap.MAP_PRIVATE | mmap.MAP_ANONYMOUS, mmap.PROT_READ | mmap.PROT_WRITE)
    cobj = ctypes.c_char.from_buffer(buf)
    base = ctypes.addressof(cobj)
    libc = ctypes.CDLL(None)
    libc.mprotect.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert libc.mprotect(base + pg, pg, 0) == 0
    try:
        M, K, N = 32, 64, 64
        assert M * K * 2 <= pg
        W = np.zeros(K // 32 * N * 18, np.uint8)
        Y = np.full((M, N), 7.0, np.float16)
        ret = bridge._lib.m4_bridge_dispatch_gemm(base + 100, M * K * 2, W.ctypes.data, W.nbytes, Y.ctypes.data,
                                                  Y.nbytes, 0, M, K, N)
        assert ret == -5
        bridge.synchronize()
        assert np.all(Y == 7.0)
        X = np.zeros((M, K), np.float16)
        ret = bridge._lib.m4_bridge_dispatch_gemm(X.ctypes.data, X.nbytes, W.ctypes.data, W.nbytes, Y.ctypes.data,
                                                  Y.nbytes, 0, M, K, N)
        assert ret == 0
        bridge.synchronize()
        assert np.all(Y == 0.0)  # zero scales: every output is 0
    finally:
        libc.mprotect(base + pg, pg, 3)
        del cobj
        buf.close()


def test_chained_host_buffer_dispatches_without_synchronize(bridge, oracle):
    """Host (pageable) buffers chained Y1 -> X2 with no synchronize between
    the two dispatches: the second must read the first's result, as the
    reference's in-order queue on zero-copy buffers gives it; also a host
    residual R that is the first dispatch's output."""
    M, K, N = 64, 256, 256
    X = synth.activations(M, K, 301)
    W1 = synth.quantized_weights(0, N, K, 302)
    W2 = synth.quantized_weights(0, N, N, 303)
    Y1 = np.full((M, N), 3.0, np.float16)
    Y2 = np.zeros((M, N), np.float16)
    Y3 = np.zeros((M, N), np.float16)
    lib = bridge._lib
    assert lib.m4_bridge_dispatch_gemm(X.ctypes.data, X.nbytes, W1.ctypes.data, W1.nbytes, Y1.ctypes.data,
                                       Y1.nbytes, 0, M, K, N) == 0
    assert lib.m4_bridge_dispatch_gemm(Y1.ctypes.data, Y1.nbytes, W2.ctypes.data, W2.nbytes, Y2.ctypes.data,
                                       Y2.nbytes, 0, M, N, N) == 0
    assert lib.m4_bridge_dispatch_gemm_residual(X.ctypes.data, X.nbytes, W1.ctypes.data, W1.nbytes,
                                                Y1.ctypes.data, Y1.nbytes, Y3.ctypes.data, Y3.nbytes, 0, M, K,
                                                N) == 0
    bridge.synchronize()
    ref1 = oracle.gemm(0, X, W1, N)
    assert maxdiff(Y1, ref1) <= TOL
    assert maxdiff(Y2, oracle.gemm(0, Y1, W2, N)) <= TOL
    assert maxdiff(Y3, oracle.gemm(0, X, W1, N, R=Y1)) <= TOL


def test_in_flight_buffers_retained_until_synchronize(bridge):
    """tests/redteam_bridge.py:486-528: the bridge holds the tensors of issued
    work until synchronize(), so dropping the caller's references is safe."""
    import gc

    import torch

    M, K, N = 512, 512, 512
    X = torch.ones((M, K), dtype=torch.float16, device="cuda")
    W = torch.zeros(K // 32 * N * 18, dtype=torch.uint8, device="cuda")
    Y = torch.empty((M, N), dtype=torch.float16, device="cuda")
    bridge.dispatch_gemm(X, W, Y, 0, M, K, N)
    before = len(bridge._in_flight_tensors)
    assert before > 0
    del X, W, Y
    gc.collect()
    bridge.synchronize()
    assert len(bridge._in_flight_tensors) == 0


@pytest.mark.parametrize("fmt,M,K,N", [(1, 128, 4096, 14336), (0, 2048, 2048, 3072), (3, 256, 2048, 5120),
                                       (0, 129, 4096, 4096), (1, 129, 4096, 4096), (7, 150, 2048, 1536),
                                       (6, 300, 2048, 1024)])
def test_under_filled_grid_shapes(bridge, oracle, fmt, M, K, N):
    """Full-size shapes whose tile grid under-fills the 256 CUs (the headline:
    112 tiles x 2 K splits; 384 tiles = 1.5 rounds; 80 tiles x 2 splits) and
    64-row tiles with a K split (M = 129, 150, 300: last 128-row tile at most
    half full), checked against the oracle on a row sample (every output
    column) and for run-to-run determinism of the split-K reduction."""
    X = synth.activations(M, K, 120 + fmt, std=0.35)
    W = synth.random_blocks(fmt, N, K, 121 + fmt)
    Y = empty16(M, N)
    bridge.dispatch_router_gemm(dev(X), dev(W), Y, fmt, M, K, N)
    bridge.synchronize()
    rows = np.unique(np.r_[0, 1, 63, 64, 127, np.arange(0, M, 37), M - 1])
    Xs = np.ascontiguousarray(X[rows])
    tolerance.check_ref(host(Y)[rows], oracle.gemm(fmt, Xs, W, N), what=f"fmt {fmt} {M}x{K}x{N}")
    Y2 = empty16(M, N)
    bridge.dispatch_router_gemm(dev(X), dev(W), Y2, fmt, M, K, N)
    bridge.synchronize()
    np.testing.assert_array_equal(host(Y2).view(np.uint16), host(Y).view(np.uint16))  # deterministic


@pytest.mark.parametrize("fmt,M,K,N", [(1, 128, 4096, 12352), (0, 100, 2176, 12300), (2, 128, 2048, 12288),
                                       (3, 65, 4096, 12352), (8, 127, 2176, 12416), (1, 128, 128, 12288),
                                       (0, 96, 384, 12352), (0, 40, 4096, 12352),
                                       (3, 150, 2048, 8200), (0, 129, 1152, 8192), (1, 140, 4096, 16384),
                                       (1, 128, 4160, 12352)])
def test_k_group_tiles(bridge, oracle, fmt, M, K, N):
    """The 128 x 64 tile whose two K groups take alternate 64-K steps and
    meet in LDS (M <= 128 with at least 192 column tiles), and the 64 x 128
    tile as two K groups (M past a multiple of 128 by at most 64, no K split
    needed: M = 129, 140, 150): ragged M and N,
    K with an odd number of step pairs (2176 = 17 pairs), one or three pairs
    (K = 128, 384: fewer rounds than the stager runs ahead), M = 40 (whichever
    small-M or tiled path takes it), K = 4160 (not whole 128-K rounds: the
    shape choice leaves the K-group tiles), checked against the oracle on a
    row sample with every column, and deterministic."""
    X = synth.activations(M, K, 140 + fmt, std=0.35)
    W = synth.random_blocks(fmt, N, K, 141 + fmt)
    Y = empty16(M, N)
    bridge.dispatch_router_gemm(dev(X), dev(W), Y, fmt, M, K, N)
    bridge.synchronize()
    rows = np.unique(np.r_[0, 1, 31, 32, 63, 64, 127, 128, M - 1])
    rows = rows[rows < M]
    Xs = np.ascontiguousarray(X[rows])
    tolerance.check_ref(host(Y)[rows], oracle.gemm(fmt, Xs, W, N), what=f"fmt {fmt} {M}x{K}x{N}")
    Y2 = empty16(M, N)
    bridge.dispatch_router_gemm(dev(X), dev(W), Y2, fmt, M, K, N)
    bridge.synchronize()
    np.testing.assert_array_equal(host(Y2).view(np.uint16), host(Y).view(np.uint16))


def test_k_group_tiles_head_layout_and_residual(bridge, oracle):
    """The K-group tile's epilogue with the direct-head layout and a residual."""
    fmt, M, K, H, D = 0, 128, 2048, 192, 64
    N = H * D
    X = synth.activations(M, K, 150, std=0.35)
    W = synth.random_blocks(fmt, N, K, 151)
    rows = np.array([0, 5, 64, 127])
    Xs = np.ascontiguousarray(X[rows])
    Yh = empty16(H, M, D)
    bridge.dispatch_head_gemm(dev(X), dev(W), Yh, fmt, M, H, D, K)
    R = synth.activations(M, N, 152)
    Yr = empty16(M, N)
    bridge.dispatch_gemm_residual(dev(X), dev(W), dev(R), Yr, fmt, M, K, N)
    bridge.synchronize()
    ref_h = oracle.gemm(fmt, Xs, W, N, head_D=D)  # [H, rows, D]
    tolerance.check_ref(host(Yh)[:, rows, :], ref_h, what="direct-head")
    tolerance.check_ref(host(Yr)[rows], oracle.gemm(fmt, Xs, W, N, R=np.ascontiguousarray(R[rows])), what="residual")


def test_gemm_q4_0_scales_beyond_fast_path(bridge, oracle):
    """Q4_0 scales with |d| > 8188 (-8 d is not finite in binary16): the tiled
    kernel's fused fma(q, d, -8 d) decode cannot form them, so the wave takes
    the exact (q - 8) d path; codes 1..15 keep every weight finite."""
    M, K, N = 129, 512, 128
    rng = np.random.default_rng(77)
    W = synth.random_blocks(0, N, K, 78).reshape(N, K // 32, 18).copy()
    d = (rng.random((N, K // 32)) * 800 + 8190) * np.where(rng.random((N, K // 32)) < 0.5, -1, 1)
    W[..., 0:2] = d.astype(np.float16)[..., None].view(np.uint8)
    lo = rng.integers(1, 16, (N, K // 32, 16))
    hi = rng.integers(1, 16, (N, K // 32, 16))
    W[..., 2:] = (lo | (hi << 4)).astype(np.uint8)
    W = W.reshape(-1)
    X = synth.activations(M, K, 79, std=1e-5)
    Y = empty16(M, N)
    bridge.dispatch_gemm(dev(X), dev(W), Y, 0, M, K, N)
    bridge.synchronize()
    ref = oracle.gemm(0, X, W, N)
    tolerance.check(host(Y), ref, tolerance.gemm_bound(ref, absxw(oracle, 0, X, W, K, N), K))


@pytest.mark.parametrize("fmt", [0, 2])
@pytest.mark.parametrize("M,K,N", [(256, 512, 256), (1024, 1024, 256)])
def test_gemm_decode_bit_exact_mixed_exact_paths(bridge, oracle, fmt, M, K, N):
    """The tiled kernel's weight decode, bit for bit, with the exact-decode
    path taken by some lanes of a wave and not others: about a third of the
    Q4_0 blocks have |d| > 8188 (-8 d not finite) and a third of the Q4_K
    super-blocks a binade gap between d and dmin above 3.  X is one-hot
    (row m selects k = m mod K), so every output is one exact product and
    Y[m, n] must equal the CPU unpack of W[n, m mod K]."""
    rng = np.random.default_rng(300 + fmt + M)
    if fmt == 0:
        W = synth.random_blocks(0, N, K, 301).reshape(N, K // 32, 18).copy()
        big = rng.random((N, K // 32)) < 0.35
        d = (rng.random((N, K // 32)) * 800 + 8190) * np.where(rng.random((N, K // 32)) < 0.5, -1, 1)
        W[big, 0:2] = d[big].astype(np.float16)[..., None].view(np.uint8)
        codes = (rng.integers(1, 16, (N, K // 32, 16)) | (rng.integers(1, 16, (N, K // 32, 16)) << 4)).astype(np.uint8)
        W[big, 2:] = codes[big]
    else:
        W = synth.random_blocks(2, N, K, 302).reshape(N, K // 256, 144).copy()
        gap = rng.random((N, K // 256)) < 0.35
        W[gap, 0:2] = np.float16(3.0).reshape(1).view(np.uint8)
        W[gap, 2:4] = (rng.random(int(gap.sum())) * 1e-4 + 1e-5).astype(np.float16)[..., None].view(np.uint8)
    W = W.reshape(-1)
    X = np.zeros((M, K), np.float16)
    X[np.arange(M), np.arange(M) % K] = 1.0
    Y = empty16(M, N)
    bridge.dispatch_gemm(dev(X), dev(W), Y, fmt, M, K, N)
    bridge.synchronize()
    wd = oracle.dequantize(fmt, W, K, N).astype(np.float32)  # [N, K]
    assert np.isfinite(wd).all()
    # +0 and -0 compare equal: the fast Q4_0 decode gives +0 where the CPU unpack gives -0
    np.testing.assert_array_equal(host(Y).astype(np.float32), wd[:, np.arange(M) % K].T)


@pytest.mark.parametrize("fmt", [0, 1, 2, 3, 8])
@pytest.mark.parametrize("M,K,N", [(1, 4096, 4096), (33, 4096, 4104), (64, 2048, 4096), (17, 1024, 4096)])
def test_gemm_small_m_wide(bridge, oracle, fmt, M, K, N):
    """The small-M projection (M <= 64) on wide outputs, every format it
    takes (config 1's shape is (33, 4096, 4096)): standard, residual and
    direct-head outputs against the oracle on sampled rows; N = 4104 leaves a
    ragged last column strip; runs are bit-identical (fixed-order split-K)."""
    rng = np.random.default_rng(500 + fmt + M)
    X = synth.activations(M, K, 501 + M, std=0.35)
    W = synth.random_blocks(fmt, N, K, 502 + fmt)
    R = synth.activations(M, N, 503)
    Y, Y2, Yr = empty16(M, N), empty16(M, N), empty16(M, N)
    bridge.dispatch_router_gemm(dev(X), dev(W), Y, fmt, M, K, N)
    bridge.dispatch_router_gemm(dev(X), dev(W), Y2, fmt, M, K, N)
    bridge.dispatch_gemm_residual(dev(X), dev(W), dev(R), Yr, fmt, M, K, N)
    D = 64
    Yh = empty16(N // D, M, D) if N % D == 0 else None
    if Yh is not None:
        bridge.dispatch_head_gemm(dev(X), dev(W), Yh, fmt, M, N // D, D, K)
    bridge.synchronize()
    rows = np.unique(np.r_[0, M - 1, rng.integers(0, M, 3)])
    Xs = np.ascontiguousarray(X[rows])
    gold = oracle.gemm(fmt, Xs, W, N)
    tolerance.check_ref(host(Y)[rows], gold, what=f"fmt {fmt} {M}x{K}x{N}")
    np.testing.assert_array_equal(host(Y2).view(np.uint16), host(Y).view(np.uint16))
    tolerance.check_ref(host(Yr)[rows], oracle.gemm(fmt, Xs, W, N, R=np.ascontiguousarray(R[rows])), what="residual")
    if Yh is not None:  # [H, M, D]: the sampled rows of every head
        np.testing.assert_array_equal(host(Yh)[:, rows, :].transpose(1, 0, 2).reshape(len(rows), N).view(np.uint16),
                                      host(Y)[rows].view(np.uint16))


@pytest.mark.parametrize("fmt,M,K,N", [(0, 129, 96, 256), (1, 200, 160, 384), (3, 300, 2080, 512),
                                       (6, 129, 160, 256), (0, 2048, 1056, 512), (3, 129, 4128, 8192)])
def test_gemm_half_last_step(bridge, oracle, fmt, M, K, N):
    """K with a half last 64-K step (K % 64 == 32) through the tiled kernel:
    the stager (or the register path) must copy zeros for the step's upper 32
    K (a K split needs K to be a multiple of 512, so no split has a half
    step); 4128 at cfg4's shape, M = 2048 on the two-B-tile instance."""
    X = synth.activations(M, K, 160 + fmt, std=0.35)
    W = synth.random_blocks(fmt, N, K, 161 + fmt)
    Y = empty16(M, N)
    bridge.dispatch_router_gemm(dev(X), dev(W), Y, fmt, M, K, N)
    bridge.synchronize()
    rows = np.unique(np.r_[0, 1, 63, 64, 127, 128, M - 1])
    rows = rows[rows < M]
    Xs = np.ascontiguousarray(X[rows])
    tolerance.check_ref(host(Y)[rows], oracle.gemm(fmt, Xs, W, N), what=f"fmt {fmt} {M}x{K}x{N}")


@pytest.mark.parametrize("fmt", [6, 7])
@pytest.mark.parametrize("M,K,N", [(1, 384, 256), (33, 384, 200), (129, 512, 256), (128, 4096, 320),
                                   (300, 1152, 136)])
def test_gemm_q8_0_and_prism(bridge, oracle, fmt, M, K, N):
    """Q8_0 weights and PRISM_Q2_0 (code 3 = +2d included) through the
    kernel-name entry point (quant_router_gemm_<fmt>_64x64) and the head and
    residual entry points; K = 384 / 1152 give 2-byte-aligned columns
    (34-byte blocks), 4096 a split-K launch; the plain dispatch_gemm keeps the
    reference's format range and refuses them with -3."""
    X = synth.activations(M, K, 90 + M, std=0.35)
    W = synth.random_blocks(fmt, N, K, 91 + fmt)
    Y = empty16(M, N)
    bridge.dispatch_router_gemm(dev(X), dev(W), Y, fmt, M, K, N)
    R = synth.activations(M, N, 92)
    Yr = empty16(M, N)
    bridge.dispatch_gemm_residual(dev(X), dev(W), dev(R), Yr, fmt, M, K, N)
    D = 8 if N % 64 else 64
    H = N // D
    Yh = empty16(H, M, D)
    bridge.dispatch_head_gemm(dev(X), dev(W), Yh, fmt, M, H, D, K)
    with pytest.raises(RuntimeError):
        bridge.dispatch_gemm(dev(X), dev(W), empty16(M, N), fmt, M, K, N)
    bridge.synchronize()
    tolerance.check_ref(host(Y), oracle.gemm(fmt, X, W, N), what="standard")
    tolerance.check_ref(host(Yr), oracle.gemm(fmt, X, W, N, R=R), what="residual")
    tolerance.check_ref(host(Yh), oracle.gemm(fmt, X, W, N, head_D=D), what="direct-head")


# --------------------------------------------------------------------------
# Projections
# --------------------------------------------------------------------------

@pytest.mark.parametrize("fmt", [0, 1, 2, 3])
@pytest.mark.parametrize("M", [1, 33, 127, 128, 129, 2048])
def test_gemm_tier1_shapes(bridge, oracle, fmt, M):
    # tests/e2e/test_tier1_feature_coverage.mm:122-223: K=512, N=256
    K, N = 512, 256
    X = synth.activations(M, K, M, std=0.35)
    W = synth.random_blocks(fmt, N, K, 7 + fmt)
    Y = empty16(M, N)
    bridge.dispatch_gemm(dev(X), dev(W), Y, fmt, M, K, N)
    bridge.synchronize()
    tolerance.check_ref(host(Y), oracle.gemm(fmt, X, W, N), what=f"tier-1 fmt {fmt} M={M}")


@pytest.mark.parametrize("fmt", [0, 1, 2, 3])
@pytest.mark.parametrize("M,K,N", [(64, 256, 96), (200, 1024, 160), (31, 2304, 64)])
def test_gemm_gaussian_quantized(bridge, oracle, fmt, M, K, N):
    if fmt == 1 and K % 64:
        pytest.skip("g64")
    X = synth.activations(M, K, 3)
    W = synth.quantized_weights(fmt, N, K, 4)
    Y = empty16(M, N)
    bridge.dispatch_gemm(dev(X), dev(W), Y, fmt, M, K, N)
    bridge.synchronize()
    assert maxdiff(host(Y), oracle.gemm(fmt, X, W, N)) <= TOL


@pytest.mark.parametrize("N", [33, 65])
def test_gemm_ragged_n_known_answer(bridge, N):
    # tests/redteam_bridge.py:438-455: N not divisible by the tile, X = 1, w = 1 -> K
    M, K = 32, 64
    blk = np.concatenate([np.array([0x00, 0x3C], np.uint8), np.full(16, 0x99, np.uint8)])
    W = np.tile(blk, (K // 32) * N)
    Y = empty16(M, N)
    bridge.dispatch_gemm(dev(np.ones((M, K), np.float16)), dev(W), Y, 0, M, K, N)
    bridge.synchronize()
    assert np.all(host(Y) == K)


def test_bridge_basic_known_answers_host_buffers(bridge):
    """tests/test_bridge_basic.py:41-150 with host (numpy) buffers: the bridge
    stages them through device memory and writes Y back at synchronize()."""
    for M, K, N in [(33, 64, 64), (64, 64, 64), (128, 128, 128)]:
        blk = np.concatenate([np.array([0x00, 0x3C], np.uint8), np.full(16, 0x99, np.uint8)])
        W = np.tile(blk, (K // 32) * N)
        Y = np.zeros((M, N), np.float16)
        bridge.dispatch_gemm(np.ones((M, K), np.float16), W, Y, 0, M, K, N, check_finite=True)
        bridge.synchronize()
        assert np.all(Y == K)
    M = K = N = 64
    blk = np.concatenate([np.array([0x00, 0x3C, 0x00, 0x00], np.uint8), np.full(16, 0x11, np.uint8)])
    Y = np.zeros((M, N), np.float16)
    bridge.dispatch_gemm(np.ones((M, K), np.float16), np.tile(blk, (K // 32) * N), Y, 1, M, K, N)
    bridge.synchronize()
    assert np.all(Y == K)
    # decode GEMV (test_bridge_basic.py:121-150)
    blk = np.concatenate([np.array([0x00, 0x3C], np.uint8), np.full(16, 0x99, np.uint8)])
    y = np.zeros(N, np.float16)
    bridge.dispatch_gemv(np.ones(K, np.float16), np.tile(blk, (K // 32) * N), y, 0)
    bridge.synchronize()
    assert np.all(y == K)


def test_host_staging_buffers_are_reused(bridge):
    """Host (numpy) buffers of changing sizes, several dispatches per
    synchronize: every output equals the device-resident dispatch bit for bit,
    and once the working set is reached repeated calls allocate no more
    staging memory (the free list refilled at synchronize is reused)."""
    import torch

    shapes = [(64, 512, 256), (130, 1024, 512), (64, 512, 256), (33, 4096, 4096), (130, 1024, 512)]
    inputs = []
    for i, (M, K, N) in enumerate(shapes):
        X = synth.activations(M, K, 700 + i)
        W = synth.quantized_weights(0, N, K, 710 + i)
        Yd = torch.empty(M, N, dtype=torch.float16, device="cuda")
        bridge.dispatch_gemm(dev(X), dev(W), Yd, 0, M, K, N)
        inputs.append((X, W, host(Yd)))
    bridge.synchronize()
    for rnd in range(2):
        outs = []
        for (M, K, N), (X, W, _) in zip(shapes, inputs):
            Y = np.zeros((M, N), np.float16)
            bridge.dispatch_gemm(X, W, Y, 0, M, K, N)
            outs.append(Y)
        bridge.synchronize()
        for Y, (_, _, Yref) in zip(outs, inputs):
            np.testing.assert_array_equal(Y.view(np.uint16), Yref.view(np.uint16))
    # the largest call again and again: the footprint (host RSS + device memory
    # the bridge holds) stays within a few MB, far below one call's 9.7 MB of staging
    X, W, _ = inputs[3]
    Y = np.zeros((33, 4096), np.float16)
    bridge.dispatch_gemm(X, W, Y, 0, 33, 4096, 4096)
    bridge.synchronize()
    before = bridge.get_uma_footprint_mb()
    for _ in range(20):
        bridge.dispatch_gemm(X, W, Y, 0, 33, 4096, 4096)
        bridge.synchronize()
    assert bridge.get_uma_footprint_mb() - before < 4.0
    np.testing.assert_array_equal(Y.view(np.uint16), inputs[3][2].view(np.uint16))


def test_gemv_and_misaligned_pointers(bridge, oracle):
    import torch

    K, N = 512, 128
    W = synth.random_blocks(2, N, K, 11)
    x = synth.activations(1, K, 12)
    y = empty16(N)
    bridge.dispatch_gemv(dev(x[0]), dev(W), y, 2)
    # X, W and Y at 2-byte offsets: accepted (only odd pointers are refused), staged internally
    xb = torch.zeros(K + 1, dtype=torch.float16, device="cuda")
    xb[1:] = dev(x[0])
    wb = torch.zeros(W.size + 2, dtype=torch.uint8, device="cuda")
    wb[2:] = dev(W)
    yb = torch.zeros(N + 1, dtype=torch.float16, device="cuda")
    lib = bridge.lib
    rc = lib.m4_bridge_dispatch_gemv(xb.data_ptr() + 2, K * 2, wb.data_ptr() + 2, W.size, yb.data_ptr() + 2,
                                     N * 2, 2, K, N)
    assert rc == 0
    assert lib.m4_bridge_dispatch_gemv(xb.data_ptr() + 1, K * 2, wb.data_ptr(), W.size, yb.data_ptr(), N * 2, 2,
                                       K, N) == -2
    bridge.synchronize()
    tolerance.check_ref(host(y), oracle.gemm(2, x, W, N)[0], what="gemv")
    np.testing.assert_array_equal(host(yb)[1:], host(y))


@pytest.mark.parametrize("fmt", [0, 2, 3])
def test_direct_head_and_residual(bridge, oracle, fmt):
    M, K, H, D = 129, 512, 4, 64
    N = H * D
    X = synth.activations(M, K, 21, std=0.35)  # test_tier1_feature_coverage.mm:151-223 inputs
    W = synth.random_blocks(fmt, N, K, 22)
    Yh = empty16(H, M, D)
    bridge.dispatch_head_gemm(dev(X), dev(W), Yh, fmt, M, H, D, K)
    R = synth.activations(M, N, 23)
    Yr = empty16(M, N)
    bridge.dispatch_gemm_residual(dev(X), dev(W), dev(R), Yr, fmt, M, K, N)
    bridge.synchronize()
    tolerance.check_ref(host(Yh), oracle.gemm(fmt, X, W, N, head_D=D), what="direct-head")
    tolerance.check_ref(host(Yr), oracle.gemm(fmt, X, W, N, R=R), what="residual")


# --------------------------------------------------------------------------
# SwiGLU
# --------------------------------------------------------------------------

@pytest.mark.parametrize("fmt", [0, 1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("M", [33, 128, 129])
def test_swiglu(bridge, oracle, fmt, M):
    # brick3_swiglu_bench.mm:268-426 verifies M in {33,127,128,129}
    K, N = 512, 256
    X = synth.activations(M, K, 31, std=0.35)
    Wg, Wu = synth.random_blocks(fmt, N, K, 32), synth.random_blocks(fmt, N, K, 33)
    out = empty16(M, N)
    bridge.dispatch_swiglu(dev(X), dev(Wg), dev(Wu), out, fmt, M, N, K)
    bridge.synchronize()
    ref = oracle.swiglu(fmt, X, Wg, Wu, N)
    Xd = X.astype(np.float64)
    Wgd, Wud = oracle.dequantize_f64(fmt, Wg, K, N), oracle.dequantize_f64(fmt, Wu, K, N)
    g, u = Xd @ Wgd.T, Xd @ Wud.T
    bound = tolerance.swiglu_bound(ref, g, u, np.abs(Xd) @ np.abs(Wgd).T, np.abs(Xd) @ np.abs(Wud).T, K)
    if fmt == 2:
        # Random Q4_K codes reach |w| ~ 2: the fp16 rounding of the weights
        # alone (the bit-exact operands) moves silu(g) u by more than 1/128 at
        # some |out| < 8 (a CPU model with exact fp16-weight products shows
        # 0.018).  The reference checks SwiGLU only on Q4_0, at 0.05
        # (brick3_swiglu_bench.mm:419), so this case keeps the error bound.
        tolerance.check(host(out), ref, bound)
    else:
        tolerance.check_ref(host(out), ref, big_bound=bound, what=f"swiglu fmt {fmt}")


@pytest.mark.parametrize("fmt", [0, 1, 2, 3])
def test_swiglu_gaussian_strict(bridge, oracle, fmt):
    """BASELINE-distribution inputs: flat 1/128."""
    M, K, N = 160, 1024, 192
    X = synth.activations(M, K, 34)
    Wg, Wu = synth.quantized_weights(fmt, N, K, 35), synth.quantized_weights(fmt, N, K, 36)
    out = empty16(M, N)
    bridge.dispatch_swiglu(dev(X), dev(Wg), dev(Wu), out, fmt, M, N, K)
    bridge.synchronize()
    assert maxdiff(host(out), oracle.swiglu(fmt, X, Wg, Wu, N)) <= TOL


# --------------------------------------------------------------------------
# Q8_0 KV cache and attention
# --------------------------------------------------------------------------

def test_quantize_kv_q8_0_bit_exact(bridge, oracle):
    rng = np.random.default_rng(41)
    x = (rng.standard_normal((4096, 32)) * 10.0 ** rng.integers(-5, 4, (4096, 1))).astype(np.float16)
    x[0] = 0
    x[1, 5] = np.float16(-65504)
    q = __import__("torch").empty(x.shape[0] * 34, dtype=__import__("torch").uint8, device="cuda")
    bridge.quantize_kv_q8_0(dev(x), q)
    bridge.synchronize()
    np.testing.assert_array_equal(host(q), oracle.quantize_q8_0(x))


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("M", [1, 33, 127, 128, 129, 256])
def test_flash_attention_q8_0(bridge, oracle, D, M):
    # brick4_attn_bench.mm:216-327: H=8, M in {33,127,128,129,256}, D in {64,128}
    import torch

    H = 8
    rng = np.random.default_rng(M * D)
    Q, K, V = ((rng.standard_normal((H, M, D)) * 0.35).astype(np.float16) for _ in range(3))
    Kq, Vq = oracle.quantize_q8_0(K), oracle.quantize_q8_0(V)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    O = empty16(H, M, D)
    bridge.dispatch_flash_attn_q8_0(dev(Q), dev(Kq), dev(Vq), O, H, M, D, scale)
    Ot = empty16(M, H * D)
    bridge.dispatch_flash_attn_q8_0(dev(Q), dev(Kq), dev(Vq), Ot, H, M, D, scale, o_token_major=True)
    bridge.synchronize()
    ref = oracle.attention_q8_0(Q, Kq, Vq, scale)
    assert maxdiff(host(O), ref) <= TOL
    np.testing.assert_array_equal(host(Ot).reshape(M, H, D).transpose(1, 0, 2), host(O))
    assert torch.isfinite(O).all()


@pytest.mark.parametrize("D,M", [(64, 1000), (64, 384), (64, 640), (128, 777), (128, 384), (128, 640), (128, 2048)])
def test_flash_attention_many_tiles(bridge, oracle, D, M):
    """Many key tiles per query block: the pipelined K/V staging across tile
    counts, the last partial tile, and (M = 384, 640: an odd number of
    128-query tiles) the middle tile that pairs with itself, both wave groups
    splitting every key tile of it and merging at the end.  Key tiles are 128
    keys at D = 64 and 64 keys at D = 128 (one unit per group on a split tile)."""
    H = 2
    rng = np.random.default_rng(D + M)
    Q, K, V = (rng.standard_normal((H, M, D)).astype(np.float16) for _ in range(3))
    Kq, Vq = oracle.quantize_q8_0(K), oracle.quantize_q8_0(V)
    O = empty16(H, M, D)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    bridge.dispatch_flash_attn_q8_0(dev(Q), dev(Kq), dev(Vq), O, H, M, D, scale)
    bridge.synchronize()
    assert maxdiff(host(O), oracle.attention_q8_0(Q, Kq, Vq, scale)) <= TOL


@pytest.mark.parametrize("M", [64, 192])
def test_flash_attention_inf_value_stays_in_its_dims(bridge, oracle, M):
    """A V block with an inf scale at key 0 (dims 32..63 of head 0 all +inf)
    reaches every output of those dims and no other.  At D = 64 a key tile is
    128 keys and the cache is padded to 64: with M = 64 or 192 the last tile
    runs past the padded length, and its masked keys must read zeros, not the
    first keys of the next dim's V^T row (P = 0 times inf is NaN)."""
    H, D = 2, 64
    rng = np.random.default_rng(M + 7)
    Q, K, V = ((rng.standard_normal((H, M, D)) * 0.5).astype(np.float16) for _ in range(3))
    Kq, Vq = oracle.quantize_q8_0(K), oracle.quantize_q8_0(V)
    blk = Vq.reshape(-1, 34)
    blk[1, 0:2] = np.frombuffer(np.float16(np.inf).tobytes(), np.uint8)  # head 0, key 0, dims 32..63
    blk[1, 2:] = 1
    O = empty16(H, M, D)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    print(f"attention inf V M={M}", flush=True)
    bridge.dispatch_flash_attn_q8_0(dev(Q), dev(Kq), dev(Vq), O, H, M, D, scale)
    bridge.synchronize()
    ref = oracle.attention_q8_0(Q, Kq, Vq, scale).astype(np.float64)
    got = host(O).astype(np.float64)
    assert np.isposinf(ref[0, :, 32:]).all() and np.isfinite(np.delete(ref[0], np.s_[32:], axis=1)).all()
    np.testing.assert_array_equal(np.isposinf(got), np.isposinf(ref))
    fin = np.isfinite(ref)
    assert np.isfinite(got[fin]).all()
    assert np.abs(got[fin] - ref[fin]).max() <= TOL


@pytest.mark.parametrize("D", [64, 128])
def test_flash_attention_negative_scale(bridge, oracle, D):
    H, M = 2, 200
    rng = np.random.default_rng(17)
    Q, K, V = ((rng.standard_normal((H, M, D)) * 0.5).astype(np.float16) for _ in range(3))
    Kq, Vq = oracle.quantize_q8_0(K), oracle.quantize_q8_0(V)
    O = empty16(H, M, D)
    bridge.dispatch_flash_attn_q8_0(dev(Q), dev(Kq), dev(Vq), O, H, M, D, -0.125)
    bridge.synchronize()
    assert maxdiff(host(O), oracle.attention_q8_0(Q, Kq, Vq, -0.125)) <= TOL


def test_flash_attention_unit_scale_inputs(bridge, oracle):
    """N(0,1) activations (BASELINE config 5 scale): larger logits."""
    H, M, D = 4, 300, 64
    rng = np.random.default_rng(5)
    Q, K, V = (rng.standard_normal((H, M, D)).astype(np.float16) for _ in range(3))
    Kq, Vq = oracle.quantize_q8_0(K), oracle.quantize_q8_0(V)
    O = empty16(H, M, D)
    bridge.dispatch_flash_attn_q8_0(dev(Q), dev(Kq), dev(Vq), O, H, M, D, 0.125)
    bridge.synchronize()
    assert maxdiff(host(O), oracle.attention_q8_0(Q, Kq, Vq, 0.125)) <= TOL


# --------------------------------------------------------------------------
# Layer
# --------------------------------------------------------------------------

def test_prefill_layer_small(bridge, oracle):
    M, dm, H, D, Nm = 192, 256, 4, 64, 512
    X = synth.activations(M, dm, 51)
    shapes = [(H * D, dm)] * 3 + [(dm, H * D), (Nm, dm), (Nm, dm), (dm, Nm)]
    Ws = [synth.quantized_weights(0, n, k, 60 + i) for i, (n, k) in enumerate(shapes)]
    out = empty16(M, dm)
    bridge.prefill_layer(dev(X), *[dev(w) for w in Ws], out, 0, M, dm, H, D, Nm, 0.125)
    bridge.synchronize()
    ref = oracle.layer(0, X, *Ws, H=H, D=D, N_mlp=Nm, scale=0.125)
    d = maxdiff(host(out), ref)
    print(f"layer max|diff| = {d}")
    # Intermediates are fp16 on both sides; an fp16 tie flipped upstream can move
    # a downstream value by about one output ulp (|y| < 8 -> ulp <= 2^-8).
    assert d <= 2 * TOL


# --------------------------------------------------------------------------
# Small-M weight-streaming kernel (split-K across workgroups)
# --------------------------------------------------------------------------

@pytest.mark.parametrize("fmt", [0, 1, 2, 3])
@pytest.mark.parametrize("M", [1, 16, 33, 64])
def test_skinny_split_k(bridge, oracle, fmt, M):
    K, N = 4096, 320  # 5 column groups, K split across workgroups
    X = synth.activations(M, K, 70 + M)
    W = synth.quantized_weights(fmt, N, K, 71)
    Y = empty16(M, N)
    for _ in range(3):  # repeated calls reuse the self-resetting split-K counters
        bridge.dispatch_gemm(dev(X), dev(W), Y, fmt, M, K, N)
    bridge.synchronize()
    assert maxdiff(host(Y), oracle.gemm(fmt, X, W, N)) <= TOL
    R = synth.activations(M, N, 72)
    Yr = empty16(M, N)
    bridge.dispatch_gemm_residual(dev(X), dev(W), dev(R), Yr, fmt, M, K, N)
    H, D = 5, 64
    Yh = empty16(H, M, D)
    bridge.dispatch_head_gemm(dev(X), dev(W), Yh, fmt, M, H, D, K)
    bridge.synchronize()
    assert maxdiff(host(Yr), oracle.gemm(fmt, X, W, N, R=R)) <= TOL
    assert maxdiff(host(Yh), oracle.gemm(fmt, X, W, N, head_D=D)) <= TOL


def test_baseline_config1_full(bridge, oracle):
    """Q4_0, M=33, K=N=4096, full output vs the oracle."""
    M, K, N = 33, 4096, 4096
    X = synth.activations(M, K, 10)
    W = synth.quantized_weights(0, N, K, 11)
    Y = empty16(M, N)
    bridge.dispatch_gemm(dev(X), dev(W), Y, 0, M, K, N)
    bridge.synchronize()
    assert maxdiff(host(Y), oracle.gemm(0, X, W, N)) <= TOL


@pytest.mark.parametrize("fmt", [0, 1, 2, 3])
@pytest.mark.parametrize("M", [65, 129, 300])
def test_tiled_split_k(bridge, oracle, fmt, M):
    """Tiled kernel with the K range split across workgroups (few tiles)."""
    K, N = 4096, 384
    X = synth.activations(M, K, 80 + M)
    W = synth.quantized_weights(fmt, N, K, 81)
    Y = empty16(M, N)
    for _ in range(2):
        bridge.dispatch_gemm(dev(X), dev(W), Y, fmt, M, K, N)
    R = synth.activations(M, N, 82)
    Yr = empty16(M, N)
    bridge.dispatch_gemm_residual(dev(X), dev(W), dev(R), Yr, fmt, M, K, N)
    bridge.synchronize()
    assert maxdiff(host(Y), oracle.gemm(fmt, X, W, N)) <= TOL
    assert maxdiff(host(Yr), oracle.gemm(fmt, X, W, N, R=R)) <= TOL


def test_gguf_q4_k_tensor_feeds_the_projection(bridge, oracle):
    """A GGML-standard Q4_K tensor read from a GGUF buffer and repacked by
    m4_gguf_load_router_weights drives the tiled projection kernel."""
    import gguf
    from test_gguf import ggml_pack_q4_k, make_gguf

    rng = np.random.default_rng(31)
    M, K, N = 129, 1024, 192
    nb = N * K // 256
    # super-block scales of real Q4_K checkpoints' magnitude (|w| <~ 1)
    q4k = ggml_pack_q4_k((rng.random(nb) * 0.0004 + 1e-5).astype(np.float16), (rng.random(nb) * 0.0004).astype(np.float16),
                         rng.integers(0, 64, (nb, 8)), rng.integers(0, 64, (nb, 8)), rng.integers(0, 16, (nb, 256)))
    ld = gguf.GGUFLoader()
    assert ld.parse_from_buffer(make_gguf([], [("blk.0.ffn_up.weight", [K, N], gguf.GGML_Q4_K, q4k.tobytes())]))
    W, fmt, k, n = ld.load_router_weights("blk.0.ffn_up.weight")
    assert (fmt, k, n) == (2, K, N)
    X = synth.activations(M, K, 32, std=0.35)
    Y = empty16(M, N)
    bridge.dispatch_gemm(dev(X), dev(W), Y, fmt, M, K, N)
    bridge.synchronize()
    tolerance.check_ref(host(Y), oracle.gemm(2, X, W, N), what="gguf q4_k")


# --------------------------------------------------------------------------
# MLX block extras: RMSNorm, RoPE, grouped-query attention, full block
# --------------------------------------------------------------------------

def ulps16(a, b):
    """Distance in binary16 steps between two fp16 arrays of the same sign pattern."""
    ia = np.asarray(a, np.float16).view(np.int16).astype(np.int32)
    ib = np.asarray(b, np.float16).view(np.int16).astype(np.int32)
    ia = np.where(ia < 0, -32768 - ia, ia)
    ib = np.where(ib < 0, -32768 - ib, ib)
    return np.abs(ia - ib)


@pytest.mark.parametrize("norm_type", [1, 2])
@pytest.mark.parametrize("M,D", [(1, 64), (37, 2048), (130, 4096), (8, 8)])
def test_rmsnorm(bridge, oracle, norm_type, M, D):
    """fp16(fp16(x r) w): the GPU forms r in fp32, the oracle in double, so
    x r near an fp16 tie may land one step away, which the exact product with
    w carries into at most two output steps; everything else is exact."""
    rng = np.random.default_rng(M + D)
    X = (rng.standard_normal((M, D)) * 3).astype(np.float16)
    w = (rng.standard_normal(D) * (0.1 if norm_type == 2 else 1.0)).astype(np.float16)
    Y = empty16(M, D)
    bridge.rmsnorm(dev(X), dev(w), Y, eps=1e-5, norm_type=norm_type)
    bridge.synchronize()
    ref = oracle.rmsnorm(X, w, eps=1e-5, norm_type=norm_type)
    u = ulps16(host(Y), ref)
    assert u.max() <= 2 and (u > 0).mean() < 0.01


@pytest.mark.parametrize("traditional", [False, True])
@pytest.mark.parametrize("H,M,D,offset", [(2, 33, 64, 0), (4, 300, 128, 4000), (1, 2048, 64, 0)])
def test_rope(bridge, oracle, traditional, H, M, D, offset):
    rng = np.random.default_rng(H * M + D)
    T = (rng.standard_normal((H, M, D)) * 2).astype(np.float16)
    t = dev(T)
    bridge.rope(t, theta=10000.0, offset=offset, traditional=traditional)
    bridge.synchronize()
    ref = oracle.rope(T, theta=10000.0, offset=offset, traditional=traditional)
    # one fp16 step of the result, plus the fp32 rotation error (a few 2^-24 of
    # the pair's magnitude), which matters only where a cos - b sin cancels
    d = np.abs(host(t).astype(np.float64) - ref.astype(np.float64))
    step = np.spacing(np.abs(ref)).astype(np.float64)
    assert np.all(d <= step + 2.0 ** -20 * float(np.abs(T).max()))
    assert (d > 0).mean() < 0.01


@pytest.mark.parametrize("H,Hkv,M,D", [(8, 2, 129, 64), (4, 1, 300, 128), (6, 3, 64, 64), (4, 2, 1025, 128)])
def test_flash_attention_gqa(bridge, oracle, H, Hkv, M, D):
    rng = np.random.default_rng(H * Hkv + M)
    Q = (rng.standard_normal((H, M, D)) * 0.5).astype(np.float16)
    K, V = ((rng.standard_normal((Hkv, M, D)) * 0.5).astype(np.float16) for _ in range(2))
    Kq, Vq = oracle.quantize_q8_0(K), oracle.quantize_q8_0(V)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    O = empty16(M, H * D)
    bridge.dispatch_flash_attn_q8_0_gqa(dev(Q), dev(Kq), dev(Vq), O, H, Hkv, M, D, scale, o_token_major=True)
    bridge.synchronize()
    ref = oracle.attention_q8_0_gqa(Q, Kq, Vq, Hkv, scale, o_token_major=True)
    assert maxdiff(host(O), ref) <= TOL


@pytest.mark.parametrize("norm_type,rope,traditional,Hq,Hkv,D", [(1, True, False, 4, 2, 64), (2, True, True, 4, 4, 64),
                                                                  (1, False, False, 4, 1, 64),
                                                                  (1, True, False, 2, 1, 128)])
def test_prefill_layer_ex(bridge, oracle, norm_type, rope, traditional, Hq, Hkv, D):
    M, dm, Nm = 160, 256, 512
    X = synth.activations(M, dm, 71)
    w_attn = (1 + 0.1 * np.random.default_rng(72).standard_normal(dm)).astype(np.float16)
    w_ffn = (1 + 0.1 * np.random.default_rng(73).standard_normal(dm)).astype(np.float16)
    if norm_type == 2:
        w_attn, w_ffn = (w_attn - 1).astype(np.float16), (w_ffn - 1).astype(np.float16)
    shapes = [(Hq * D, dm), (Hkv * D, dm), (Hkv * D, dm), (dm, Hq * D), (Nm, dm), (Nm, dm), (dm, Nm)]
    Ws = [synth.quantized_weights(0, n, k, 80 + i) for i, (n, k) in enumerate(shapes)]
    out = empty16(M, dm)
    bridge.prefill_layer_ex(dev(X), dev(w_attn), *[dev(w) for w in Ws[:4]], dev(w_ffn), *[dev(w) for w in Ws[4:]], out,
                            0, M, dm, Hq, Hkv, D, Nm, 0.125, norm_type=norm_type, norm_eps=1e-5, rope=rope,
                            rope_theta=10000.0, rope_offset=17, rope_traditional=traditional)
    bridge.synchronize()
    ref = oracle.layer_ex(0, X, w_attn, *Ws[:4], w_ffn, *Ws[4:], Hq, Hkv, D, Nm, 0.125, norm_type=norm_type,
                          eps=1e-5, rope=rope, theta=10000.0, offset=17, traditional=traditional)
    d = maxdiff(host(out), ref)
    print(f"layer_ex max|diff| = {d}")
    # fp16 intermediates on both sides; a tie flipped upstream (norm, RoPE) moves
    # a downstream value by about one output step
    assert d <= 2 * TOL


@pytest.mark.parametrize("fmt", [0, 1, 2, 3])
@pytest.mark.parametrize("M,K,N", [(1030, 1024, 200), (2048, 2048, 512), (1024, 4096, 264)])
def test_tall_narrow_projections(bridge, oracle, fmt, M, K, N):
    """M >= 1024 with N too small for the wide tile to fill the GPU: the
    128 x 128 tile with (or without) a K split; ragged M and N edges."""
    X = synth.activations(M, K, 95 + fmt)
    W = synth.quantized_weights(fmt, N, K, 96 + fmt)
    Y = empty16(M, N)
    bridge.dispatch_gemm(dev(X), dev(W), Y, fmt, M, K, N)
    bridge.synchronize()
    ref = oracle.gemm(fmt, X, W, N)
    assert maxdiff(host(Y), ref) <= TOL



def test_deferred_tripwire_on_device_output(bridge):
    """A projection whose output is not finite (Q4_0 scales of +inf: (q - 8) inf
    is inf or NaN) raises FloatingPointError at synchronize when the dispatch
    asked for the check (core/bridge/m4_bridge.py:176-177, 227-233); the same
    call without the check, and a clean one with it, do not."""
    M, K, N = 40, 256, 64
    W = synth.random_blocks(0, N, K, 5).reshape(N, K // 32, 18).copy()
    W[..., 0:2] = np.array([np.inf], np.float16).view(np.uint8)
    W = W.reshape(-1)
    X = synth.activations(M, K, 6)
    Y = empty16(M, N)
    bridge.dispatch_gemm(dev(X), dev(W), Y, 0, M, K, N, check_finite=True)
    with pytest.raises(FloatingPointError):
        bridge.synchronize()
    bridge.dispatch_gemm(dev(X), dev(W), Y, 0, M, K, N)
    bridge.synchronize()
    Wc = synth.random_blocks(0, N, K, 7)
    bridge.dispatch_gemm(dev(X), dev(Wc), Y, 0, M, K, N, check_finite=True)
    bridge.synchronize()


def test_every_format_zero_weights_and_nan_activation(bridge):
    """tests/redteam_bridge.py:227-272 and :531-580: all six projection formats
    with all-zero weight blocks run and give a finite (zero) output; an
    activation NaN injected with zero weights trips the deferred check."""
    import torch

    M, K, N = 64, 256, 64
    X = torch.ones((M, K), dtype=torch.float16, device="cuda")
    for fmt, blk_w, blk_b in [(0, 32, 18), (1, 32, 20), (2, 256, 144), (3, 32, 12), (4, 256, 160), (5, 256, 144)]:
        W = torch.zeros((K // blk_w) * N * blk_b, dtype=torch.uint8, device="cuda")
        Y = torch.full((M, N), 3.0, dtype=torch.float16, device="cuda")
        assert bridge.dispatch_gemm(X, W, Y, fmt, M, K, N, check_finite=True) == 0
        bridge.synchronize()
        assert torch.all(Y == 0), fmt
    Xn = torch.ones((M, K), dtype=torch.float16, device="cuda")
    Xn[0, 0] = float("nan")
    W = torch.zeros((K // 32) * N * 18, dtype=torch.uint8, device="cuda")
    Y = torch.zeros((M, N), dtype=torch.float16, device="cuda")
    bridge.dispatch_gemm(Xn, W, Y, 0, M, K, N, check_finite=True)
    with pytest.raises(FloatingPointError):
        bridge.synchronize()


def test_extension_entry_points_error_codes(bridge):
    """Argument checks of the block-extra entry points, before any device work."""
    lib = bridge.lib
    x = empty16(64, 128)
    w = empty16(128)
    assert lib.m4_bridge_rmsnorm(x.data_ptr(), x.numel() * 2, w.data_ptr(), 256, x.data_ptr(), x.numel() * 2, 64,
                                 128, 1e-5, 3) == -3
    assert lib.m4_bridge_rmsnorm(x.data_ptr(), x.numel() * 2, w.data_ptr(), 256, x.data_ptr(), x.numel() * 2, 64,
                                 124, 1e-5, 1) == -4
    assert lib.m4_bridge_rmsnorm(None, 0, w.data_ptr(), 256, x.data_ptr(), x.numel() * 2, 64, 128, 1e-5, 1) == -2
    assert lib.m4_bridge_rmsnorm(x.data_ptr(), 100, w.data_ptr(), 256, x.data_ptr(), x.numel() * 2, 64, 128,
                                 1e-5, 1) == -2
    assert lib.m4_bridge_rope(x.data_ptr(), x.numel() * 2, 1, 64, 120, 1e4, 0, 0) == -4
    assert lib.m4_bridge_rope(x.data_ptr(), x.numel() * 2, 1, 64, 128, 0.0, 0, 0) == -4
    assert lib.m4_bridge_rope(x.data_ptr(), 16, 1, 64, 128, 1e4, 0, 0) == -2
    q8 = torch_empty_u8(64 * 128 // 32 * 34)
    assert lib.m4_bridge_dispatch_flash_attn_q8_0_gqa(x.data_ptr(), x.numel() * 2, q8.data_ptr(), q8.numel(),
                                                      q8.data_ptr(), q8.numel(), x.data_ptr(), x.numel() * 2,
                                                      2, 3, 64, 64, 0.125, 0) == -4
    p = [x.data_ptr()] * 11
    assert lib.m4_bridge_prefill_layer_ex(*p, 0, 64, 128, 4, 3, 64, 256, 0.125, 1, 1e-5, 1, 1e4, 0, 0) == -4
    assert lib.m4_bridge_prefill_layer_ex(*p, 0, 64, 128, 4, 2, 64, 256, 0.125, 5, 1e-5, 1, 1e4, 0, 0) == -3
    assert lib.m4_bridge_prefill_layer_ex(*p[:2], None, *p[3:], 0, 64, 128, 4, 2, 64, 256, 0.125, 1, 1e-5, 1, 1e4,
                                          0, 0) == -2


def torch_empty_u8(n):
    import torch

    return torch.empty(n, dtype=torch.uint8, device="cuda")


# --------------------------------------------------------------------------
# MLX_4BIT_G64 (format 8): MLX's native 64-element groups
# --------------------------------------------------------------------------

def test_mlx_g64_decode_equals_router_repack(bridge):
    """The native g64 decoder and the MLX_4BIT decoder of the lossless
    g64 -> 32-element repack give the same binary16 weights, bit for bit."""
    N, K = 96, 1024
    scale, bias, packed = synth.quantize_mlx_g64(synth.gaussian_weights(N, K, 401))
    Wg = synth.mlx_g64_blocks(scale, bias, packed)
    Wr = synth.mlx_g64_to_router_blocks(scale, bias, packed)
    a, b = empty16(N, K), empty16(N, K)
    bridge.dequantize(dev(Wg), a, 8, K, N)
    bridge.dequantize(dev(Wr), b, 1, K, N)
    bridge.synchronize()
    np.testing.assert_array_equal(host(a).view(np.uint16), host(b).view(np.uint16))


@pytest.mark.parametrize("M", [1, 16, 33, 64, 127, 128, 129, 300, 2048])
@pytest.mark.parametrize("kind", ["random", "quantized"])
def test_mlx_g64_projection(bridge, oracle, M, kind):
    """Small-M (M <= 64, K split) and tiled kernels, standard, residual and
    direct-head outputs, on reference-style random groups and on N(0, 0.02)
    weights quantized by MLX's rule."""
    K, N = (512, 256) if M in (127, 2048) else (2048, 320)
    std = 0.35 if kind == "random" else 1.0
    X = synth.activations(M, K, 410 + M, std=std)
    W = weights(kind, 8, N, K, 411 + M)
    Y = empty16(M, N)
    bridge.dispatch_router_gemm(dev(X), dev(W), Y, 8, M, K, N)
    R = synth.activations(M, N, 412)
    Yr = empty16(M, N)
    bridge.dispatch_gemm_residual(dev(X), dev(W), dev(R), Yr, 8, M, K, N)
    H, D = N // 64, 64
    Yh = empty16(H, M, D)
    bridge.dispatch_head_gemm(dev(X), dev(W), Yh, 8, M, H, D, K)
    with pytest.raises(RuntimeError):  # the reference's projection entry point keeps formats 0..5
        bridge.dispatch_gemm(dev(X), dev(W), empty16(M, N), 8, M, K, N)
    bridge.synchronize()
    tolerance.check_ref(host(Y), oracle.gemm(8, X, W, N), what=f"g64 {kind} M={M}")
    tolerance.check_ref(host(Yr), oracle.gemm(8, X, W, N, R=R), what="g64 residual")
    tolerance.check_ref(host(Yh), oracle.gemm(8, X, W, N, head_D=D), what="g64 direct-head")


@pytest.mark.parametrize("rope", [False, True])
def test_prefill_layer_writes_its_q8_0_kv_cache(bridge, oracle, rope):
    """m4_bridge_prefill_layer_ex_kv hands back the layer's Q8_0 KV cache
    (unified_prefill_engine.mm:548-572): its blocks are the Q8_0 quantization
    (bit-exact) of the K and V the layer projected -- recomputed here with the
    head-major projection and RoPE entry points -- and the layer output equals
    the entry point without the cache outputs, bit for bit."""
    import torch

    M, dm, Hq, Hkv, D, Nm = 192, 256, 4, 2, 64, 512
    X = synth.activations(M, dm, 301)
    shapes = [(Hq * D, dm), (Hkv * D, dm), (Hkv * D, dm), (dm, Hq * D), (Nm, dm), (Nm, dm), (dm, Nm)]
    Ws = [dev(synth.quantized_weights(0, n, k, 310 + i)) for i, (n, k) in enumerate(shapes)]
    Xd = dev(X)
    nb = Hkv * M * D // 32
    Kq = torch.zeros(nb * 34, dtype=torch.uint8, device="cuda")
    Vq = torch.zeros(nb * 34, dtype=torch.uint8, device="cuda")
    out_kv, out = empty16(M, dm), empty16(M, dm)
    lib = bridge.lib
    args = (0, M, dm, Hq, Hkv, D, Nm, 0.125, 1, 1e-5, int(rope), 10000.0, 3, 0)
    ptr = [t.data_ptr() for t in Ws]
    assert lib.m4_bridge_prefill_layer_ex_kv(Xd.data_ptr(), None, *ptr[:4], None, *ptr[4:], out_kv.data_ptr(),
                                             Kq.data_ptr(), Vq.data_ptr(), *args) == 0
    assert lib.m4_bridge_prefill_layer_ex(Xd.data_ptr(), None, *ptr[:4], None, *ptr[4:], out.data_ptr(), *args) == 0
    assert lib.m4_bridge_prefill_layer_ex_kv(Xd.data_ptr(), None, *ptr[:4], None, *ptr[4:], out.data_ptr(),
                                             Kq.data_ptr(), None, *args) == -2
    K = empty16(Hkv, M, D)
    V = empty16(Hkv, M, D)
    bridge.dispatch_head_gemm(Xd, Ws[1], K, 0, M, Hkv, D, dm)
    bridge.dispatch_head_gemm(Xd, Ws[2], V, 0, M, Hkv, D, dm)
    if rope:
        bridge.rope(K, theta=10000.0, offset=3)
    bridge.synchronize()
    np.testing.assert_array_equal(host(out_kv).view(np.uint16), host(out).view(np.uint16))
    np.testing.assert_array_equal(host(Kq), oracle.quantize_q8_0(host(K)))
    np.testing.assert_array_equal(host(Vq), oracle.quantize_q8_0(host(V)))


@pytest.mark.parametrize("fmt", [0, 1, 2, 3, 8])
@pytest.mark.parametrize("M", [1, 16, 33, 64])
def test_small_m_wide_n(bridge, oracle, fmt, M):
    """Small M, wide ragged N (last 64-column group partly out of range), K
    split across workgroups: standard, residual and direct-head outputs."""
    K, N = 2048, 4096 + 48
    X = synth.activations(M, K, 600 + M)
    W = synth.quantized_weights(fmt, N, K, 601 + fmt)
    Y = empty16(M, N)
    bridge.dispatch_router_gemm(dev(X), dev(W), Y, fmt, M, K, N)
    R = synth.activations(M, N, 602)
    Yr = empty16(M, N)
    bridge.dispatch_gemm_residual(dev(X), dev(W), dev(R), Yr, fmt, M, K, N)
    H, D = N // 16, 16
    Yh = empty16(H, M, D)
    bridge.dispatch_head_gemm(dev(X), dev(W), Yh, fmt, M, H, D, K)
    bridge.synchronize()
    assert maxdiff(host(Y), oracle.gemm(fmt, X, W, N)) <= TOL
    assert maxdiff(host(Yr), oracle.gemm(fmt, X, W, N, R=R)) <= TOL
    assert maxdiff(host(Yh), oracle.gemm(fmt, X, W, N, head_D=D)) <= TOL
