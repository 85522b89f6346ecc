"""m4_bridge_dispatch_gemm_noalloc: the projection entry point that allocates
nothing (split-K partials in the library's fixed device scratch array).

Checked through the C-ABI against m4_bridge_dispatch_gemm on the same inputs,
bit for bit (both run the same kernels; the split-K sums are taken in split
order, so the workspace they live in cannot change a bit), on two calls in a
row -- the second smaller, so stale partials of the first would show -- and at
the BASELINE headline and config 1 (single kernels with no partials: the
entry point must run them unchanged).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _run(lib, fn, X, W, fmt, M, K, N):
    import torch

    Y = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
    rc = fn(X.data_ptr(), X.numel() * 2, W.data_ptr(), W.numel(), Y.data_ptr(), Y.numel() * 2, fmt, M, K, N)
    assert rc == 0, (rc, lib.m4_bridge_last_error())
    return Y


@pytest.mark.parametrize("calls", [
    [(1, 128, 4096, 14336), (0, 33, 4096, 4096)],    # headline (K groups), then config 1 (small-M, one kernel)
    [(0, 300, 4096, 384), (2, 65, 2048, 256)],       # tiled split-K shapes, second smaller
    [(3, 48, 4096, 2048), (1, 16, 2048, 512)],       # small-M split-K, second smaller
])
def test_noalloc_matches_dispatch_gemm(bridge, calls):
    import torch

    lib = bridge.lib
    for i, (fmt, M, K, N) in enumerate(calls):
        print(f"noalloc call {i}: fmt={fmt} M={M} K={K} N={N}", flush=True)
        X = _dev(synth.activations(M, K, 500 + i))
        W = _dev(synth.quantized_weights(fmt, N, K, 510 + i))
        Yn = _run(lib, lib.m4_bridge_dispatch_gemm_noalloc, X, W, fmt, M, K, N)
        Yr = _run(lib, lib.m4_bridge_dispatch_gemm, X, W, fmt, M, K, N)
        bridge.synchronize()
        assert torch.isfinite(Yn).all()
        np.testing.assert_array_equal(Yn.cpu().numpy().view(np.uint16), Yr.cpu().numpy().view(np.uint16))


def test_noalloc_refusals(bridge):
    """Host buffers (would need staging) give -2, a shape whose partials
    exceed the scratch gives -4; the bridge keeps working afterwards."""
    lib = bridge.lib
    M, K, N = 32, 256, 64
    Xh = synth.activations(M, K, 520)
    Wh = synth.quantized_weights(0, N, K, 521)
    Yh = np.zeros((M, N), np.float16)
    assert lib.m4_bridge_dispatch_gemm_noalloc(Xh.ctypes.data, Xh.nbytes, Wh.ctypes.data, Wh.nbytes, Yh.ctypes.data,
                                               Yh.nbytes, 0, M, K, N) == -2
    assert b"device memory" in lib.m4_bridge_last_error()
    # small-M kernel, K split 16: 16 x 48 x 12288 floats of partials > 8 Mi
    import torch

    M, K, N = 48, 16384, 12288
    X = torch.zeros(M, K, dtype=torch.float16, device="cuda")
    W = torch.zeros(N * K // 32 * 18, dtype=torch.uint8, device="cuda")
    Y = torch.zeros(M, N, dtype=torch.float16, device="cuda")
    rc = lib.m4_bridge_dispatch_gemm_noalloc(X.data_ptr(), X.numel() * 2, W.data_ptr(), W.numel(), Y.data_ptr(),
                                             Y.numel() * 2, 0, M, K, N)
    assert rc == -4, rc
    assert b"fixed scratch" in lib.m4_bridge_last_error()
    M, K, N = 8, 256, 64
    Xs = _dev(synth.activations(M, K, 522))
    Ws = _dev(synth.quantized_weights(0, N, K, 523))
    Ya = _run(lib, lib.m4_bridge_dispatch_gemm_noalloc, Xs, Ws, 0, M, K, N)
    Yb = _run(lib, lib.m4_bridge_dispatch_gemm, Xs, Ws, 0, M, K, N)
    bridge.synchronize()
    np.testing.assert_array_equal(Ya.cpu().numpy().view(np.uint16), Yb.cpu().numpy().view(np.uint16))
