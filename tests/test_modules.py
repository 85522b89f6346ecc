"""The quantized linear layer (modules.py) against the reference's module
behaviour (src/engine/modules.py) and its tests (tests/test_modules_basic.py:
40-136): format normalisation, byte sizing and validation errors, the
synthetic weight generator (unit weights decode to exactly +1 through the
pinned oracle dequantizer; a seed gives the same bytes), and on the GPU the
prefill / decode / 1-D / batched forward paths, including parity against the
oracle on seeded random blocks.
"""
from __future__ import annotations

import numpy as np
import pytest

import modules
import synth
import tolerance
from m4_bridge import QuantFormat


def test_normalize_format():
    assert modules.normalize_format(0) == QuantFormat.QUANT_Q4_0
    assert modules.normalize_format(QuantFormat.QUANT_Q4_K) == QuantFormat.QUANT_Q4_K
    assert modules.normalize_format("q4_0") == QuantFormat.QUANT_Q4_0
    assert modules.normalize_format(" mlx_4bit ") == QuantFormat.QUANT_MLX_4BIT
    assert modules.normalize_format("QUANT_TERNARY_1_58") == QuantFormat.QUANT_TERNARY_1_58
    with pytest.raises(ValueError):
        modules.normalize_format("q5_k")
    with pytest.raises(TypeError):
        modules.normalize_format(1.5)


def test_compute_quantized_weight_bytes():
    assert modules.compute_quantized_weight_bytes(0, 4096, 4096) == 128 * 4096 * 18
    assert modules.compute_quantized_weight_bytes("mlx_4bit", 4096, 14336) == 128 * 14336 * 20
    assert modules.compute_quantized_weight_bytes(QuantFormat.QUANT_Q4_K, 4096, 4096) == 16 * 4096 * 144
    assert modules.compute_quantized_weight_bytes(3, 2048, 8192) == 64 * 8192 * 12
    assert modules.compute_quantized_weight_bytes(4, 256, 2) == 2 * 160
    with pytest.raises(ValueError):
        modules.compute_quantized_weight_bytes(0, 0, 4)
    with pytest.raises(ValueError):
        modules.compute_quantized_weight_bytes(2, 128, 4)  # Q4_K needs whole 256-element super-blocks


@pytest.mark.parametrize("fmt,w_expected", [(0, 1.0), (1, 1.0), (3, 1.0), (2, 1.0 / 32.0)])
def test_unit_synthetic_weights_decode_to_constants(oracle, fmt, w_expected):
    K, N = 512, 8
    W = modules.generate_synthetic_quantized_weights(fmt, K, N, scale=1.0, unit_weights=True, device="cpu")
    assert W.numel() == modules.compute_quantized_weight_bytes(fmt, K, N)
    w = oracle.dequantize_f64(fmt, W.numpy(), K, N)
    np.testing.assert_array_equal(w, np.full_like(w, w_expected))


@pytest.mark.parametrize("fmt", [0, 1, 2, 3, 4, 5])
def test_seeded_synthetic_weights_are_deterministic(fmt):
    a = modules.generate_synthetic_quantized_weights(fmt, 512, 4, unit_weights=False, seed=7, device="cpu")
    b = modules.generate_synthetic_quantized_weights(fmt, 512, 4, unit_weights=False, seed=7, device="cpu")
    c = modules.generate_synthetic_quantized_weights(fmt, 512, 4, unit_weights=False, seed=8, device="cpu")
    assert bool((a == b).all())
    assert not bool((a == c).all())


def test_layer_validation_errors():
    with pytest.raises(ValueError):
        modules.M4QuantizedLinear(100, 8, format=0)        # not whole 32-blocks
    with pytest.raises(ValueError):
        modules.M4QuantizedLinear(0, 8, format=0)
    with pytest.raises(ValueError):
        modules.M4QuantizedLinear(128, 8, format="q4_k")    # super-block format, 128 % 256 != 0
    with pytest.raises(ValueError):
        modules.M4QuantizedLinear.from_quantized(bytes(17), 0, 32, 1)  # 18 bytes expected
    with pytest.raises(KeyError):
        modules.M4QuantizedLinear(256, 8, format=6)         # Q8_0 weights: no layer format, as in the reference


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", [0, 1, 3])
def test_layer_prefill_decode_and_1d(bridge, fmt):
    """tests/test_modules_basic.py:40-86: unit weights, x = ones -> every output K."""
    import torch

    K, N = 64, 64
    layer = modules.M4QuantizedLinear(K, N, format=fmt)
    layer.init_synthetic_weights(scale=1.0)
    for M in (2, 33, 64, 128):
        y = layer(torch.ones(M, K, dtype=torch.float16, device="cuda"))
        bridge.synchronize()
        assert y.shape == (M, N) and y.dtype == torch.float16
        assert bool((y == K).all()), f"format {fmt} M={M}"
    y = layer(torch.ones(1, K, dtype=torch.float16, device="cuda"))   # decode row -> GEMV
    y1 = layer(torch.ones(K, dtype=torch.float16, device="cuda"))     # 1-D input -> GEMV
    bridge.synchronize()
    assert y.shape == (1, N) and bool((y == K).all())
    assert y1.shape == (N,) and bool((y1 == K).all())


@pytest.mark.gpu
def test_layer_super_block_and_batching(bridge):
    """tests/test_modules_basic.py:89-136: Q4_K unit weights (K / 32 per output)
    and leading batch dimensions through GEMV and GEMM."""
    import torch

    K, N = 256, 64
    layer = modules.M4QuantizedLinear(K, N, format="q4_k")
    layer.init_synthetic_weights(scale=1.0)
    y = layer(torch.ones(16, K, dtype=torch.float16, device="cuda"), check_finite=True)
    assert y.shape == (16, N) and bool((y == K / 32).all())
    for shape in ((1, 1, K), (4, 1, K), (2, 16, K)):
        yb = layer(torch.ones(*shape, dtype=torch.float16, device="cuda"))
        bridge.synchronize()
        assert yb.shape == (*shape[:-1], N) and bool((yb == K / 32).all())
    e = layer(torch.ones(0, 3, K, dtype=torch.float16, device="cuda"))
    assert e.shape == (0, 3, N)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt,M", [(0, 33), (1, 128), (3, 129), (2, 64)])
def test_layer_random_blocks_match_the_oracle(bridge, oracle, fmt, M):
    import torch

    K, N = 512, 192
    layer = modules.M4QuantizedLinear(K, N, format=fmt)
    layer.init_synthetic_weights(scale=0.05, unit_weights=False, seed=11 + fmt)
    X = synth.activations(M, K, 3 + fmt, std=0.35)
    y = layer(torch.from_numpy(X).cuda())
    bridge.synchronize()
    gold = oracle.gemm(fmt, X, layer.weight.cpu().numpy(), N)
    tolerance.check_ref(y.cpu().numpy(), gold, what=f"layer fmt {fmt} M={M}")
