"""The BASELINE-configuration quantizers (synth.py) against their closed forms.

BASELINE.json's configs draw W ~ N(0, 0.02) and quantize it; the reference
ships no quantizer for these layouts (its generators draw random codes,
bench_universal_router.mm:36-103), so the build defines them and pins them
here by what their definitions fix:

* Q4_0:    d = m / -8 with m the signed value of max |w| of the block; codes
           0..15; the absmax element is exact; |w - (q - 8) d| <= |d| / 2
           (plus the fp16 rounding of d), |d| at the one clamped code (+8).
* MLX g64: scale = fp16((max - min) / 15), bias = fp16(min); codes 0..15, 8
           per u32 LSB first; the min element has code 0, the max code 15;
           |w - (q scale + bias)| <= scale / 2 plus the fp16 roundings.
* Q4_K:    d = fp16(max_j scale_j / 63), dmin = fp16(max_j min_j / 63) over
           the 8 sub-blocks (scale_j = (max - min') / 15, min' = min(min, 0));
           6-bit sc / m in range; the widest sub-block has sc near 63;
           reconstruction error bounded by the affine fit's step.
* Ternary: codes {0, 1, 2} (never 3) with frequencies {.25, .5, .25}; ONE
           per-tensor scale replicated into every block.
Reconstructions go through the oracle's pinned dequantizer, so a quantizer
that packs codes or scales in the wrong place fails the error bound.
"""
from __future__ import annotations

import numpy as np

import synth

F16_REL = 2.0 ** -11  # unit roundoff of binary16


def test_q4_0_closed_form(oracle):
    N, K = 64, 1024
    w = synth.gaussian_weights(N, K, 5)
    W = synth.quantize_q4_0(w).reshape(N, K // 32, 18)
    b = w.reshape(N, K // 32, 32).astype(np.float64)
    # d = signed absmax / -8, stored as fp16
    idx = np.abs(b).argmax(-1)
    m = np.take_along_axis(b, idx[..., None], -1)[..., 0]
    d16 = W[..., 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    np.testing.assert_array_equal(d16, (m / -8.0).astype(np.float32).astype(np.float16).astype(np.float64))
    # codes 0..15 in the reference nibble order (byte i: element i low, i + 16 high)
    q = np.concatenate([W[..., 2:] & 15, W[..., 2:] >> 4], -1).astype(np.int64)
    assert q.min() >= 0 and q.max() <= 15
    wh = oracle.dequantize_f64(0, W.reshape(-1), K, N).reshape(N, K // 32, 32)
    np.testing.assert_array_equal(wh, (q - 8) * d16[..., None])
    err = np.abs(b - wh)
    # the absmax element maps to code 0 (q - 8 = -8) and is exact up to d's rounding
    amax_err = np.take_along_axis(err, idx[..., None], -1)[..., 0]
    assert np.all(amax_err <= 8 * np.abs(m / -8.0 - d16) + 1e-12)
    assert np.all(np.take_along_axis(q, idx[..., None], -1) == 0)
    clamped = b / np.where(d16 != 0, d16, 1)[..., None] > 7.5
    lim = np.abs(d16)[..., None] * (0.5 + 8 * F16_REL) + 1e-9
    assert np.all(err[~clamped] <= np.broadcast_to(lim, err.shape)[~clamped])
    assert np.all(err[clamped] <= np.broadcast_to(np.abs(d16)[..., None] * (1 + 8 * F16_REL), err.shape)[clamped])


def test_mlx_g64_closed_form(oracle):
    N, K = 48, 1024
    w = synth.gaussian_weights(N, K, 6)
    scale, bias, packed = synth.quantize_mlx_g64(w)
    g = w.reshape(N, K // 64, 64).astype(np.float64)
    mn, mx = g.min(-1), g.max(-1)
    np.testing.assert_array_equal(scale, ((mx - mn) / 15.0).astype(np.float32).astype(np.float16))
    np.testing.assert_array_equal(bias, mn.astype(np.float32).astype(np.float16))
    # 8 codes per u32, element 8i + j at bits 4j of word i
    assert packed.shape == (N, K // 8) and packed.dtype == np.uint32
    q = np.stack([(packed >> np.uint32(4 * j)) & np.uint32(15) for j in range(8)], -1).reshape(N, K // 64, 64)
    q = q.astype(np.int64)
    s, bb = scale.astype(np.float64)[..., None], bias.astype(np.float64)[..., None]
    wh = q * s + bb
    err = np.abs(g - wh)
    lim = s / 2 + np.abs(bb) * F16_REL + 15 * s * F16_REL + 1e-9
    assert np.all(err <= lim)
    assert np.all(np.take_along_axis(q, g.argmin(-1)[..., None], -1) == 0)
    assert np.all(np.take_along_axis(q, g.argmax(-1)[..., None], -1) == 15)
    # the router blocks decode (oracle, exact double) to the same affine values
    W = synth.mlx_g64_to_router_blocks(scale, bias, packed)
    np.testing.assert_array_equal(oracle.dequantize_f64(1, W, K, N).reshape(N, K // 64, 64), wh)


def test_q4_k_closed_form(oracle):
    N, K = 32, 2048
    w = synth.gaussian_weights(N, K, 7)
    W = synth.quantize_q4_k(w).reshape(N, K // 256, 144)
    b = w.reshape(N, K // 256, 8, 32).astype(np.float64)
    lo = np.minimum(b.min(-1), 0.0)
    scale = (b.max(-1) - lo) / 15.0
    minv = -lo
    d16 = W[..., 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    dm16 = W[..., 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    np.testing.assert_array_equal(d16, (scale.max(-1) / 63.0).astype(np.float32).astype(np.float16))
    np.testing.assert_array_equal(dm16, (minv.max(-1) / 63.0).astype(np.float32).astype(np.float16))
    # 6-bit scales / mins unpacked as the reference's gold does (cpu_gold_reference.h:121-127)
    s = W[..., 4:16].astype(np.int64)
    sc = np.concatenate([s[..., 0:4] & 63, s[..., 4:8] & 63], -1)
    mm = np.concatenate([(s[..., 8:12] & 15) | ((s[..., 0:4] >> 6) << 4),
                         (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)], -1)
    assert sc.max() <= 63 and mm.max() <= 63
    # the widest sub-block's scale is the super-block's: sc = 63 up to d's fp16 rounding
    widest = np.take_along_axis(sc, scale.argmax(-1)[..., None], -1)[..., 0]
    assert np.all(widest >= 62)
    A = d16[..., None] * sc
    B = dm16[..., None] * mm
    # sc, m are the nearest 6-bit multiples
    assert np.all(np.abs(A - scale) <= d16[..., None] * (0.5 + 63 * F16_REL) + 1e-12)
    assert np.all(np.abs(B - minv) <= dm16[..., None] * (0.5 + 63 * F16_REL) + 1e-12)
    wh = oracle.dequantize_f64(2, W.reshape(-1), K, N).reshape(N, K // 256, 8, 32)
    err = np.abs(b - wh)
    # one affine step of the fit, plus what the 6-bit rounding of the scale
    # (over 15 steps) and of the min shift the covered range by
    lim = A / 2 + np.abs(B - minv) + 15 * np.abs(A - scale) + 1e-9
    assert np.all(err <= lim[..., None])
    # and the fit is tight in absolute terms for N(0, 0.02) weights
    assert err.max() < 0.02


def test_ternary_closed_form(oracle):
    N, K = 256, 2048
    W = synth.ternary_weights(N, K, 8).reshape(N, K // 32, 12)
    d = W[..., 0:2].copy().view(np.float16)[..., 0]
    assert np.all(d == np.float16(0.02)), "one per-tensor scale in every block"
    assert np.all(W[..., 2:4] == 0)
    words = W[..., 4:12].copy().view(np.uint32)
    c = np.stack([(words >> np.uint32(2 * j)) & np.uint32(3) for j in range(16)], -1).reshape(N, K // 32, 32)
    assert c.max() <= 2, "code 3 never emitted"
    freq = np.bincount(c.reshape(-1), minlength=3) / c.size
    # n = 524288 draws: 6 standard deviations of a frequency is < 0.004
    np.testing.assert_allclose(freq, [0.25, 0.5, 0.25], atol=0.004)
    wh = oracle.dequantize_f64(3, W.reshape(-1), K, N).reshape(N, K // 32, 32)
    np.testing.assert_array_equal(wh, (c.astype(np.int64) - 1) * np.float64(np.float16(0.02)))
