"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each check is chosen so a plausible mistake in the restatement fails it:
known-answer tests from the reference's own suites, layout probes (one code
set at a time), closed forms at exactly representable scales, agreement of
the reference's two independent texts (its generator's packing vs its gold's
unpacking), an independent IEEE implementation (numpy) for the fp16
rounding, and brute-force numpy evaluation of the reductions.
"""
from __future__ import annotations

import numpy as np
import pytest

import synth

F16_ONE = np.array([1.0], np.float16).view(np.uint8)


def _f16(x):
    return np.array([x], np.float16).view(np.uint8)


# --------------------------------------------------------------------------
# binary16 conversions
# --------------------------------------------------------------------------

def test_f16_roundtrip_exhaustive(oracle):
    h = np.arange(65536, dtype=np.uint16).view(np.float16)
    finite = np.isfinite(h)
    d = oracle.f16_to_f64(h)
    np.testing.assert_array_equal(d[finite], h[finite].astype(np.float64))
    back = oracle.f64_to_f16(d[finite])
    np.testing.assert_array_equal(back.view(np.uint16), h[finite].view(np.uint16))


def test_f64_to_f16_matches_numpy_rne(oracle):
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000) * 10.0 ** rng.integers(-9, 5, 200000),
        # exact ties between adjacent halves, both parities, incl. subnormals
        (np.arange(-3000, 3000) + 0.5) * 2.0 ** -24,
        (np.arange(1024, 2048) + 0.5) * 2.0 ** -10,
        np.array([65504.0, 65519.99, 65520.0, -65520.0, 1e-9, -1e-9, 0.0, -0.0]),
    ])
    ours = oracle.f64_to_f16(x).view(np.uint16)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)  # numpy: single RNE rounding
    np.testing.assert_array_equal(ours, ref)


# --------------------------------------------------------------------------
# Dequantization: known answers and layout probes
# --------------------------------------------------------------------------

def _q4_0_block(d, qs):
    return np.concatenate([_f16(d), np.asarray(qs, np.uint8)])


def test_q4_0_kat_nibble8_is_zero(oracle):
    # tests/e2e/test_tier1_feature_coverage.mm:248-257
    w = oracle.dequantize(0, _q4_0_block(0.5, [0x88] * 16), 32, 1)
    assert np.all(w == 0)


def test_q4_0_layout_and_values(oracle):
    # byte i low nibble -> element i, high nibble -> element i+16; w = (q-8)*d
    for i in range(16):
        for hi in (False, True):
            for q in range(16):
                qs = np.full(16, 0x88, np.uint8)
                qs[i] = (q << 4 | 8) if hi else (0x80 | q)
                w = oracle.dequantize(0, _q4_0_block(0.25, qs), 32, 1)[0].astype(np.float64)
                exp = np.zeros(32)
                exp[i + 16 if hi else i] = (q - 8) * 0.25
                np.testing.assert_array_equal(w, exp)


def test_mlx_kat(oracle):
    # d = 0, bias = 0.5: every weight 0.5 (test_tier1_feature_coverage.mm:287-297)
    blk = np.concatenate([_f16(0.0), _f16(0.5), np.full(16, 0x37, np.uint8)])
    w = oracle.dequantize(1, blk, 32, 1)
    assert np.all(w == 0.5) and float(w.astype(np.float64).sum()) == 16.0
    # w = q*d + bias: probe every code at an exact scale
    for q in range(16):
        blk = np.concatenate([_f16(0.125), _f16(-1.0), np.full(16, q | (q << 4), np.uint8)])
        assert np.all(oracle.dequantize(1, blk, 32, 1) == q * 0.125 - 1.0)


def test_ternary_kat_and_layout(oracle):
    # 0x55555555 = code 1 everywhere -> 0 (test_tier1_feature_coverage.mm:363-376)
    blk = np.concatenate([_f16(0.75), np.zeros(2, np.uint8),
                          np.array([0x55555555, 0x55555555], np.uint32).view(np.uint8)])
    assert np.all(oracle.dequantize(3, blk, 32, 1) == 0)
    # element j <- bits 2j of qs[j // 16]; code c -> (c-1)*d, code 3 -> +2d (CPU gold)
    for j in range(32):
        for c in range(4):
            words = np.array([0x55555555, 0x55555555], np.uint32)
            words[j // 16] = (words[j // 16] & ~np.uint32(3 << (2 * (j % 16)))) | np.uint32(c << (2 * (j % 16)))
            blk = np.concatenate([_f16(0.5), np.zeros(2, np.uint8), words.view(np.uint8)])
            w = oracle.dequantize(3, blk, 32, 1)[0].astype(np.float64)
            exp = np.zeros(32)
            exp[j] = (c - 1) * 0.5
            np.testing.assert_array_equal(w, exp)


def test_q4_k_scale_packing_agrees_with_reference_generator(oracle):
    """The reference packs (sc, min) in its generator (bench_universal_router.mm:
    70-78) and unpacks them in its gold (cpu_gold_reference.h:121-127); synth
    restates the former, the oracle the latter.  With d = dmin = 1, q = 0 gives
    -min and q = 1 gives sc - min for every sub-block."""
    rng = np.random.default_rng(1)
    for trial in range(64):
        sc = rng.integers(0, 64, 8) if trial else np.arange(8) * 9
        mn = rng.integers(0, 64, 8) if trial else 63 - np.arange(8) * 9
        blk = np.zeros(144, np.uint8)
        blk[0:2] = _f16(1.0)
        blk[2:4] = _f16(1.0)
        blk[4:16] = synth._pack_q4k_scales(sc[None], mn[None])[0]
        blk[16:] = 0x10  # low nibble 0 (elements 0..15), high nibble 1 (16..31) of each sub-block
        w = oracle.dequantize(2, blk, 256, 1)[0].astype(np.float64).reshape(8, 32)
        np.testing.assert_array_equal(w[:, :16], np.repeat(-mn[:, None].astype(float), 16, 1))
        np.testing.assert_array_equal(w[:, 16:], np.repeat((sc - mn)[:, None].astype(float), 16, 1))


def test_q4_k_sub_block_qs_layout(oracle):
    # sub-block s uses qs[16s .. 16s+15]; byte i -> elements 32s+i and 32s+i+16
    for s in range(8):
        for i in (0, 7, 15):
            blk = np.zeros(144, np.uint8)
            blk[0:2] = _f16(0.5)
            blk[4:16] = synth._pack_q4k_scales(np.full((1, 8), 2), np.zeros((1, 8), int))[0]
            blk[16 + 16 * s + i] = 0x31
            w = oracle.dequantize(2, blk, 256, 1)[0].astype(np.float64)
            exp = np.zeros(256)
            exp[32 * s + i] = 1 * 0.5 * 2
            exp[32 * s + i + 16] = 3 * 0.5 * 2
            np.testing.assert_array_equal(w, exp)


@pytest.mark.parametrize("fmt", [0, 1, 2, 3])
def test_dequant_f64_rounds_to_dequant(oracle, fmt):
    W = synth.random_blocks(fmt, 8, 512, 40 + fmt)
    np.testing.assert_array_equal(oracle.dequantize_f64(fmt, W, 512, 8).astype(np.float16),
                                  oracle.dequantize(fmt, W, 512, 8))


def test_dequant_single_rounding_q4_k(oracle):
    """q*(d*sc) - dmin*m is rounded ONCE to fp16 (no fp16 intermediate)."""
    rng = np.random.default_rng(2)
    W = synth.random_blocks(2, 16, 512, 3)
    w = oracle.dequantize(2, W, 512, 16).astype(np.float64)
    blk = W.reshape(16, 2, 144)
    d = blk[..., 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    dmin = blk[..., 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    # decode sc/min through the generator-side packing inverse (independent: bit masks per the header)
    s = blk[..., 4:16].astype(np.int64)
    sc = np.concatenate([s[..., 0:4] & 63, s[..., 4:8] & 63], -1)
    mn = np.concatenate([(s[..., 8:12] & 15) | ((s[..., 0:4] >> 6) << 4),
                         (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)], -1)
    qs = blk[..., 16:].reshape(16, 2, 8, 16).astype(np.int64)
    q = np.concatenate([qs & 15, qs >> 4], -1)  # [n, sb, s, 32]
    exact = q * (d[..., None, None] * sc[..., None]) - (dmin[..., None, None] * mn[..., None])
    np.testing.assert_array_equal(w.reshape(exact.shape), exact.astype(np.float16).astype(np.float64))
    assert rng is not None


# --------------------------------------------------------------------------
# Projections
# --------------------------------------------------------------------------

def test_bridge_kat_q4_0_ones(oracle):
    # tests/test_bridge_basic.py:41-83: d = 1.0 (0x3C00), nibbles 0x99 -> w = 1; X = 1 -> Y = K
    for M, K, N in [(33, 64, 64), (64, 64, 64), (128, 128, 128)]:
        blk = np.concatenate([np.array([0x00, 0x3C], np.uint8), np.full(16, 0x99, np.uint8)])
        W = np.tile(blk, (K // 32) * N)
        Y = oracle.gemm(0, np.ones((M, K), np.float16), W, N)
        assert np.all(Y == K)


def test_bridge_kat_mlx_ones(oracle):
    # tests/test_bridge_basic.py:86-118: d = 1, bias = 0, nibbles 1 -> Y = K
    M = K = N = 64
    blk = np.concatenate([np.array([0x00, 0x3C, 0x00, 0x00], np.uint8), np.full(16, 0x11, np.uint8)])
    Y = oracle.gemm(1, np.ones((M, K), np.float16), np.tile(blk, (K // 32) * N), N)
    assert np.all(Y == K)


@pytest.mark.parametrize("fmt", [0, 1, 2, 3])
def test_gemm_matches_numpy_matmul(oracle, fmt):
    """Oracle GEMM vs numpy float64 matmul of the (separately pinned)
    dequantized weights: catches transposed operands, index and block-order
    mistakes.  Both are double; outputs may differ by one fp16 ulp only where
    the double sums straddle a rounding boundary."""
    M, K, N = 37, 512, 96
    X = synth.activations(M, K, 10 + fmt)
    W = synth.random_blocks(fmt, N, K, 20 + fmt)
    Y = oracle.gemm(fmt, X, W, N).astype(np.float64)
    Wd = oracle.dequantize_f64(fmt, W, K, N)
    ref = (X.astype(np.float64) @ Wd.T).astype(np.float16).astype(np.float64)
    diff = np.abs(Y - ref)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert np.all(diff <= ulp)
    assert np.mean(diff == 0) > 0.999


def test_gemm_direct_head_and_residual(oracle):
    M, K, H, D = 20, 256, 4, 64
    N = H * D
    X = synth.activations(M, K, 5)
    W = synth.random_blocks(0, N, K, 6)
    Y = oracle.gemm(0, X, W, N)
    Yh = oracle.gemm(0, X, W, N, head_D=D)
    # [M, N] -> [H, M, D] index map (quant_router_kernels.metal:570-574)
    np.testing.assert_array_equal(Yh, Y.reshape(M, H, D).transpose(1, 0, 2))
    R = synth.activations(M, N, 7)
    Yr = oracle.gemm(0, X, W, N, R=R).astype(np.float64)
    Wd = oracle.dequantize_f64(0, W, K, N)
    ref = (X.astype(np.float64) @ Wd.T + R.astype(np.float64)).astype(np.float16).astype(np.float64)
    assert np.all(np.abs(Yr - ref) <= np.spacing(np.abs(ref).astype(np.float16)))


def test_swiglu_matches_numpy(oracle):
    M, K, N = 9, 256, 64
    X = synth.activations(M, K, 1)
    Wg, Wu = synth.random_blocks(0, N, K, 2), synth.random_blocks(0, N, K, 3)
    out = oracle.swiglu(0, X, Wg, Wu, N).astype(np.float64)
    g = X.astype(np.float64) @ oracle.dequantize_f64(0, Wg, K, N).T
    u = X.astype(np.float64) @ oracle.dequantize_f64(0, Wu, K, N).T
    ref = (g / (1 + np.exp(-g)) * u).astype(np.float16).astype(np.float64)
    assert np.all(np.abs(out - ref) <= np.spacing(np.abs(ref).astype(np.float16)))


# --------------------------------------------------------------------------
# Q8_0 and attention
# --------------------------------------------------------------------------

def test_q8_0_special_cases(oracle):
    # amax = 0 -> d = 0, every code 0 (brick4_attn_bench.mm:48)
    q = oracle.quantize_q8_0(np.zeros(32, np.float16))
    assert np.all(q == 0)
    # x = k * d exactly (d = 1/127 * 127 -> amax 127 gives d = 1): codes are k
    x = np.arange(-16, 16).astype(np.float16) * np.float16(4.0)
    x[0] = -127 * 0.5  # amax 63.5 -> d = 0.5
    q = oracle.quantize_q8_0(x)
    assert q[:2].copy().view(np.float16)[0] == np.float16(0.5)
    codes = q[2:].view(np.int8)
    np.testing.assert_array_equal(codes[1:], (np.arange(-15, 16) * 8).astype(np.int8))
    assert codes[0] == -127


def test_q8_0_bounds_and_rounding_brute_force(oracle):
    """Every code is round-half-away(x / d) with the float d = amax/127, and
    |x - q*d| <= d/2; the largest magnitude maps to +-127."""
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((500, 32)) * 10.0 ** rng.integers(-4, 3, (500, 1))).astype(np.float16)
    q = oracle.quantize_q8_0(x).reshape(500, 34)
    d16 = q[:, :2].copy().view(np.float16)[:, 0]
    codes = q[:, 2:].view(np.int8).astype(np.int64)
    xf = x.astype(np.float32)
    amax = np.abs(xf).max(1)
    d = (amax / np.float32(127)).astype(np.float32)
    np.testing.assert_array_equal(d16, d.astype(np.float16))
    assert np.all(np.abs(codes).max(1) == 127)
    err = np.abs(xf.astype(np.float64) - codes * d[:, None].astype(np.float64))
    assert np.all(err <= d[:, None] * 0.5 * (1 + 1e-5))
    deq = oracle.dequantize_q8_0(q.reshape(-1)).reshape(500, 32)
    np.testing.assert_array_equal(deq, (codes * d16[:, None].astype(np.float32)).astype(np.float16))


def test_attention_special_cases(oracle):
    rng = np.random.default_rng(5)
    H, M, D = 2, 40, 64
    V = rng.standard_normal((H, M, D)).astype(np.float16)
    # uniform scores (Q = 0) -> O[i] = mean(V[0..i])
    O = oracle.attention(np.zeros((H, M, D), np.float16), V, V, 0.125).astype(np.float64)
    csum = np.cumsum(V.astype(np.float64), axis=1) / np.arange(1, M + 1)[None, :, None]
    ref = csum.astype(np.float16).astype(np.float64)
    # double sums in a different order: equal up to one fp16 ulp at rounding boundaries
    assert np.all(np.abs(O - ref) <= np.spacing(np.abs(ref).astype(np.float16)))
    assert np.mean(O == ref) > 0.99
    # row 0 attends only to key 0 -> O[0] = V[0]
    Q = rng.standard_normal((H, M, D)).astype(np.float16)
    O = oracle.attention(Q, Q, V, 0.125)
    np.testing.assert_array_equal(O[:, 0], V[:, 0])


def test_attention_matches_numpy_and_layouts(oracle):
    rng = np.random.default_rng(6)
    H, M, D = 3, 50, 64
    Q, K, V = (rng.standard_normal((H, M, D)).astype(np.float16) for _ in range(3))
    scale = 1.0 / np.sqrt(D)
    O = oracle.attention(Q, K, V, scale).astype(np.float64)
    s = np.einsum("hid,hjd->hij", Q.astype(np.float64), K.astype(np.float64)) * np.float64(np.float32(scale))
    s = np.where(np.tril(np.ones((M, M), bool))[None], s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    ref = np.einsum("hij,hjd->hid", p, V.astype(np.float64)).astype(np.float16).astype(np.float64)
    assert np.all(np.abs(O - ref) <= np.spacing(np.abs(ref).astype(np.float16)))
    Ot = oracle.attention(Q, K, V, scale, o_token_major=True)
    np.testing.assert_array_equal(Ot.reshape(M, H, D).transpose(1, 0, 2), O.astype(np.float16))
    # the Q8_0 variant is attention on the dequantized cache
    Kq, Vq = oracle.quantize_q8_0(K), oracle.quantize_q8_0(V)
    O8 = oracle.attention_q8_0(Q, Kq, Vq, scale)
    Kd = oracle.dequantize_q8_0(Kq).reshape(H, M, D)
    Vd = oracle.dequantize_q8_0(Vq).reshape(H, M, D)
    np.testing.assert_array_equal(O8, oracle.attention(Q, Kd, Vd, scale))


def test_layer_composes_pinned_pieces(oracle):
    rng = np.random.default_rng(7)
    M, dm, H, D, Nm = 24, 128, 2, 64, 256
    X = synth.activations(M, dm, 8)
    Ws = [synth.random_blocks(0, n, k, 30 + i) for i, (n, k) in
          enumerate([(H * D, dm)] * 3 + [(dm, H * D), (Nm, dm), (Nm, dm), (dm, Nm)])]
    out, it = oracle.layer(0, X, *Ws, H=H, D=D, N_mlp=Nm, scale=0.125, intermediates=True)
    q = oracle.gemm(0, X, Ws[0], H * D, head_D=D)
    np.testing.assert_array_equal(it["Q"], q)
    O = oracle.attention_q8_0(it["Q"], oracle.quantize_q8_0(it["K"]), oracle.quantize_q8_0(it["V"]), 0.125,
                              o_token_major=True)
    np.testing.assert_array_equal(it["O"], O)
    np.testing.assert_array_equal(it["Xmid"], oracle.gemm(0, O, Ws[3], dm, R=X))
    np.testing.assert_array_equal(it["S"], oracle.swiglu(0, it["Xmid"], Ws[4], Ws[5], Nm))
    np.testing.assert_array_equal(out, oracle.gemm(0, it["S"], Ws[6], dm, R=it["Xmid"]))
    assert rng is not None


# --------------------------------------------------------------------------
# VAR_RATE_AFFINE, EXL3, PRISM_Q2_0, Q8_0 weights
# --------------------------------------------------------------------------

def _var_closed_form(blk_flat, codes, N, K):
    """Closed form of cpu_gold_reference.h:225-320 from the DRAWN codes (stream
    order j) and the header fields, permutation applied as the gold's dest_idx."""
    b = blk_flat.reshape(N, K // 256, 160)
    d = b[..., 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    bias = b[..., 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    w = np.zeros((N, K // 256, 8, 32))
    for s in range(8):
        S = d * b[..., 4 + s].astype(np.float64) * 0.0625
        B = bias + d * (b[..., 12 + s].astype(np.float64) - 128.0) * 0.0625
        mode = b[..., 20 + s]
        depth, order = mode & 7, (mode >> 3) & 3
        zero = np.where(depth == 3, 4.0, np.where(depth == 5, 16.0, 8.0))
        for j in range(32):
            u = (codes[:, :, s, j].astype(np.float64) - zero) * S + B
            dst = np.where(order == 1, ((j & 1) << 4) | (j >> 1), np.where(order == 2, 31 - j, j))
            np.put_along_axis(w[:, :, s], dst[..., None], u[..., None], axis=-1)
    return w.reshape(N, K)


def test_var_rate_generator_packing_agrees_with_gold_unpacking(oracle):
    """synth restates the reference generator (bench_universal_router.mm:105-158,
    3/5-bit codes as LSB-first streams, 4-bit as nibble pairs); the oracle
    restates the gold's unpacking (cpu_gold_reference.h:233-320).  Every drawn
    code must come back at its permuted position (orders 0, 1, 2)."""
    N, K = 6, 512
    got = {}
    W = synth.var_rate_blocks(N, K, 11, got)
    np.testing.assert_array_equal(oracle.dequantize_f64(4, W, K, N), _var_closed_form(W, got["codes"], N, K))


def test_var_rate_order_probe(oracle):
    """One nonzero code at stream position j lands on element dest(j):
    order 1 interleaves (even j -> j/2, odd j -> 16 + j/2), order 2 reverses."""
    for order in (0, 1, 2, 3):
        for j in (0, 1, 2, 15, 16, 17, 30, 31):
            blk = np.zeros(160, np.uint8)
            blk[0:2] = _f16(16.0)                      # d: S = 16 * 16 / 16 = 16
            blk[4] = 16
            blk[12] = 128                              # B = 0
            blk[20] = (order << 3) | 4                 # sub-block 0: 4-bit
            codes = np.full(32, 8, np.uint8)           # code 8 -> weight 0
            codes[j] = 9                               # -> weight S = 16
            blk[32:48] = synth._pack_nibbles32(codes)
            w = oracle.dequantize_f64(4, blk, 256, 1)[0][:32]
            dest = {1: ((j & 1) << 4) | (j >> 1), 2: 31 - j}.get(order, j)
            exp = np.zeros(32)
            exp[dest] = 16.0
            np.testing.assert_array_equal(w, exp)


def test_var_rate_depth_and_offsets(oracle):
    """Mode depth decides the zero point (4, 8, 16) and the payload width; the
    payload of sub-block s starts at byte 32 + {0,12,24,40,56,72,88,108}[s]."""
    for s in range(8):
        for depth, width, zero in ((3, 12, 4), (4, 16, 8), (5, 20, 16)):
            if synth.VAR_OFFSETS[s] + width > 128:
                continue
            blk = np.zeros(160, np.uint8)
            blk[0:2] = _f16(16.0)
            blk[4 + s] = 16
            blk[12 + s] = 128
            blk[20 + s] = depth
            codes = np.arange(32) % (1 << depth)
            off = 32 + synth.VAR_OFFSETS[s]
            if depth == 4:
                blk[off:off + 16] = synth._pack_nibbles32(codes)
            else:
                blk[off:off + width] = synth._pack_stream(codes.reshape(4, 8), depth).reshape(-1)
            w = oracle.dequantize_f64(4, blk, 256, 1)[0][32 * s:32 * s + 32]
            np.testing.assert_array_equal(w, (codes - zero) * 16.0)


def test_exl3_generator_packing_agrees_with_gold_unpacking(oracle):
    """synth restates the reference generator (bench_universal_router.mm:160-193);
    the oracle the gold (cpu_gold_reference.h:345-392): w = (bias + S cb[q]) +
    R cb[q + 8] for every drawn 3-bit code."""
    N, K = 5, 512
    got = {}
    W = synth.exl3_blocks(N, K, 12, got)
    b = W.reshape(N, K // 256, 144)
    d = b[..., 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    bias = b[..., 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    cb = b[..., 20:36].copy().view(np.int8).astype(np.float64)
    exp = np.zeros((N, K // 256, 8, 32))
    for s in range(8):
        S = d * b[..., 4 + s] * 0.015625
        R = d * (b[..., 12 + s].astype(np.float64) - 128.0) * 0.0078125
        q = got["codes"][:, :, s].astype(np.int64)
        cbb = np.take_along_axis(cb, q, axis=-1)
        cbr = np.take_along_axis(cb, q + 8, axis=-1)
        exp[:, :, s] = bias[..., None] + S[..., None] * cbb + R[..., None] * cbr
    np.testing.assert_array_equal(oracle.dequantize_f64(5, W, K, N), exp.reshape(N, K))
    # the generator's codebook: (c - 3.5) * 8 and (c - 3.5) * 3 truncated toward zero
    np.testing.assert_array_equal(cb[0, 0], [-28, -20, -12, -4, 4, 12, 20, 28, -10, -7, -4, -1, 1, 4, 7, 10])


def test_prism_layout_probe(oracle):
    """Code c at bits 2j of byte i is element 4i + j (cpu_gold_reference.h:
    418-426); the Metal unpacker reads the same element as bits 2(e % 16) of
    little-endian word e / 16 of the sub-block (quant_router_kernels.metal:414-436)."""
    for e in (0, 1, 3, 4, 15, 16, 31, 64, 127):
        for c, val in ((0, -1.0), (2, 1.0), (3, 2.0)):
            blk = np.zeros(34, np.uint8)
            blk[0:2] = _f16(0.5)
            words = np.full(8, 0x55555555, np.uint32)   # every code 1 -> weight 0
            sub, r = divmod(e, 32)
            wi, bit = sub * 2 + r // 16, 2 * (r % 16)
            words[wi] = (words[wi] & ~np.uint32(3 << bit)) | np.uint32(c << bit)
            blk[2:] = words.view(np.uint8)
            w = oracle.dequantize_f64(7, blk, 128, 1)[0]
            exp = np.zeros(128)
            exp[e] = val * 0.5
            np.testing.assert_array_equal(w, exp)


def test_q8_0_weights_match_kv_dequantizer(oracle):
    """The Q8_0 weight decoder equals the Q8_0 KV dequantizer pinned above
    (same 34-byte block, w = q d)."""
    x = (np.random.default_rng(3).standard_normal(64 * 32) * 3).astype(np.float16)
    q = oracle.quantize_q8_0(x)
    np.testing.assert_array_equal(oracle.dequantize(6, q, 64 * 32, 1).reshape(-1).view(np.uint16),
                                  oracle.dequantize_q8_0(q).reshape(-1).view(np.uint16))


# --------------------------------------------------------------------------
# RMSNorm / RoPE / grouped-query attention of the MLX block
# (src/engine/model.py:17-48, :112-116, :215-236)
# --------------------------------------------------------------------------

def test_rmsnorm_closed_forms(oracle):
    # x = (3, 4): mean square 12.5, normed = x / sqrt(12.5 + eps)
    x = np.array([[3.0, 4.0]], np.float16)
    w = np.array([1.0, -2.0], np.float16)
    r = 1.0 / np.sqrt(12.5 + 1e-5)
    expect = np.float16(np.float16(np.array([3.0, 4.0]) * r) * np.array([1.0, -2.0]))
    np.testing.assert_array_equal(oracle.rmsnorm(x, w), expect[None, :])
    # a row of ones returns w (1 / sqrt(1 + 1e-5) rounds to 1 in fp16)
    w = np.random.default_rng(0).standard_normal(64).astype(np.float16)
    np.testing.assert_array_equal(oracle.rmsnorm(np.ones((3, 64), np.float16), w), np.tile(w, (3, 1)))
    # gemma_add_one with w = 0 is the plain normalisation; scale invariance of the normalised row
    x = np.random.default_rng(1).standard_normal((4, 256)).astype(np.float16)
    z = np.zeros(256, np.float16)
    a = oracle.rmsnorm(x, z, eps=0.0, norm_type=2).astype(np.float64)
    b = oracle.rmsnorm((x.astype(np.float64) * 4).astype(np.float16), z, eps=0.0, norm_type=2).astype(np.float64)
    np.testing.assert_array_equal(a, b)  # x * 4 is exact in fp16
    np.testing.assert_allclose((a ** 2).mean(1), 1.0, rtol=2e-3)


def test_rope_closed_forms(oracle):
    # theta = 10000, D = 4, position 1: pair (0, 2) rotates by 1 rad, pair (1, 3) by 0.01 rad
    x = np.zeros((1, 1, 4), np.float16)
    x[0, 0, 0] = 1.0
    x[0, 0, 1] = 1.0
    y = oracle.rope(x, offset=1).astype(np.float64)[0, 0]
    np.testing.assert_array_equal(y, np.float16([np.cos(1.0), np.cos(0.01), np.sin(1.0), np.sin(0.01)]))
    # position 0 is the identity; offset shifts positions
    T = np.random.default_rng(2).standard_normal((3, 5, 64)).astype(np.float16)
    np.testing.assert_array_equal(oracle.rope(T[:, :1]), T[:, :1])
    np.testing.assert_array_equal(oracle.rope(T, offset=7)[:, 1:], oracle.rope(np.concatenate([T[:, :1], T], 1),
                                                                                  offset=6)[:, 2:])
    # rotations keep each pair's norm (to fp16 rounding)
    y = oracle.rope(T, offset=100).astype(np.float64)
    n0 = T.astype(np.float64)[..., :32] ** 2 + T.astype(np.float64)[..., 32:] ** 2
    n1 = y[..., :32] ** 2 + y[..., 32:] ** 2
    np.testing.assert_allclose(n1, n0, rtol=4e-3, atol=1e-3)
    # traditional pairs (2i, 2i+1) == split-half pairs (i, i + D/2) under the interleave permutation
    perm = np.concatenate([np.arange(0, 64, 2), np.arange(1, 64, 2)])
    yt = oracle.rope(T, offset=3, traditional=True)
    ys = oracle.rope(T[..., perm], offset=3, traditional=False)
    np.testing.assert_array_equal(yt[..., perm], ys)


def test_grouped_query_attention_is_repeated_kv(oracle):
    rng = np.random.default_rng(3)
    H, Hkv, M, D = 4, 2, 40, 64
    Q = rng.standard_normal((H, M, D)).astype(np.float16)
    K = rng.standard_normal((Hkv, M, D)).astype(np.float16)
    V = rng.standard_normal((Hkv, M, D)).astype(np.float16)
    a = oracle.attention_gqa(Q, K, V, 0.125)
    b = oracle.attention(Q, np.repeat(K, H // Hkv, axis=0), np.repeat(V, H // Hkv, axis=0), 0.125)
    np.testing.assert_array_equal(a, b)
    a1 = oracle.attention_gqa(Q, K[:1], V[:1], 0.125, o_token_major=True)
    b1 = oracle.attention(Q, np.repeat(K[:1], H, 0), np.repeat(V[:1], H, 0), 0.125, o_token_major=True)
    np.testing.assert_array_equal(a1, b1)


def test_layer_ex_reduces_to_the_router_layer(oracle):
    """No norms, no RoPE and Hkv = H: the MLX-block layer is the router layer."""
    rng = np.random.default_rng(4)
    M, dm, H, D, Nm = 24, 256, 4, 64, 256
    X = (rng.standard_normal((M, dm)) * 0.5).astype(np.float16)
    W = [synth.quantized_weights(0, n, k, 10 + i) for i, (n, k) in
         enumerate([(H * D, dm), (H * D, dm), (H * D, dm), (dm, H * D), (Nm, dm), (Nm, dm), (dm, Nm)])]
    a = oracle.layer(0, X, *W, H, D, Nm, 0.125)
    b = oracle.layer_ex(0, X, None, *W[:4], None, *W[4:], H, H, D, Nm, 0.125, rope=False)
    np.testing.assert_array_equal(a, b)


def test_row_sampled_attention_and_layer_equal_the_full_ones(oracle):
    """attention_q8_0_rows / layer_ex_rows (the checkers of the full-size GPU
    tests) equal rows of the pinned full attention / layer: GQA, RoPE at each
    row's own position, both norms, and the plain router layer."""
    rng = np.random.default_rng(1)
    H, Hkv, M, D = 4, 2, 150, 64
    Q, K, V = (rng.standard_normal((h, M, D)).astype(np.float16) for h in (H, Hkv, Hkv))
    Kq, Vq = oracle.quantize_q8_0(K), oracle.quantize_q8_0(V)
    full = oracle.attention_q8_0_gqa(Q, Kq, Vq, Hkv, 0.125)
    pos = np.array([0, 1, 63, 64, 149, 77])
    r = oracle.attention_q8_0_rows(Q[:, pos], Kq, Vq, pos, M, Hkv, 0.125)
    np.testing.assert_array_equal(r, full[:, pos])
    rt = oracle.attention_q8_0_rows(Q[:, pos], Kq, Vq, pos, M, Hkv, 0.125, o_token_major=True)
    np.testing.assert_array_equal(rt.reshape(pos.size, H, D).transpose(1, 0, 2), r)
    M, dm, Hq, Hkv, D, Nm = 96, 128, 4, 2, 32, 256
    X = synth.activations(M, dm, 3)
    shapes = [(Hq * D, dm), (Hkv * D, dm), (Hkv * D, dm), (dm, Hq * D), (Nm, dm), (Nm, dm), (dm, Nm)]
    Ws = [synth.quantized_weights(0, n, k, 10 + i) for i, (n, k) in enumerate(shapes)]
    na = (1 + 0.1 * rng.standard_normal(dm)).astype(np.float16)
    nf = (1 + 0.1 * rng.standard_normal(dm)).astype(np.float16)
    pos = np.array([0, 5, 31, 95, 40])
    for norms, rope in (((na, nf), True), ((None, None), False)):
        full = oracle.layer_ex(0, X, norms[0], *Ws[:4], norms[1], *Ws[4:], Hq=Hq, Hkv=Hkv, D=D, N_mlp=Nm,
                               scale=0.17, rope=rope, theta=500000.0, offset=5)
        r = oracle.layer_ex_rows(0, X, norms[0], *Ws[:4], norms[1], *Ws[4:], pos, Hq=Hq, Hkv=Hkv, D=D, N_mlp=Nm,
                                 scale=0.17, rope=rope, theta=500000.0, offset=5)
        np.testing.assert_array_equal(r, full[pos])
    Wl = [synth.quantized_weights(0, n, k, 30 + i) for i, (n, k) in
          enumerate([(Hq * D, dm)] * 3 + [(dm, Hq * D), (Nm, dm), (Nm, dm), (dm, Nm)])]
    full = oracle.layer(0, X, *Wl, H=Hq, D=D, N_mlp=Nm, scale=0.17)
    r = oracle.layer_ex_rows(0, X, None, *Wl[:4], None, *Wl[4:], pos, Hq=Hq, Hkv=Hq, D=D, N_mlp=Nm, scale=0.17)
    np.testing.assert_array_equal(r, full[pos])


def test_mlx_g64_block_known_answers(oracle):
    """MLX_4BIT_G64 blocks: element 8j + i is nibble i of code word j and
    w = scale * q + bias (mlx.core.dequantize); a layout probe with one
    nonzero nibble at a time catches swapped words or nibble order, and the
    block's decode equals the MLX_4BIT decode of the g64 -> router repack."""
    blk = np.zeros(36, np.uint8)
    blk[0:2] = np.array([0.25], np.float16).view(np.uint8)
    blk[2:4] = np.array([-1.0], np.float16).view(np.uint8)
    for j in range(8):
        for i in range(8):
            b = blk.copy()
            words = np.zeros(8, np.uint32)
            words[j] = np.uint32(15) << np.uint32(4 * i)
            b[4:] = words.view(np.uint8)
            w = oracle.dequantize_f64(8, b, 64, 1)[0]
            expect = np.full(64, -1.0)
            expect[8 * j + i] = 15 * 0.25 - 1.0
            np.testing.assert_array_equal(w, expect)
    scale, bias, packed = synth.quantize_mlx_g64(synth.gaussian_weights(8, 256, 9))
    np.testing.assert_array_equal(oracle.dequantize_f64(8, synth.mlx_g64_blocks(scale, bias, packed), 256, 8),
                                  oracle.dequantize_f64(1, synth.mlx_g64_to_router_blocks(scale, bias, packed), 256, 8))
