"""The prefill model (model.py) mirroring src/engine/config.py and
src/engine/model.py: configuration checks and the embedding bounds on the CPU;
on the GPU a small model checked block by block against the oracle's block
(each fed the GPU's previous hidden state, so every step is held to the block
bound on its own), then the final norm and the LM head, and the model's one
call equal to that chain bit for bit.

The block bound is relative to each row's magnitude: both sides quantize K and
V to Q8_0, and a one-step fp16 difference upstream (fp32 vs double sums, an
RMSNorm near-tie) that moves a block's absmax shifts its codes, so an output
row can differ by about one Q8_0 step (1/127 of its scale) where the fp16
values themselves agree to a step.  The weights use scale 0.01: at the
reference's default (0.5 / sqrt(hidden) with uniform codes) the attention
scores reach ~40 and the softmax is an argmax, which such a step can flip."""
from __future__ import annotations

import numpy as np
import pytest

import model
import tolerance
from m4_bridge import QuantFormat
from tolerance import TOL


def test_engine_config_checks():
    c = model.EngineConfig()
    assert (c.q_dim, c.kv_dim, c.weight_format) == (512, 128, QuantFormat.QUANT_Q4_0)
    assert c.scale == pytest.approx(0.125)
    assert model.EngineConfig(weight_format="q4_k").weight_format == QuantFormat.QUANT_Q4_K
    assert model.EngineConfig(norm_type=" RMSNorm ").norm_type == "rmsnorm"
    bad = [dict(num_layers=0), dict(num_q_heads=6, num_kv_heads=4), dict(norm_eps=0.0), dict(rope_theta=-1.0),
           dict(backend="cuda"), dict(backend="mlx"), dict(kv_mode="out_of_core"), dict(kv_mode="disk"),
           dict(activation="geglu"), dict(activation="relu"), dict(norm_type="layernorm"), dict(head_dim=96),
           dict(max_context_length=0)]
    for kw in bad:
        with pytest.raises(ValueError):
            model.EngineConfig(**kw)
    with pytest.raises(ValueError):
        model.EngineConfig(weight_format="q5_0")


def test_embedding_bounds_and_gather():
    import torch

    e = model.Embedding(16, 8)
    e.weight = torch.arange(128, dtype=torch.float16).reshape(16, 8).to(e.weight.device)
    out = e(torch.tensor([3, 0, 15]))
    assert out.shape == (3, 8) and out[0, 0].item() == 24 and out[2, 7].item() == 127
    for bad in ([16], [-1], [2, 99]):
        with pytest.raises(IndexError):
            e(torch.tensor(bad))


def _host(t):
    return t.detach().cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("fmt,norm_type,Hq,Hkv,D", [(0, "rmsnorm", 4, 2, 64), (2, "gemma_add_one", 4, 2, 64),
                                                    (0, "rmsnorm", 2, 1, 128)])
def test_model_prefill_block_by_block(bridge, oracle, fmt, norm_type, Hq, Hkv, D):
    import torch

    cfg = model.EngineConfig(num_layers=2, hidden_dim=256, num_q_heads=Hq, num_kv_heads=Hkv, head_dim=D,
                             intermediate_dim=512, vocab_size=512, weight_format=fmt, norm_type=norm_type,
                             rope_theta=10000.0)
    m = model.TransformerModel(cfg)
    m.init_synthetic_weights(seed=11, scale=0.01)
    if norm_type == "gemma_add_one":  # non-trivial norm weights on both paths
        for layer in m.layers:
            for nrm in (layer.input_norm, layer.post_attention_norm):
                nrm.weight = (0.1 * torch.randn(cfg.hidden_dim, generator=torch.Generator().manual_seed(3))).to(
                    torch.float16).cuda()
    tokens = np.random.default_rng(12).integers(0, cfg.vocab_size, 80)
    logits = m(tokens)
    assert logits.shape == (80, cfg.vocab_size)
    for layer in m.layers:
        Kq, Vq = layer.kv_q8
        assert Kq.shape == (Hkv, 80, D // 32 * 34) and Vq.shape == (Hkv, 80, D // 32 * 34)

    nt = model._NORM_TYPES[norm_type]
    h = m.embedding(torch.as_tensor(tokens))
    np.testing.assert_array_equal(_host(h), _host(m.embedding.weight)[tokens])
    for i, layer in enumerate(m.layers):
        print(f"model block {i} fmt {fmt} D {D}", flush=True)
        x = _host(h)
        h = layer(h)
        ws = [_host(w.weight) for w in (layer.wq, layer.wk, layer.wv, layer.wo, layer.w_gate, layer.w_up,
                                        layer.w_down)]
        ref = oracle.layer_ex(fmt, x, _host(layer.input_norm.weight), *ws[:4], _host(layer.post_attention_norm.weight),
                              *ws[4:], cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim, cfg.intermediate_dim,
                              cfg.scale, norm_type=nt, eps=cfg.norm_eps, rope=True, theta=cfg.rope_theta, offset=0,
                              traditional=cfg.rope_traditional)
        bridge.synchronize()
        ref = ref.astype(np.float64)
        diff = np.abs(_host(h).astype(np.float64) - ref)
        row_scale = np.maximum(1.0, np.abs(ref).max(axis=1, keepdims=True))
        print(f"  block {i} max|diff| = {diff.max()}, max|ref| = {np.abs(ref).max()}")
        assert np.all(diff <= 2 * TOL * row_scale)  # two Q8_0 steps of the row's scale
    xn = _host(h)
    hn = m.norm(h)
    bridge.synchronize()
    # the norm bound of test_rmsnorm: r in fp32 here, in double in the oracle, so x r near an fp16 tie
    # may land one step away and the product with w carries it into at most two output steps
    refn = oracle.rmsnorm(xn, _host(m.norm.weight), cfg.norm_eps, nt).astype(np.float64)
    step = np.spacing(np.abs(refn).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(_host(hn).astype(np.float64) - refn) <= 2 * step)
    lg = m.lm_head(hn)
    bridge.synchronize()
    tolerance.check_ref(_host(lg), oracle.gemm(fmt, _host(hn), _host(m.lm_head.weight), cfg.vocab_size),
                        what="lm head")
    # the model's one call is that chain
    np.testing.assert_array_equal(_host(lg).view(np.uint16), _host(logits).view(np.uint16))


@pytest.mark.gpu
def test_model_batch_of_one_and_no_cache(bridge):
    cfg = model.EngineConfig(num_layers=1, hidden_dim=256, num_q_heads=4, num_kv_heads=4, head_dim=64,
                             intermediate_dim=256, vocab_size=256)
    m = model.TransformerModel(cfg)
    m.init_synthetic_weights(seed=5)
    # the reference's seeds and draw order (src/engine/model.py:307-334)
    emb = (np.random.RandomState(5).randn(256, 256) * 0.02).astype(np.float16)
    np.testing.assert_array_equal(_host(m.embedding.weight), emb)
    scale = 0.5 / np.sqrt(256)
    import modules
    np.testing.assert_array_equal(
        _host(m.lm_head.weight),
        _host(modules.generate_synthetic_quantized_weights(0, 256, 256, scale=scale, seed=5 + 9999)))
    np.testing.assert_array_equal(
        _host(m.layers[0].w_up.weight),
        _host(modules.generate_synthetic_quantized_weights(0, 256, 256, scale=scale, seed=5 + 100 + 5 * 7)))
    a = m([[1, 2, 3, 4, 5]], use_cache=False)
    assert a.shape == (1, 5, 256) and m.layers[0].kv_q8 is None
    b = m([1, 2, 3, 4, 5])
    assert m.layers[0].kv_q8 is not None
    np.testing.assert_array_equal(_host(a[0]).view(np.uint16), _host(b).view(np.uint16))
    m.reset()
    assert m.layers[0].kv_q8 is None
    with pytest.raises(ValueError):
        m([1, 2], mask="none-causal")
    with pytest.raises(IndexError):
        m([300])
