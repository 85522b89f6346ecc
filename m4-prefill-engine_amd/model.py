"""Prefill model over the HIP bridge -- the caller of the block entry point,
with the reference's model names and configuration (src/engine/config.py
EngineConfig :13-95; src/engine/model.py RMSNorm :17-46, Embedding :48-63,
TransformerBlock :66-270, TransformerModel :273-368).

A block is one call of m4_bridge_prefill_layer_ex_kv: RMSNorm -> Q/K/V head
projections -> RoPE -> Q8_0 K/V -> grouped-query causal attention over that
Q8_0 cache -> O projection + residual -> RMSNorm -> fused SwiGLU -> down
projection + residual, all on the GPU with no host round trip between the
steps.  Where this differs from the reference's MLX model:

* attention reads the Q8_0 KV cache the block writes, as the reference's
  unified prefill engine does (unified_prefill_engine.mm:548-572), instead of
  the MLX model's fp16 scaled-dot-product attention;
* a call is the prefill of one fresh sequence (RoPE positions start at
  `rope_offset`, 0 by default).  Each block keeps the Q8_0 K / V it wrote
  (`kv_q8`) for a decoder to continue from; the MLX KV-cache object, decoding
  and the out-of-core cache modes are not part of this path;
* backend "m4" and activation "swiglu" only (the block's fused SwiGLU); the
  other values the reference accepts raise ValueError here.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional, Union

import numpy as np

from m4_bridge import HIPBridge, QuantFormat, m4_bridge_init, m4_bridge_synchronize
from modules import M4QuantizedLinear, normalize_format

_NORM_TYPES = {"rmsnorm": 1, "gemma_add_one": 2}


@dataclass
class EngineConfig:
    """Model shape and execution settings (src/engine/config.py:13-95): the
    same fields, defaults and validation, restricted to what the native block
    runs."""

    num_layers: int = 4
    hidden_dim: int = 512
    num_q_heads: int = 8
    num_kv_heads: int = 2
    head_dim: int = 64
    intermediate_dim: int = 1024
    vocab_size: int = 1024
    rope_theta: float = 10000.0
    activation: str = "swiglu"
    norm_type: str = "rmsnorm"
    backend: str = "m4"
    kv_mode: str = "in_ram"
    weight_format: Union[int, QuantFormat, str] = 0
    max_context_length: int = 2048
    norm_eps: float = 1e-5
    rope_traditional: bool = False

    def __post_init__(self) -> None:
        for name in ("num_layers", "hidden_dim", "num_q_heads", "num_kv_heads", "head_dim", "intermediate_dim",
                     "vocab_size"):
            if getattr(self, name) <= 0:
                raise ValueError(f"{name} must be > 0, got {getattr(self, name)}")
        if self.num_q_heads % self.num_kv_heads != 0:
            raise ValueError(f"num_q_heads ({self.num_q_heads}) must be divisible by num_kv_heads "
                             f"({self.num_kv_heads}) for GQA/MHA")
        if self.max_context_length <= 0:
            raise ValueError(f"max_context_length must be positive, got {self.max_context_length}")
        if self.norm_eps <= 0:
            raise ValueError(f"norm_eps must be positive, got {self.norm_eps}")
        if self.rope_theta <= 0:
            raise ValueError(f"rope_theta must be positive, got {self.rope_theta}")
        self.backend = self.backend.lower().strip()
        if self.backend not in ("m4", "mlx"):
            raise ValueError(f"Unsupported backend '{self.backend}'. Must be 'm4' or 'mlx'.")
        if self.backend != "m4":
            raise ValueError("backend 'mlx' (stock MLX layers) has no counterpart here; use 'm4'")
        self.kv_mode = self.kv_mode.lower().strip()
        if self.kv_mode not in ("in_ram", "out_of_core"):
            raise ValueError(f"Unsupported kv_mode '{self.kv_mode}'. Must be 'in_ram' or 'out_of_core'.")
        if self.kv_mode != "in_ram":
            raise ValueError("kv_mode 'out_of_core' is not part of the prefill path; use 'in_ram'")
        self.activation = self.activation.lower().strip()
        if self.activation not in ("swiglu", "geglu"):
            raise ValueError(f"Unsupported activation '{self.activation}'. Must be 'swiglu' or 'geglu'.")
        if self.activation != "swiglu":
            raise ValueError("activation 'geglu' is not supported by the native block (fused SwiGLU)")
        self.norm_type = self.norm_type.lower().strip()
        if self.norm_type not in _NORM_TYPES:
            raise ValueError(f"Unsupported norm_type '{self.norm_type}'. Must be 'rmsnorm' or 'gemma_add_one'.")
        if self.head_dim not in (64, 128):
            raise ValueError(f"head_dim must be 64 or 128 for the attention kernels, got {self.head_dim}")
        self.weight_format = normalize_format(self.weight_format)

    @property
    def scale(self) -> float:
        """Attention scaling factor: 1.0 / sqrt(head_dim)."""
        return 1.0 / math.sqrt(self.head_dim)

    @property
    def q_dim(self) -> int:
        return self.num_q_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.num_kv_heads * self.head_dim


def _bridge() -> HIPBridge:
    b = HIPBridge.get_instance()
    if not b.is_initialized():
        m4_bridge_init()
    return b


def _device() -> str:
    import torch

    return "cuda" if torch.cuda.is_available() else "cpu"


class RMSNorm:
    """RMSNorm / Gemma-style 'gemma_add_one' norm (src/engine/model.py:17-46)
    on the bridge's kernel: fp16(fp16(x / sqrt(mean(x^2) + eps)) * w), with
    (1 + w) for gemma_add_one.  Rows of a [..., dims] fp16 tensor."""

    def __init__(self, dims: int, eps: float = 1e-5, norm_type: str = "rmsnorm") -> None:
        import torch

        self.dims = int(dims)
        self.eps = float(eps)
        self.norm_type = norm_type.lower().strip()
        if self.norm_type not in _NORM_TYPES:
            raise ValueError(f"Unsupported norm_type '{norm_type}'")
        self.weight = torch.empty(self.dims, dtype=torch.float16, device=_device())
        self.init_synthetic_weights()

    def init_synthetic_weights(self) -> None:
        self.weight.fill_(0.0 if self.norm_type == "gemma_add_one" else 1.0)

    def __call__(self, x):
        import torch

        if x.shape[-1] != self.dims:
            raise ValueError(f"last dimension {x.shape[-1]} does not match dims {self.dims}")
        x2 = x.to(torch.float16).contiguous().reshape(-1, self.dims)
        y = torch.empty_like(x2)
        _bridge().rmsnorm(x2, self.weight, y, eps=self.eps, norm_type=_NORM_TYPES[self.norm_type])
        return y.reshape(x.shape)


class Embedding:
    """Token-id gather (src/engine/model.py:48-63), IndexError for ids outside
    [0, vocab_size)."""

    def __init__(self, vocab_size: int, hidden_dim: int) -> None:
        import torch

        self.vocab_size = int(vocab_size)
        self.hidden_dim = int(hidden_dim)
        self.weight = torch.zeros((self.vocab_size, self.hidden_dim), dtype=torch.float16, device=_device())

    def __call__(self, tokens):
        import torch

        t = torch.as_tensor(tokens, dtype=torch.long)
        if t.numel() and (int(t.min()) < 0 or int(t.max()) >= self.vocab_size):
            raise IndexError(f"Token ID out of vocabulary bounds [0, {self.vocab_size})")
        return self.weight[t.to(self.weight.device)]


class TransformerBlock:
    """One transformer block (src/engine/model.py:66-270) as one call of the
    native block entry point.  Accepts [M, hidden] or [1, M, hidden] fp16."""

    def __init__(self, config: EngineConfig) -> None:
        c = config
        self.config = c
        self.scale = c.scale
        fmt = c.weight_format
        self.input_norm = RMSNorm(c.hidden_dim, c.norm_eps, c.norm_type)
        self.wq = M4QuantizedLinear(c.hidden_dim, c.q_dim, format=fmt)
        self.wk = M4QuantizedLinear(c.hidden_dim, c.kv_dim, format=fmt)
        self.wv = M4QuantizedLinear(c.hidden_dim, c.kv_dim, format=fmt)
        self.wo = M4QuantizedLinear(c.q_dim, c.hidden_dim, format=fmt)
        self.post_attention_norm = RMSNorm(c.hidden_dim, c.norm_eps, c.norm_type)
        self.w_gate = M4QuantizedLinear(c.hidden_dim, c.intermediate_dim, format=fmt)
        self.w_up = M4QuantizedLinear(c.hidden_dim, c.intermediate_dim, format=fmt)
        self.w_down = M4QuantizedLinear(c.intermediate_dim, c.hidden_dim, format=fmt)
        self.kv_q8 = None  # (Kq, Vq) uint8 [num_kv_heads, M, head_dim / 32 * 34] of the last call

    def reset(self) -> None:
        """Drops the Q8_0 K / V kept from the last call."""
        self.kv_q8 = None

    def init_synthetic_weights(self, scale: Optional[float] = None, seed: Optional[int] = None,
                               unit_weights: bool = False) -> None:
        """Deterministic weights with the reference's seeds (src/engine/model.py:158-179)."""
        base_seed = seed if seed is not None else 42
        actual_scale = scale if scale is not None else (0.5 / math.sqrt(self.config.hidden_dim))
        self.input_norm.init_synthetic_weights()
        self.post_attention_norm.init_synthetic_weights()
        for idx, layer in enumerate([self.wq, self.wk, self.wv, self.wo, self.w_gate, self.w_up, self.w_down]):
            layer.init_synthetic_weights(scale=actual_scale, unit_weights=unit_weights, seed=base_seed + idx * 7)

    def __call__(self, x, rope_offset: int = 0, keep_kv: bool = True):
        import torch

        c = self.config
        is_3d = x.dim() == 3
        if is_3d:
            if x.shape[0] != 1:
                raise ValueError("one sequence per call (batch 1)")
            x = x[0]
        if x.dim() != 2 or x.shape[1] != c.hidden_dim:
            raise ValueError(f"expected [M, {c.hidden_dim}] activations, got {tuple(x.shape)}")
        x = x.to(torch.float16).contiguous()
        M = x.shape[0]
        out = torch.empty_like(x)
        kv_bytes = c.num_kv_heads * M * (c.head_dim // 32) * 34
        Kq = torch.empty(kv_bytes, dtype=torch.uint8, device=x.device)
        Vq = torch.empty(kv_bytes, dtype=torch.uint8, device=x.device)
        _bridge().prefill_layer_ex_kv(
            x, self.input_norm.weight, self.wq.weight, self.wk.weight, self.wv.weight, self.wo.weight,
            self.post_attention_norm.weight, self.w_gate.weight, self.w_up.weight, self.w_down.weight, out, Kq, Vq,
            int(c.weight_format), M, c.hidden_dim, c.num_q_heads, c.num_kv_heads, c.head_dim, c.intermediate_dim,
            self.scale, norm_type=_NORM_TYPES[c.norm_type], norm_eps=c.norm_eps, rope=True,
            rope_theta=c.rope_theta, rope_offset=int(rope_offset), rope_traditional=c.rope_traditional)
        if keep_kv:
            shape = (c.num_kv_heads, M, (c.head_dim // 32) * 34)
            self.kv_q8 = (Kq.view(shape), Vq.view(shape))
        return out[None] if is_3d else out


class TransformerModel:
    """Embedding -> blocks -> final norm -> LM head (src/engine/model.py:273-368),
    prefill of one sequence: tokens [M] (or [1, M]) -> logits [M, vocab_size]."""

    def __init__(self, config: EngineConfig) -> None:
        c = config
        self.config = c
        self.embedding = Embedding(c.vocab_size, c.hidden_dim)
        self.layers: List[TransformerBlock] = [TransformerBlock(c) for _ in range(c.num_layers)]
        self.norm = RMSNorm(c.hidden_dim, c.norm_eps, c.norm_type)
        self.lm_head = M4QuantizedLinear(c.hidden_dim, c.vocab_size, format=c.weight_format)

    def reset(self) -> None:
        for layer in self.layers:
            layer.reset()

    def init_synthetic_weights(self, scale: Optional[float] = None, seed: Optional[int] = 42,
                               unit_weights: bool = False) -> None:
        """Deterministic weights with the reference's seeds and draw order
        (src/engine/model.py:307-334): embedding N(0, 0.02) from numpy's
        RandomState(seed), block i from seed + 100 (i + 1), LM head seed + 9999."""
        import torch

        base_seed = seed if seed is not None else 42
        actual_scale = scale if scale is not None else (0.5 / math.sqrt(self.config.hidden_dim))
        rng = np.random.RandomState(base_seed)
        emb = (rng.randn(self.config.vocab_size, self.config.hidden_dim) * 0.02).astype(np.float16)
        self.embedding.weight = torch.from_numpy(emb).to(self.embedding.weight.device)
        for i, layer in enumerate(self.layers):
            layer.init_synthetic_weights(scale=actual_scale, seed=base_seed + (i + 1) * 100, unit_weights=unit_weights)
        self.norm.init_synthetic_weights()
        self.lm_head.init_synthetic_weights(scale=actual_scale, seed=base_seed + 9999, unit_weights=unit_weights)

    def __call__(self, tokens, mask: Optional[str] = None, use_cache: bool = True, rope_offset: int = 0):
        import torch

        if mask not in (None, "causal"):
            raise ValueError("only the causal mask of a prefill is supported")
        t = torch.as_tensor(tokens, dtype=torch.long)
        is_1d = t.dim() == 1
        if not is_1d:
            if t.dim() != 2 or t.shape[0] != 1:
                raise ValueError("tokens must be [M] or [1, M]")
            t = t[0]
        h = self.embedding(t)
        for layer in self.layers:
            h = layer(h, rope_offset=rope_offset, keep_kv=use_cache)
        h = self.norm(h)
        logits = self.lm_head(h)
        m4_bridge_synchronize()
        return logits if is_1d else logits[None]
