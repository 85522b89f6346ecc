"""Quantized linear layer over the HIP bridge -- the Python caller of the
projection entry points, with the reference's names and behaviour
(src/engine/modules.py: FORMAT_SPECS :33-82, normalize_format :85-99,
compute_quantized_weight_bytes :101-112, generate_synthetic_quantized_weights
:115-199, M4QuantizedLinear :290-426).

Tensors are torch tensors on the GPU instead of MLX unified-memory arrays: the
weight is a flat uint8 tensor of packed blocks, activations and outputs fp16.
The forward pass dispatches GEMV for a single row and GEMM otherwise, over any
leading batch dimensions, and the optional finite check is deferred to the
bridge's synchronize as in the reference.  The stock-MLX baseline layer and
the fp16 dequantization helper of the reference module are not part of the
projection path and have no counterpart here.
"""
from __future__ import annotations

from typing import Optional, Union

import numpy as np

from m4_bridge import (
    HIPBridge,
    QuantFormat,
    m4_bridge_dispatch_gemm,
    m4_bridge_dispatch_gemv,
    m4_bridge_init,
    m4_bridge_synchronize,
)

# Format specification table (block size, bytes per block, bits per weight),
# the reference's six dispatchable formats (src/engine/modules.py:33-82).
FORMAT_SPECS = {
    QuantFormat.QUANT_Q4_0: {"name": "QUANT_Q4_0", "block_size": 32, "struct_size": 18, "bits_per_weight": 4.5,
                             "is_super_block": False},
    QuantFormat.QUANT_MLX_4BIT: {"name": "QUANT_MLX_4BIT", "block_size": 32, "struct_size": 20,
                                 "bits_per_weight": 5.0, "is_super_block": False},
    QuantFormat.QUANT_Q4_K: {"name": "QUANT_Q4_K", "block_size": 256, "struct_size": 144, "bits_per_weight": 4.5,
                             "is_super_block": True},
    QuantFormat.QUANT_TERNARY_1_58: {"name": "QUANT_TERNARY_1_58", "block_size": 32, "struct_size": 12,
                                     "bits_per_weight": 3.0, "is_super_block": False},
    QuantFormat.QUANT_VAR_RATE_AFFINE: {"name": "QUANT_VAR_RATE_AFFINE", "block_size": 256, "struct_size": 160,
                                        "bits_per_weight": 5.0, "is_super_block": True},
    QuantFormat.QUANT_EXL3: {"name": "QUANT_EXL3", "block_size": 256, "struct_size": 144, "bits_per_weight": 4.5,
                             "is_super_block": True},
}


def normalize_format(format_val: Union[int, QuantFormat, str]) -> QuantFormat:
    """int, QuantFormat or name ("q4_0", "QUANT_Q4_0", ...) -> QuantFormat
    (src/engine/modules.py:85-99): ValueError for an unknown name, TypeError
    for any other type."""
    if isinstance(format_val, QuantFormat):
        return format_val
    if isinstance(format_val, int):
        return QuantFormat(format_val)
    if isinstance(format_val, str):
        name = format_val.upper().strip()
        if not name.startswith("QUANT_"):
            name = f"QUANT_{name}"
        for qf in QuantFormat:
            if qf.name == name:
                return qf
        raise ValueError(f"Unknown quantization format string: '{format_val}'")
    raise TypeError(f"Invalid format type: {type(format_val)}")


def compute_quantized_weight_bytes(format_val: Union[int, QuantFormat, str], in_features: int,
                                   out_features: int) -> int:
    """Bytes of the packed [out_features, in_features] weight (src/engine/modules.py:101-112)."""
    if in_features <= 0 or out_features <= 0:
        raise ValueError(
            f"in_features ({in_features}) and out_features ({out_features}) must be positive integers > 0")
    fmt = normalize_format(format_val)
    spec = FORMAT_SPECS[fmt]
    if in_features % spec["block_size"] != 0:
        raise ValueError(f"in_features ({in_features}) must be divisible by {spec['block_size']} for {fmt.name}")
    return (in_features // spec["block_size"]) * out_features * spec["struct_size"]


def _f16_bytes(v) -> np.ndarray:
    return np.frombuffer(np.float16(v).tobytes(), dtype=np.uint8)


def generate_synthetic_quantized_weights(format_val: Union[int, QuantFormat, str], in_features: int,
                                         out_features: int, scale: float = 1.0, unit_weights: bool = False,
                                         seed: Optional[int] = None, device: Optional[str] = None):
    """Deterministic packed weights (src/engine/modules.py:115-199), as a flat
    uint8 torch tensor on `device` (the GPU when one is present).  Unit
    weights (or no seed) give every weight the value `scale` (Q4_K: scale / 32
    per unit code); otherwise the blocks are drawn from numpy's RandomState
    with the reference's draw order, so a seed gives the reference's bytes."""
    import torch

    fmt = normalize_format(format_val)
    spec = FORMAT_SPECS[fmt]
    bs, ss = spec["block_size"], spec["struct_size"]
    nblocks = (in_features // bs) * out_features
    raw = np.zeros(nblocks * ss, dtype=np.uint8)
    rng = np.random.RandomState(seed) if seed is not None else None
    unit = unit_weights or rng is None
    s16 = np.float16(scale)

    if fmt == QuantFormat.QUANT_Q4_0:
        for b in range(nblocks):
            s = s16 if unit else np.float16(scale * rng.uniform(0.5, 1.5))
            raw[b * 18:b * 18 + 2] = _f16_bytes(s)
            raw[b * 18 + 2:b * 18 + 18] = 0x99 if unit else rng.randint(0, 256, size=16, dtype=np.uint8)  # code 9 -> +1
    elif fmt == QuantFormat.QUANT_MLX_4BIT:
        for b in range(nblocks):
            s = s16 if unit else np.float16(scale * rng.uniform(0.5, 1.5))
            bias = np.float16(0.0) if unit else np.float16(scale * rng.uniform(-0.1, 0.1))
            raw[b * 20:b * 20 + 2] = _f16_bytes(s)
            raw[b * 20 + 2:b * 20 + 4] = _f16_bytes(bias)
            raw[b * 20 + 4:b * 20 + 20] = 0x11 if unit else rng.randint(0, 256, size=16, dtype=np.uint8)  # code 1
    elif fmt == QuantFormat.QUANT_TERNARY_1_58:
        for b in range(nblocks):
            s = s16 if unit else np.float16(scale * rng.uniform(0.5, 1.5))
            raw[b * 12:b * 12 + 2] = _f16_bytes(s)
            word = np.uint32(0xAAAAAAAA) if unit else np.uint32(rng.randint(0, 0xFFFFFFFF))  # code 2 -> +1
            raw[b * 12 + 4:b * 12 + 8] = np.frombuffer(word.tobytes(), dtype=np.uint8)
            raw[b * 12 + 8:b * 12 + 12] = np.frombuffer(word.tobytes(), dtype=np.uint8)
    elif fmt == QuantFormat.QUANT_Q4_K:
        eff = scale / 32.0
        for b in range(nblocks):
            o = b * 144
            d = np.float16(eff) if unit else np.float16(eff * rng.uniform(0.5, 1.5))
            dmin = np.float16(0.0) if unit else np.float16(eff * rng.uniform(0.0001, 0.001))
            raw[o:o + 2] = _f16_bytes(d)
            raw[o + 2:o + 4] = _f16_bytes(dmin)
            if unit:  # sc = 1, min = 0 for every sub-block, codes 1
                raw[o + 4:o + 8] = 1
                raw[o + 8:o + 12] = 1
                raw[o + 12:o + 16] = 0
                raw[o + 16:o + 144] = 0x11
            else:
                sc = rng.randint(1, 64, size=8, dtype=np.uint8)
                mn = rng.randint(0, 64, size=8, dtype=np.uint8)
                packed = np.zeros(12, dtype=np.uint8)
                for j in range(4):
                    packed[j] = (sc[j] & 0x3F) | ((mn[j] >> 4) << 6)
                    packed[j + 4] = (sc[j + 4] & 0x3F) | ((mn[j + 4] >> 4) << 6)
                    packed[j + 8] = (mn[j] & 0x0F) | ((mn[j + 4] & 0x0F) << 4)
                raw[o + 4:o + 16] = packed
                raw[o + 16:o + 144] = rng.randint(0, 256, size=128, dtype=np.uint8)
    else:  # VAR_RATE_AFFINE / EXL3: a valid fp16 scale in every header, zero codes
        for b in range(nblocks):
            s = s16 if unit else np.float16(scale * rng.uniform(0.5, 1.5))
            raw[b * ss:b * ss + 2] = _f16_bytes(s)

    if device is None:
        device = "cuda" if torch.cuda.is_available() else "cpu"
    return torch.from_numpy(raw).to(device)


def _torch_module_base():
    import torch

    return torch.nn.Module


class M4QuantizedLinear(_torch_module_base()):
    """Quantized linear layer on the HIP kernels (src/engine/modules.py:290-426):
    y = x . W^T with W the packed [out_features, in_features] blocks.  GEMV
    for one row (a 1-D input or one row over the leading dimensions), GEMM
    otherwise; any leading batch dimensions; fp16 in and out."""

    def __init__(self, in_features: int, out_features: int,
                 format: Union[int, QuantFormat, str] = QuantFormat.QUANT_Q4_0, weight=None) -> None:
        super().__init__()
        import torch

        self.in_features = int(in_features)
        self.out_features = int(out_features)
        self.format = normalize_format(format)
        self.spec = FORMAT_SPECS[self.format]  # KeyError for formats the layer does not take, as in the reference
        if self.in_features <= 0 or self.out_features <= 0:
            raise ValueError(f"in_features ({self.in_features}) and out_features ({self.out_features}) must be "
                             f"positive integers > 0")
        bs = self.spec["block_size"]
        if self.in_features % bs != 0:
            raise ValueError(f"in_features={self.in_features} must be divisible by {bs} for format {self.format.name}")
        if self.spec["is_super_block"] and self.in_features % 256 != 0:
            raise ValueError(
                f"Super-block format {self.format.name} requires in_features ({self.in_features}) % 256 == 0")
        expected = compute_quantized_weight_bytes(self.format, self.in_features, self.out_features)
        device = "cuda" if torch.cuda.is_available() else "cpu"
        if weight is None:
            w = torch.zeros(expected, dtype=torch.uint8, device=device)
        else:
            w = weight if isinstance(weight, torch.Tensor) else torch.from_numpy(np.array(weight, copy=True))
            w = w.reshape(-1).view(torch.uint8) if w.dtype != torch.uint8 else w.reshape(-1)
            nbytes = w.numel() * w.element_size()
            if nbytes != expected:
                raise ValueError(f"Weight buffer size mismatch for {self.format.name}: expected {expected} bytes, "
                                 f"got {nbytes} bytes")
            w = w.to(device)
        self.register_buffer("weight", w.contiguous(), persistent=True)
        if not HIPBridge.get_instance().is_initialized():
            m4_bridge_init()

    @classmethod
    def from_quantized(cls, weights, format: Union[int, QuantFormat, str], in_features: int,
                       out_features: int) -> "M4QuantizedLinear":
        """Layer over pre-quantized packed blocks (a tensor, array or bytes)."""
        if isinstance(weights, (bytes, bytearray)):
            weights = np.frombuffer(weights, dtype=np.uint8).copy()
        return cls(in_features=in_features, out_features=out_features, format=format, weight=weights)

    def init_synthetic_weights(self, scale: float = 1.0, unit_weights: bool = True,
                               seed: Optional[int] = None) -> None:
        """Fills the weight with generate_synthetic_quantized_weights."""
        self.weight = generate_synthetic_quantized_weights(self.format, self.in_features, self.out_features,
                                                           scale=scale, unit_weights=unit_weights, seed=seed,
                                                           device=str(self.weight.device))

    def forward(self, x, check_finite: bool = False):
        import torch

        if x.dim() < 1:
            raise ValueError(f"Input tensor must have at least 1 dimension, got ndim={x.dim()} with shape "
                             f"{tuple(x.shape)}")
        K, N = self.in_features, self.out_features
        if x.shape[-1] != K:
            raise ValueError(f"Input feature dimension {x.shape[-1]} does not match layer in_features {K}")
        if x.numel() == 0:
            return torch.zeros((*x.shape[:-1], N), dtype=torch.float16, device=x.device)
        if x.dtype != torch.float16:
            x = x.to(torch.float16)
        x = x.contiguous()
        if x.dim() == 1:
            y = torch.empty((N,), dtype=torch.float16, device=x.device)
            m4_bridge_dispatch_gemv(x, self.weight, y, int(self.format), K, N, check_finite=check_finite)
            if check_finite:
                m4_bridge_synchronize()
            return y
        lead = x.shape[:-1]
        x2 = x.reshape(-1, K)
        m = x2.shape[0]
        y2 = torch.empty((m, N), dtype=torch.float16, device=x.device)
        if m == 1:
            m4_bridge_dispatch_gemv(x2, self.weight, y2, int(self.format), K, N, check_finite=check_finite)
        else:
            m4_bridge_dispatch_gemm(x2, self.weight, y2, int(self.format), m, K, N, check_finite=check_finite)
        if check_finite:
            m4_bridge_synchronize()
        return y2.reshape(*lead, N)
