"""GGUF ingestion for the quantization router: ctypes over include/m4_gguf.h.

`GGUFLoader` keeps the method names of the reference's C++ loader
(core/weights/gguf_loader.h:46-129): open, parse_from_buffer, close, is_open,
version, tensor_count, metadata_count, alignment, tensor_data_offset,
file_size, has_metadata, get_metadata, get_string_metadata,
get_uint32_metadata, get_uint64_metadata, has_tensor, get_tensor_info,
tensor_names, get_tensor_raw_data and extract_q2_0_tensor.  On top of it,
`load_router_weights` returns a tensor in the router's block layout (the
bytes the projection entry points take as W), and `repack_ggml_q4_k` /
`repack_mlx_g64` expose the two lossless layout conversions.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from pathlib import Path
from typing import Optional, Union

import numpy as np

import m4_bridge

_VP, _SZ, _I, _U32, _U64, _I64 = (ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_uint32,
                                  ctypes.c_uint64, ctypes.c_int64)
_CP = ctypes.c_char_p


class TensorInfo(ctypes.Structure):
    """m4_gguf_tensor_info."""
    _fields_ = [("n_dims", ctypes.c_uint32), ("dims", ctypes.c_uint64 * 4), ("type", ctypes.c_uint32),
                ("offset", ctypes.c_uint64)]


# name -> (argtypes, restype); every symbol declared in include/m4_gguf.h
SIGNATURES = {
    "m4_gguf_open": ([_CP], _VP),
    "m4_gguf_parse_buffer": ([_VP, _SZ], _VP),
    "m4_gguf_close": ([_VP], None),
    "m4_gguf_version": ([_VP], _U32),
    "m4_gguf_tensor_count": ([_VP], _U64),
    "m4_gguf_metadata_count": ([_VP], _U64),
    "m4_gguf_alignment": ([_VP], _U32),
    "m4_gguf_tensor_data_offset": ([_VP], _U64),
    "m4_gguf_file_size": ([_VP], _SZ),
    "m4_gguf_has_metadata": ([_VP, _CP], ctypes.c_bool),
    "m4_gguf_metadata_type": ([_VP, _CP], _I),
    "m4_gguf_get_string_metadata": ([_VP, _CP, ctypes.c_char_p, _SZ], _I64),
    "m4_gguf_get_uint32_metadata": ([_VP, _CP, _U32], _U32),
    "m4_gguf_get_uint64_metadata": ([_VP, _CP, _U64], _U64),
    "m4_gguf_get_number_metadata": ([_VP, _CP, ctypes.c_double], ctypes.c_double),
    "m4_gguf_get_array_length": ([_VP, _CP], _I64),
    "m4_gguf_has_tensor": ([_VP, _CP], ctypes.c_bool),
    "m4_gguf_get_tensor_info": ([_VP, _CP, ctypes.POINTER(TensorInfo)], _I),
    "m4_gguf_tensor_name": ([_VP, _U64], _CP),
    "m4_gguf_get_tensor_raw_data": ([_VP, _CP], _VP),
    "m4_gguf_extract_q2_0_tensor": ([_VP, _CP, _VP, _SZ, ctypes.POINTER(_U64), ctypes.POINTER(_U64)], _I64),
    "m4_gguf_load_router_weights": ([_VP, _CP, _VP, _SZ, ctypes.POINTER(_I), ctypes.POINTER(_U32),
                                     ctypes.POINTER(_U32)], _I64),
    "m4_repack_ggml_q4_k": ([_VP, _SZ, _VP], _I),
    "m4_repack_mlx_g64": ([_VP, _VP, _VP, _U32, _U32, _VP], _I),
}

# GGUF metadata value types (gguf_loader.h:12-26) and GGML tensor types
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_Q4_K = 0, 1, 2, 8, 12
GGML_PRISM_Q2_0, GGML_PRISM_Q2_0_ALT = 100, 42

_lib: Optional[ctypes.CDLL] = None


def library(path: Optional[Union[str, Path]] = None) -> ctypes.CDLL:
    global _lib
    if _lib is None or path is not None:
        lib = m4_bridge.load_library(path)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


@dataclass
class GGUFTensorInfo:
    """GGUFTensorInfo (gguf_loader.h:38-45)."""
    name: str
    n_dims: int
    dims: list
    type: int
    offset: int


class GGUFLoader:
    def __init__(self, lib_path: Optional[Union[str, Path]] = None) -> None:
        self._lib = library(lib_path)
        self._h: Optional[int] = None
        self._buf = None  # keeps a parsed buffer alive

    # -- lifetime -------------------------------------------------------------
    def open(self, filepath: Union[str, Path]) -> bool:
        self.close()
        h = self._lib.m4_gguf_open(str(filepath).encode())
        self._h = h or None
        return self._h is not None

    def parse_from_buffer(self, data: Union[bytes, bytearray, np.ndarray]) -> bool:
        self.close()
        arr = np.frombuffer(bytes(data), np.uint8) if not isinstance(data, np.ndarray) else \
            np.ascontiguousarray(data, np.uint8)
        h = self._lib.m4_gguf_parse_buffer(arr.ctypes.data, arr.nbytes)
        if h:
            self._h, self._buf = h, arr
        return self._h is not None

    def close(self) -> None:
        if self._h is not None:
            self._lib.m4_gguf_close(self._h)
        self._h, self._buf = None, None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def is_open(self) -> bool:
        return self._h is not None

    # -- header ---------------------------------------------------------------
    def version(self) -> int:
        return int(self._lib.m4_gguf_version(self._h))

    def tensor_count(self) -> int:
        return int(self._lib.m4_gguf_tensor_count(self._h))

    def metadata_count(self) -> int:
        return int(self._lib.m4_gguf_metadata_count(self._h))

    def alignment(self) -> int:
        return int(self._lib.m4_gguf_alignment(self._h))

    def tensor_data_offset(self) -> int:
        return int(self._lib.m4_gguf_tensor_data_offset(self._h))

    def file_size(self) -> int:
        return int(self._lib.m4_gguf_file_size(self._h))

    # -- metadata -------------------------------------------------------------
    def has_metadata(self, key: str) -> bool:
        return bool(self._lib.m4_gguf_has_metadata(self._h, key.encode()))

    def get_string_metadata(self, key: str, default: str = "") -> str:
        n = self._lib.m4_gguf_get_string_metadata(self._h, key.encode(), None, 0)
        if n < 0:
            return default
        buf = ctypes.create_string_buffer(n + 1)
        self._lib.m4_gguf_get_string_metadata(self._h, key.encode(), buf, n + 1)
        return buf.raw[:n].decode("utf-8", errors="replace")

    def get_uint32_metadata(self, key: str, default: int = 0) -> int:
        return int(self._lib.m4_gguf_get_uint32_metadata(self._h, key.encode(), default))

    def get_uint64_metadata(self, key: str, default: int = 0) -> int:
        return int(self._lib.m4_gguf_get_uint64_metadata(self._h, key.encode(), default))

    def get_metadata(self, key: str):
        """Scalar value (int/float/bool/str), array length as ('array', n), or None."""
        t = self._lib.m4_gguf_metadata_type(self._h, key.encode())
        if t < 0:
            return None
        if t == STRING:
            return self.get_string_metadata(key)
        if t == ARRAY:
            return ("array", int(self._lib.m4_gguf_get_array_length(self._h, key.encode())))
        v = self._lib.m4_gguf_get_number_metadata(self._h, key.encode(), 0.0)
        if t in (FLOAT32, FLOAT64):
            return float(v)
        if t == BOOL:
            return bool(v)
        return int(v)

    # -- tensors --------------------------------------------------------------
    def has_tensor(self, name: str) -> bool:
        return bool(self._lib.m4_gguf_has_tensor(self._h, name.encode()))

    def get_tensor_info(self, name: str) -> Optional[GGUFTensorInfo]:
        ti = TensorInfo()
        if self._lib.m4_gguf_get_tensor_info(self._h, name.encode(), ctypes.byref(ti)) != 0:
            return None
        return GGUFTensorInfo(name, ti.n_dims, [int(ti.dims[d]) for d in range(min(ti.n_dims, 4))], ti.type,
                              ti.offset)

    def tensor_names(self) -> list:
        return [self._lib.m4_gguf_tensor_name(self._h, i).decode() for i in range(self.tensor_count())]

    def get_tensor_raw_data(self, name: str) -> Optional[int]:
        """Address of the tensor's first byte (None past the end / missing)."""
        p = self._lib.m4_gguf_get_tensor_raw_data(self._h, name.encode())
        return int(p) if p else None

    def extract_q2_0_tensor(self, name: str):
        """(blocks uint8 [n, 34], K, N) or None (gguf_loader.mm:349-409)."""
        info = self.get_tensor_info(name)
        if info is None or not info.dims:
            return None
        n = int(np.prod(info.dims, dtype=np.uint64))
        out = np.empty(max(1, n // 128) * 34, np.uint8)
        k, nn = _U64(), _U64()
        r = self._lib.m4_gguf_extract_q2_0_tensor(self._h, name.encode(), out.ctypes.data, out.nbytes,
                                                  ctypes.byref(k), ctypes.byref(nn))
        if r < 0:
            return None
        return out[: r * 34].reshape(r, 34), int(k.value), int(nn.value)

    def load_router_weights(self, name: str):
        """(W uint8 bytes in router layout, format, K, N); raises ValueError with
        the entry point's status when the tensor cannot feed the router."""
        f, k, n = _I(), _U32(), _U32()
        need = self._lib.m4_gguf_load_router_weights(self._h, name.encode(), None, 0, ctypes.byref(f),
                                                     ctypes.byref(k), ctypes.byref(n))
        if need < 0:
            raise ValueError(f"{name}: m4_gguf_load_router_weights status {need}")
        out = np.empty(need, np.uint8)
        r = self._lib.m4_gguf_load_router_weights(self._h, name.encode(), out.ctypes.data, out.nbytes,
                                                  ctypes.byref(f), ctypes.byref(k), ctypes.byref(n))
        if r != need:
            raise ValueError(f"{name}: m4_gguf_load_router_weights status {r}")
        return out, int(f.value), int(k.value), int(n.value)


def repack_ggml_q4_k(blocks: np.ndarray) -> np.ndarray:
    """GGML block_q4_K bytes [n * 144] -> router Q4_K bytes (same weights)."""
    src = np.ascontiguousarray(blocks, np.uint8).reshape(-1)
    assert src.size % 144 == 0
    out = np.empty_like(src)
    library().m4_repack_ggml_q4_k(src.ctypes.data, src.size // 144, out.ctypes.data)
    return out


def repack_mlx_g64(wq: np.ndarray, scales: np.ndarray, biases: np.ndarray) -> np.ndarray:
    """MLX 4-bit g64 (wq uint32 [N, K/8], scales/biases fp16 [N, K/64]) ->
    router MLX_4BIT blocks (uint8 [N * K/32 * 20])."""
    wq = np.ascontiguousarray(wq, np.uint32)
    N, K = wq.shape[0], wq.shape[1] * 8
    if K % 64:
        raise ValueError(f"K = {K} is not a whole number of 64-element groups")
    sc = np.ascontiguousarray(scales, np.float16)
    bi = np.ascontiguousarray(biases, np.float16)
    assert sc.shape == (N, K // 64) and bi.shape == (N, K // 64)
    out = np.empty(N * (K // 32) * 20, np.uint8)
    r = library().m4_repack_mlx_g64(wq.ctypes.data, sc.ctypes.data, bi.ctypes.data, N, K, out.ctypes.data)
    if r != 0:
        raise ValueError(f"m4_repack_mlx_g64 status {r}")
    return out
