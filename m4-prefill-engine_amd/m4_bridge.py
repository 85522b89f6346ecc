"""ctypes bridge to libm4_bridge.so -- the MI355X quantization-router prefill path.

Mirrors the reference's Python bridge (core/bridge/m4_bridge.py:18-280): the
same class and module-level names, format ints, M/K/N inference, non-zero
status -> RuntimeError mapping, deferred NaN/Inf tripwire at synchronize(),
and in-flight buffer retention until synchronize().  Buffers are torch-ROCm
tensors (device pointers, zero-copy) or numpy arrays (host memory, staged by
the library).  There is no fallback: if the shared library is missing the
constructor raises.
"""
from __future__ import annotations

import ctypes
import os
from enum import IntEnum
from pathlib import Path
from typing import Any, Optional, Union


class QuantFormat(IntEnum):
    """core/bridge/m4_bridge.py:18-24 (ids 0..5 are dispatchable)."""
    QUANT_Q4_0 = 0
    QUANT_MLX_4BIT = 1
    QUANT_Q4_K = 2
    QUANT_TERNARY_1_58 = 3
    QUANT_VAR_RATE_AFFINE = 4
    QUANT_EXL3 = 5
    # beyond the reference's dispatchable range (kernel-name entry points only)
    QUANT_Q8_0 = 6
    QUANT_PRISM_Q2_0 = 7
    QUANT_MLX_4BIT_G64 = 8  # MLX's native 64-element groups (36 B / 64)


LIB_NAME = "libm4_bridge.so"


def _find_library_path() -> Path:
    """Library location: $M4_BRIDGE_LIB_PATH (or the reference's
    $M4_BRIDGE_DYLIB_PATH), then next to this file, then the cwd
    (core/bridge/m4_bridge.py:27-44)."""
    for var in ("M4_BRIDGE_LIB_PATH", "M4_BRIDGE_DYLIB_PATH"):
        env = os.environ.get(var)
        if env and Path(env).is_file():
            return Path(env)
    here = Path(__file__).resolve().parent
    candidates = [here / LIB_NAME, here.parent / LIB_NAME, Path.cwd() / LIB_NAME]
    for cand in candidates:
        if cand.is_file():
            return cand
    raise FileNotFoundError(
        f"Could not locate {LIB_NAME}. Checked: {[str(c) for c in candidates]}. "
        "Build it with `python m4-prefill-engine_amd/build.py` or set M4_BRIDGE_LIB_PATH."
    )


_VP, _SZ, _I, _U32, _F = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_uint32, ctypes.c_float

# name -> (argtypes, restype); every symbol declared in include/m4_mlx_bridge.h
SIGNATURES = {
    "m4_bridge_init": ([ctypes.c_char_p], ctypes.c_bool),
    "m4_bridge_get_expected_weight_bytes": ([_I, _U32, _U32], _SZ),
    "m4_bridge_dispatch_gemm": ([_VP, _SZ, _VP, _SZ, _VP, _SZ, _I, _U32, _U32, _U32], _I),
    "m4_bridge_dispatch_gemv": ([_VP, _SZ, _VP, _SZ, _VP, _SZ, _I, _U32, _U32], _I),
    "m4_bridge_synchronize": ([], None),
    "m4_bridge_get_uma_footprint_mb": ([], ctypes.c_double),
    "m4_bridge_is_initialized": ([], ctypes.c_bool),
    "m4_bridge_shutdown": ([], None),
    "m4_bridge_validate_gemm": ([_VP, _SZ, _VP, _SZ, _VP, _SZ, _I, _U32, _U32, _U32], _I),
    "m4_bridge_dispatch_gemm_noalloc": ([_VP, _SZ, _VP, _SZ, _VP, _SZ, _I, _U32, _U32, _U32], _I),
    "m4_bridge_dispatch_router_gemm": ([_VP, _SZ, _VP, _SZ, _VP, _SZ, _I, _U32, _U32, _U32], _I),
    "m4_bridge_dispatch_head_gemm": ([_VP, _SZ, _VP, _SZ, _VP, _SZ, _I, _U32, _U32, _U32, _U32], _I),
    "m4_bridge_dispatch_router_kernel": ([ctypes.c_char_p, _VP, _SZ, _VP, _SZ, _VP, _SZ,
                                          ctypes.POINTER(ctypes.c_uint32), _U32], _I),
    "m4_bridge_dispatch_gemm_residual": ([_VP, _SZ, _VP, _SZ, _VP, _SZ, _VP, _SZ, _I, _U32, _U32, _U32], _I),
    "m4_bridge_dispatch_swiglu": ([_VP, _SZ, _VP, _SZ, _VP, _SZ, _VP, _SZ, _I, _U32, _U32, _U32], _I),
    "m4_bridge_quantize_kv_q8_0": ([_VP, _SZ, _VP, _SZ, ctypes.c_uint64], _I),
    "m4_bridge_dispatch_flash_attn_q8_0": ([_VP, _SZ, _VP, _SZ, _VP, _SZ, _VP, _SZ, _U32, _U32, _U32, _F, _I], _I),
    "m4_bridge_prefill_layer": ([_VP] * 9 + [_I, _U32, _U32, _U32, _U32, _U32, _F], _I),
    "m4_bridge_dispatch_flash_attn_q8_0_gqa": ([_VP, _SZ, _VP, _SZ, _VP, _SZ, _VP, _SZ, _U32, _U32, _U32, _U32, _F,
                                                _I], _I),
    "m4_bridge_rmsnorm": ([_VP, _SZ, _VP, _SZ, _VP, _SZ, _U32, _U32, _F, _I], _I),
    "m4_bridge_rope": ([_VP, _SZ, _U32, _U32, _U32, _F, _U32, _I], _I),
    "m4_bridge_prefill_layer_ex": ([_VP] * 11 + [_I, _U32, _U32, _U32, _U32, _U32, _U32, _F, _I, _F, _I, _F, _U32,
                                                 _I], _I),
    "m4_bridge_prefill_layer_ex_kv": ([_VP] * 13 + [_I, _U32, _U32, _U32, _U32, _U32, _U32, _F, _I, _F, _I, _F,
                                                    _U32, _I], _I),
    "m4_bridge_dequantize": ([_VP, _SZ, _VP, _SZ, _I, _U32, _U32], _I),
    "m4_bridge_set_stream": ([_VP], _I),
    "m4_bridge_get_stream": ([], _VP),
    "m4_bridge_last_error": ([], ctypes.c_char_p),
    "m4_probe_hbm_bandwidth": ([_SZ, _I, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)], _I),
    "m4_probe_mfma_f16": ([_U32, _I, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)], _I),
    "m4_probe_mfma_f16_random": ([_U32, _I, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)], _I),
    "m4_registry_get": ([_I, _VP], _I),
    "m4_registry_get_by_name": ([ctypes.c_char_p], _I),
    "m4_registry_available_formats": ([ctypes.POINTER(_I), _I], _I),
    "m4_registry_compute_weight_bytes": ([_I, ctypes.c_uint64], ctypes.c_uint64),
    "m4_registry_has_format": ([_I], ctypes.c_bool),
    "m4_registry_register_codec": ([_VP], _I),
}


class CodecInfo(ctypes.Structure):
    """m4_quant_codec_info (include/m4_mlx_bridge.h)."""
    _fields_ = [
        ("format", ctypes.c_int),
        ("name", ctypes.c_char_p),
        ("description", ctypes.c_char_p),
        ("block_size", ctypes.c_uint32),
        ("struct_size", ctypes.c_uint64),
        ("bits_per_weight", ctypes.c_double),
        ("gemm_kernel_name", ctypes.c_char_p),
        ("head_gemm_kernel_name", ctypes.c_char_p),
    ]


def load_library(path: Optional[Union[str, Path]] = None) -> ctypes.CDLL:
    # One HIP runtime per process: torch-ROCm ships its own libamdhip64.so.7.
    # Importing torch first makes the library bind to that already-loaded
    # runtime (same SONAME) instead of loading /opt/rocm's beside it, which
    # would leave torch without a usable device.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(str(Path(path) if path else _find_library_path()))
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


def _is_torch(x: Any) -> bool:
    return type(x).__module__.startswith("torch")


class HIPBridge:
    """Counterpart of the reference's MetalUMABridge (core/bridge/m4_bridge.py:47-242)."""

    _instance: Optional["HIPBridge"] = None
    _retained_contig: list = []

    def __init__(self, lib_path: Optional[Union[str, Path]] = None) -> None:
        self._lib = load_library(lib_path)
        self._in_flight_tensors: list[tuple] = []
        self._pending_finite_checks: list = []

    @property
    def lib(self) -> ctypes.CDLL:
        return self._lib

    @classmethod
    def get_instance(cls, lib_path: Optional[Union[str, Path]] = None) -> "HIPBridge":
        if cls._instance is None:
            cls._instance = cls(lib_path)
        return cls._instance

    # -- buffers ------------------------------------------------------------
    @classmethod
    def extract_buffer_address_and_size(cls, arr: Any) -> tuple[int, int]:
        """(address, nbytes) of a torch tensor or numpy array; non-contiguous
        inputs are made contiguous and retained until synchronize()
        (core/bridge/m4_bridge.py:110-127)."""
        if _is_torch(arr):
            if not arr.is_contiguous():
                arr = arr.contiguous()
                cls._retained_contig.append(arr)
            return int(arr.data_ptr()), int(arr.numel() * arr.element_size())
        import numpy as np

        a = arr
        if not isinstance(a, np.ndarray):
            raise TypeError(f"unsupported buffer type {type(arr)!r}")
        if not a.flags["C_CONTIGUOUS"]:
            a = np.ascontiguousarray(a)
            cls._retained_contig.append(a)
        return int(a.ctypes.data), int(a.nbytes)

    def _bind_stream(self, *bufs: Any) -> None:
        """Issue on torch's current stream when any buffer is a CUDA tensor, so
        the kernels are ordered after the work that produced the inputs."""
        for b in bufs:
            if _is_torch(b) and b.is_cuda:
                import torch

                self._lib.m4_bridge_set_stream(ctypes.c_void_p(torch.cuda.current_stream(b.device).cuda_stream))
                return

    def _check(self, name: str, ret: int) -> int:
        if ret != 0:
            raise RuntimeError(f"{name} failed with status code {ret}")
        return ret

    # -- reference API ------------------------------------------------------
    def init(self, metallib_path: Optional[str] = None) -> bool:
        c_path = metallib_path.encode("utf-8") if metallib_path else None
        return bool(self._lib.m4_bridge_init(c_path))

    def is_initialized(self) -> bool:
        return bool(self._lib.m4_bridge_is_initialized())

    def get_expected_weight_bytes(self, format: Union[int, QuantFormat], K: int, N: int) -> int:
        return int(self._lib.m4_bridge_get_expected_weight_bytes(int(format), K, N))

    def dispatch_gemm(self, X, W, Y, format, M=None, K=None, N=None, check_finite: bool = False) -> int:
        """Y[M,N] = X[M,K] . W^T (core/bridge/m4_bridge.py:136-179)."""
        x_ptr, x_bytes = self.extract_buffer_address_and_size(X)
        w_ptr, w_bytes = self.extract_buffer_address_and_size(W)
        y_ptr, y_bytes = self.extract_buffer_address_and_size(Y)
        if M is None:
            M = X.shape[0] if len(X.shape) >= 2 else 1
        if K is None:
            K = X.shape[1] if len(X.shape) >= 2 else X.shape[0]
        if N is None:
            N = Y.shape[1] if len(Y.shape) >= 2 else Y.shape[0]
        self._bind_stream(X, W, Y)
        ret = self._lib.m4_bridge_dispatch_gemm(x_ptr, x_bytes, w_ptr, w_bytes, y_ptr, y_bytes, int(format),
                                                int(M), int(K), int(N))
        self._check("m4_bridge_dispatch_gemm", ret)
        self._in_flight_tensors.append((X, W, Y))
        if check_finite:
            self._pending_finite_checks.append(Y)
        return ret

    def dispatch_gemv(self, x, W, y, format, K=None, N=None, check_finite: bool = False) -> int:
        """y[N] = W . x (core/bridge/m4_bridge.py:181-220)."""
        x_ptr, x_bytes = self.extract_buffer_address_and_size(x)
        w_ptr, w_bytes = self.extract_buffer_address_and_size(W)
        y_ptr, y_bytes = self.extract_buffer_address_and_size(y)
        if K is None:
            K = x.shape[-1]
        if N is None:
            N = y.shape[-1]
        self._bind_stream(x, W, y)
        ret = self._lib.m4_bridge_dispatch_gemv(x_ptr, x_bytes, w_ptr, w_bytes, y_ptr, y_bytes, int(format),
                                                int(K), int(N))
        self._check("m4_bridge_dispatch_gemv", ret)
        self._in_flight_tensors.append((x, W, y))
        if check_finite:
            self._pending_finite_checks.append(y)
        return ret

    def synchronize(self) -> None:
        """Waits for the issued work, releases retained buffers, then runs the
        deferred NaN/Inf tripwire (core/bridge/m4_bridge.py:222-233)."""
        self._lib.m4_bridge_synchronize()
        self._in_flight_tensors.clear()
        self._retained_contig.clear()
        if self._pending_finite_checks:
            checks = list(self._pending_finite_checks)
            self._pending_finite_checks.clear()
            for t in checks:
                if not _all_finite(t):
                    raise FloatingPointError(
                        "Tripwire assertion failed: Non-finite values (NaN/Inf) detected in output tensor.")

    def get_uma_footprint_mb(self) -> float:
        return float(self._lib.m4_bridge_get_uma_footprint_mb())

    def shutdown(self) -> None:
        self._in_flight_tensors.clear()
        self._retained_contig.clear()
        self._pending_finite_checks.clear()
        self._lib.m4_bridge_shutdown()

    # -- router extensions ----------------------------------------------------
    def dispatch_router_gemm(self, X, W, Y, format, M=None, K=None, N=None, check_finite: bool = False) -> int:
        """Y = X . W^T for every format with a kernel, PRISM_Q2_0 and Q8_0 weights
        included (quant_router_gemm_<fmt>_64x64, quant_router_kernels.metal:588-750)."""
        x_ptr, x_bytes = self.extract_buffer_address_and_size(X)
        w_ptr, w_bytes = self.extract_buffer_address_and_size(W)
        y_ptr, y_bytes = self.extract_buffer_address_and_size(Y)
        M = X.shape[0] if M is None else M
        K = X.shape[1] if K is None else K
        N = Y.shape[1] if N is None else N
        self._bind_stream(X, W, Y)
        ret = self._lib.m4_bridge_dispatch_router_gemm(x_ptr, x_bytes, w_ptr, w_bytes, y_ptr, y_bytes, int(format),
                                                       int(M), int(K), int(N))
        self._check("m4_bridge_dispatch_router_gemm", ret)
        self._in_flight_tensors.append((X, W, Y))
        if check_finite:
            self._pending_finite_checks.append(Y)
        return ret

    def dispatch_head_gemm(self, X, W, Y, format, M, H, D, K, check_finite: bool = False) -> int:
        """Direct-head projection: Y [H, M, D] (quant_router_kernels.metal:754-927)."""
        a = [self.extract_buffer_address_and_size(t) for t in (X, W, Y)]
        self._bind_stream(X, W, Y)
        ret = self._lib.m4_bridge_dispatch_head_gemm(a[0][0], a[0][1], a[1][0], a[1][1], a[2][0], a[2][1],
                                                     int(format), M, H, D, K)
        self._check("m4_bridge_dispatch_head_gemm", ret)
        self._in_flight_tensors.append((X, W, Y))
        if check_finite:
            self._pending_finite_checks.append(Y)
        return ret

    def dispatch_router_kernel(self, kernel_name: str, X, W, Y, *dims, check_finite: bool = False) -> int:
        """A router kernel by its Metal pipeline name with that kernel's slots:
        buffers A = X, B = W, C = Y, then the constants -- (M, N, K) for
        quant_router_gemm_<fmt>_64x64, (M, H, D, K) for the head kernels
        (quant_router_kernels.metal:588-927).  The vector-ALU ternary names
        quant_router_{,head_}gemm_ternary_1_58_vec (:934-1201) compute the same
        projection on the matrix-core path."""
        a = [self.extract_buffer_address_and_size(t) for t in (X, W, Y)]
        self._bind_stream(X, W, Y)
        arr = (ctypes.c_uint32 * max(len(dims), 1))(*[int(d) for d in dims])
        ret = self._lib.m4_bridge_dispatch_router_kernel(kernel_name.encode(), a[0][0], a[0][1], a[1][0], a[1][1],
                                                         a[2][0], a[2][1], arr, len(dims))
        self._check("m4_bridge_dispatch_router_kernel", ret)
        self._in_flight_tensors.append((X, W, Y))
        if check_finite:
            self._pending_finite_checks.append(Y)
        return ret

    def dispatch_gemm_residual(self, X, W, R, Y, format, M, K, N) -> int:
        a = [self.extract_buffer_address_and_size(t) for t in (X, W, R, Y)]
        self._bind_stream(X, W, R, Y)
        ret = self._lib.m4_bridge_dispatch_gemm_residual(a[0][0], a[0][1], a[1][0], a[1][1], a[2][0], a[2][1],
                                                         a[3][0], a[3][1], int(format), M, K, N)
        self._check("m4_bridge_dispatch_gemm_residual", ret)
        self._in_flight_tensors.append((X, W, R, Y))
        return ret

    def dispatch_swiglu(self, X, Wg, Wu, Out, format, M, N_mlp, K) -> int:
        """Out = silu(X . Wg^T) * (X . Wu^T) (brick3_swiglu_kernels.metal:428-698)."""
        a = [self.extract_buffer_address_and_size(t) for t in (X, Wg, Wu, Out)]
        self._bind_stream(X, Wg, Wu, Out)
        ret = self._lib.m4_bridge_dispatch_swiglu(a[0][0], a[0][1], a[1][0], a[1][1], a[2][0], a[2][1],
                                                  a[3][0], a[3][1], int(format), M, N_mlp, K)
        self._check("m4_bridge_dispatch_swiglu", ret)
        self._in_flight_tensors.append((X, Wg, Wu, Out))
        return ret

    def quantize_kv_q8_0(self, src, dst, num_blocks: Optional[int] = None) -> int:
        """fp16 -> Q8_0 blocks (unified_kernels.metal:118-145)."""
        s = self.extract_buffer_address_and_size(src)
        d = self.extract_buffer_address_and_size(dst)
        nb = s[1] // 64 if num_blocks is None else num_blocks
        self._bind_stream(src, dst)
        ret = self._lib.m4_bridge_quantize_kv_q8_0(s[0], s[1], d[0], d[1], nb)
        self._check("m4_bridge_quantize_kv_q8_0", ret)
        self._in_flight_tensors.append((src, dst))
        return ret

    def dispatch_flash_attn_q8_0(self, Q, Kq, Vq, O, H, M, D, scale, o_token_major: bool = False) -> int:
        """Causal attention over a Q8_0 KV cache (brick4_attn_kernels.metal:572-911)."""
        a = [self.extract_buffer_address_and_size(t) for t in (Q, Kq, Vq, O)]
        self._bind_stream(Q, Kq, Vq, O)
        ret = self._lib.m4_bridge_dispatch_flash_attn_q8_0(a[0][0], a[0][1], a[1][0], a[1][1], a[2][0], a[2][1],
                                                           a[3][0], a[3][1], H, M, D, float(scale),
                                                           int(bool(o_token_major)))
        self._check("m4_bridge_dispatch_flash_attn_q8_0", ret)
        self._in_flight_tensors.append((Q, Kq, Vq, O))
        return ret

    def prefill_layer(self, X, Wq, Wk, Wv, Wo, Wg, Wu, Wd, X_out, format, M, d_model, H, D, N_mlp,
                      attn_scale) -> int:
        """One prefill layer (models/transformer_layer.mm:75-218) over device tensors."""
        bufs = (X, Wq, Wk, Wv, Wo, Wg, Wu, Wd, X_out)
        ptrs = [self.extract_buffer_address_and_size(t)[0] for t in bufs]
        self._bind_stream(*bufs)
        ret = self._lib.m4_bridge_prefill_layer(*ptrs, int(format), M, d_model, H, D, N_mlp, float(attn_scale))
        self._check("m4_bridge_prefill_layer", ret)
        self._in_flight_tensors.append(bufs)
        return ret

    def dispatch_flash_attn_q8_0_gqa(self, Q, Kq, Vq, O, H, Hkv, M, D, scale, o_token_major: bool = False) -> int:
        """Grouped-query causal attention: K/V hold Hkv heads (src/engine/model.py:234-236)."""
        a = [self.extract_buffer_address_and_size(t) for t in (Q, Kq, Vq, O)]
        self._bind_stream(Q, Kq, Vq, O)
        ret = self._lib.m4_bridge_dispatch_flash_attn_q8_0_gqa(a[0][0], a[0][1], a[1][0], a[1][1], a[2][0], a[2][1],
                                                               a[3][0], a[3][1], H, Hkv, M, D, float(scale),
                                                               int(bool(o_token_major)))
        self._check("m4_bridge_dispatch_flash_attn_q8_0_gqa", ret)
        self._in_flight_tensors.append((Q, Kq, Vq, O))
        return ret

    def rmsnorm(self, X, w, Y, eps: float = 1e-5, norm_type: int = 1) -> int:
        """RMSNorm over the rows of X [M, D] (src/engine/model.py:39-48); norm_type 2 = gemma_add_one."""
        a = [self.extract_buffer_address_and_size(t) for t in (X, w, Y)]
        M, D = X.shape
        self._bind_stream(X, w, Y)
        ret = self._lib.m4_bridge_rmsnorm(a[0][0], a[0][1], a[1][0], a[1][1], a[2][0], a[2][1], M, D, float(eps),
                                          int(norm_type))
        self._check("m4_bridge_rmsnorm", ret)
        self._in_flight_tensors.append((X, w, Y))
        return ret

    def rope(self, T, theta: float = 10000.0, offset: int = 0, traditional: bool = False) -> int:
        """RoPE in place on T [H, M, D] (nn.RoPE, src/engine/model.py:112-116)."""
        ptr, nbytes = self.extract_buffer_address_and_size(T)
        H, M, D = T.shape
        self._bind_stream(T)
        ret = self._lib.m4_bridge_rope(ptr, nbytes, H, M, D, float(theta), int(offset), int(bool(traditional)))
        self._check("m4_bridge_rope", ret)
        self._in_flight_tensors.append((T,))
        return ret

    def prefill_layer_ex(self, X, w_attn, Wq, Wk, Wv, Wo, w_ffn, Wg, Wu, Wd, X_out, format, M, d_model, Hq, Hkv, D,
                         N_mlp, attn_scale, norm_type: int = 1, norm_eps: float = 1e-5, rope: bool = True,
                         rope_theta: float = 10000.0, rope_offset: int = 0, rope_traditional: bool = False) -> int:
        """The MLX transformer block on the router's kernels (src/engine/model.py:181-265)."""
        bufs = (X, w_attn, Wq, Wk, Wv, Wo, w_ffn, Wg, Wu, Wd, X_out)
        ptrs = [None if t is None else self.extract_buffer_address_and_size(t)[0] for t in bufs]
        self._bind_stream(*[t for t in bufs if t is not None])
        ret = self._lib.m4_bridge_prefill_layer_ex(*ptrs, int(format), M, d_model, Hq, Hkv, D, N_mlp,
                                                   float(attn_scale), int(norm_type), float(norm_eps), int(bool(rope)),
                                                   float(rope_theta), int(rope_offset), int(bool(rope_traditional)))
        self._check("m4_bridge_prefill_layer_ex", ret)
        self._in_flight_tensors.append(bufs)
        return ret

    def prefill_layer_ex_kv(self, X, w_attn, Wq, Wk, Wv, Wo, w_ffn, Wg, Wu, Wd, X_out, Kq_out, Vq_out, format, M,
                            d_model, Hq, Hkv, D, N_mlp, attn_scale, norm_type: int = 1, norm_eps: float = 1e-5,
                            rope: bool = True, rope_theta: float = 10000.0, rope_offset: int = 0,
                            rope_traditional: bool = False) -> int:
        """prefill_layer_ex that also writes the layer's Q8_0 K / V cache
        (unified_prefill_engine.mm:548-572) to Kq_out / Vq_out."""
        bufs = (X, w_attn, Wq, Wk, Wv, Wo, w_ffn, Wg, Wu, Wd, X_out, Kq_out, Vq_out)
        ptrs = [None if t is None else self.extract_buffer_address_and_size(t)[0] for t in bufs]
        self._bind_stream(*[t for t in bufs if t is not None])
        ret = self._lib.m4_bridge_prefill_layer_ex_kv(*ptrs, int(format), M, d_model, Hq, Hkv, D, N_mlp,
                                                      float(attn_scale), int(norm_type), float(norm_eps),
                                                      int(bool(rope)), float(rope_theta), int(rope_offset),
                                                      int(bool(rope_traditional)))
        self._check("m4_bridge_prefill_layer_ex_kv", ret)
        self._in_flight_tensors.append(bufs)
        return ret

    def dequantize(self, W, out, format, K, N) -> int:
        a = [self.extract_buffer_address_and_size(t) for t in (W, out)]
        self._bind_stream(W, out)
        ret = self._lib.m4_bridge_dequantize(a[0][0], a[0][1], a[1][0], a[1][1], int(format), K, N)
        self._check("m4_bridge_dequantize", ret)
        self._in_flight_tensors.append((W, out))
        return ret

    def last_error(self) -> str:
        return (self._lib.m4_bridge_last_error() or b"").decode()


# The reference's class name, for callers written against it.
MetalUMABridge = HIPBridge


def _all_finite(t: Any) -> bool:
    if _is_torch(t):
        import torch

        return bool(torch.isfinite(t).all().item())
    import numpy as np

    a = np.asarray(t)
    if a.dtype == np.uint16:
        a = a.view(np.float16)
    return bool(np.isfinite(a).all())


# Module-level convenience functions matching the C-ABI (core/bridge/m4_bridge.py:245-280)
def m4_bridge_init(metallib_path: Optional[str] = None) -> bool:
    return HIPBridge.get_instance().init(metallib_path)


def m4_bridge_dispatch_gemm(X, W, Y, format, M=None, K=None, N=None, check_finite: bool = False) -> int:
    return HIPBridge.get_instance().dispatch_gemm(X, W, Y, format, M, K, N, check_finite=check_finite)


def m4_bridge_dispatch_gemv(x, W, y, format, K=None, N=None, check_finite: bool = False) -> int:
    return HIPBridge.get_instance().dispatch_gemv(x, W, y, format, K, N, check_finite=check_finite)


def m4_bridge_synchronize() -> None:
    HIPBridge.get_instance().synchronize()


def m4_bridge_get_uma_footprint_mb() -> float:
    return HIPBridge.get_instance().get_uma_footprint_mb()
