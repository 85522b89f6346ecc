"""ctypes bindings of liboracle.so (the CPU restatement of the reference's gold path).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker -- never by the product.
Arrays are numpy; fp16 tensors are passed as float16 arrays (bit patterns).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE), "-B", "liboracle.so"], check=True)
    return LIB


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists() or LIB.stat().st_mtime < (HERE / "oracle.c").stat().st_mtime:
            build()
        L = ctypes.CDLL(str(LIB))
        vp, u32, i, sz, f = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int, ctypes.c_size_t, ctypes.c_float
        L.orc_f16_to_f64.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f64.restype = ctypes.c_double
        L.orc_f64_to_f16.argtypes = [ctypes.c_double]
        L.orc_f64_to_f16.restype = ctypes.c_uint16
        L.orc_f64_to_f16_array.argtypes = [vp, vp, sz]
        L.orc_f16_to_f64_array.argtypes = [vp, vp, sz]
        L.orc_dequantize.argtypes = [i, vp, vp, u32, u32]
        L.orc_dequantize.restype = i
        L.orc_dequantize_f64.argtypes = [i, vp, vp, u32, u32]
        L.orc_dequantize_f64.restype = i
        L.orc_gemm.argtypes = [i, vp, vp, vp, vp, u32, u32, u32, i, u32, u32, i]
        L.orc_gemm.restype = i
        L.orc_swiglu.argtypes = [i, vp, vp, vp, vp, u32, u32, u32, i]
        L.orc_swiglu.restype = i
        L.orc_quantize_q8_0.argtypes = [vp, vp, sz]
        L.orc_dequantize_q8_0.argtypes = [vp, vp, sz]
        L.orc_attention.argtypes = [vp, vp, vp, vp, u32, u32, u32, f, i, i]
        L.orc_attention_q8_0.argtypes = [vp, vp, vp, vp, u32, u32, u32, f, i, i]
        L.orc_layer.argtypes = [i] + [vp] * 9 + [u32, u32, u32, u32, u32, f] + [vp] * 6 + [i]
        L.orc_layer.restype = i
        L.orc_attention_gqa.argtypes = [vp, vp, vp, vp, u32, u32, u32, u32, f, i, i]
        L.orc_attention_gqa.restype = i
        L.orc_attention_q8_0_gqa.argtypes = [vp, vp, vp, vp, u32, u32, u32, u32, f, i, i]
        L.orc_attention_q8_0_gqa.restype = i
        L.orc_rmsnorm.argtypes = [vp, vp, vp, u32, u32, f, i]
        L.orc_rmsnorm.restype = i
        L.orc_rope.argtypes = [vp, u32, u32, u32, f, u32, i]
        L.orc_rope.restype = i
        L.orc_layer_ex.argtypes = [i] + [vp] * 11 + [u32] * 6 + [f, i, f, i, f, u32, i, i]
        L.orc_layer_ex.restype = i
        L.orc_attention_rows.argtypes = [vp] * 5 + [u32] * 5 + [f, i, i]
        L.orc_attention_rows.restype = i
        L.orc_layer_ex_rows.argtypes = [i] + [vp] * 12 + [u32] * 7 + [f, i, f, i, f, u32, i, i]
        L.orc_layer_ex_rows.restype = i
        _lib = L
    return _lib


def threads() -> int:
    return int(os.environ.get("ORACLE_THREADS", os.cpu_count() or 1))


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return ctypes.c_void_p(a.ctypes.data)


def f64_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float64)
    out = np.empty(x.shape, np.float16)
    lib().orc_f64_to_f16_array(_p(x), _p(out), x.size)
    return out


def f16_to_f64(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float16)
    out = np.empty(x.shape, np.float64)
    lib().orc_f16_to_f64_array(_p(x), _p(out), x.size)
    return out


def dequantize(fmt: int, W: np.ndarray, K: int, N: int) -> np.ndarray:
    W = np.ascontiguousarray(W, dtype=np.uint8)
    out = np.empty((N, K), np.float16)
    rc = lib().orc_dequantize(fmt, _p(W), _p(out), K, N)
    assert rc == 0, rc
    return out


def dequantize_f64(fmt: int, W: np.ndarray, K: int, N: int) -> np.ndarray:
    """Exact double weights [N, K] (what the gold multiplies the activations by)."""
    W = np.ascontiguousarray(W, dtype=np.uint8)
    out = np.empty((N, K), np.float64)
    rc = lib().orc_dequantize_f64(fmt, _p(W), _p(out), K, N)
    assert rc == 0, rc
    return out


def gemm(fmt: int, X: np.ndarray, W: np.ndarray, N: int, R: np.ndarray | None = None, head_D: int = 0,
         nthreads: int | None = None) -> np.ndarray:
    """fp16(X . W^T [+ R]); head_D > 0 gives the [N/head_D, M, head_D] layout."""
    X = np.ascontiguousarray(X, dtype=np.float16)
    M, K = X.shape
    W = np.ascontiguousarray(W, dtype=np.uint8)
    if head_D:
        out = np.empty((N // head_D, M, head_D), np.float16)
    else:
        out = np.empty((M, N), np.float16)
    rp = None
    if R is not None:
        R = np.ascontiguousarray(R, dtype=np.float16)
        rp = _p(R)
    rc = lib().orc_gemm(fmt, _p(X), _p(W), _p(out), rp, M, N, K, 1 if head_D else 0,
                        N // head_D if head_D else 0, head_D, nthreads or threads())
    assert rc == 0, rc
    return out


def swiglu(fmt: int, X: np.ndarray, Wg: np.ndarray, Wu: np.ndarray, N: int, nthreads: int | None = None):
    X = np.ascontiguousarray(X, dtype=np.float16)
    M, K = X.shape
    out = np.empty((M, N), np.float16)
    Wg = np.ascontiguousarray(Wg, dtype=np.uint8)
    Wu = np.ascontiguousarray(Wu, dtype=np.uint8)
    rc = lib().orc_swiglu(fmt, _p(X), _p(Wg), _p(Wu), _p(out), M, N, K, nthreads or threads())
    assert rc == 0, rc
    return out


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float16).reshape(-1)
    nb = x.size // 32
    out = np.empty(nb * 34, np.uint8)
    lib().orc_quantize_q8_0(_p(x), _p(out), nb)
    return out


def dequantize_q8_0(q: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    nb = q.size // 34
    out = np.empty(nb * 32, np.float16)
    lib().orc_dequantize_q8_0(_p(q), _p(out), nb)
    return out


def attention(Q, K, V, scale: float, o_token_major: bool = False, nthreads: int | None = None):
    Q, K, V = (np.ascontiguousarray(a, dtype=np.float16) for a in (Q, K, V))
    H, M, D = Q.shape
    out = np.empty((M, H * D) if o_token_major else (H, M, D), np.float16)
    lib().orc_attention(_p(Q), _p(K), _p(V), _p(out), H, M, D, scale, int(o_token_major), nthreads or threads())
    return out


def attention_q8_0(Q, Kq, Vq, scale: float, o_token_major: bool = False, nthreads: int | None = None):
    Q = np.ascontiguousarray(Q, dtype=np.float16)
    H, M, D = Q.shape
    Kq = np.ascontiguousarray(Kq, dtype=np.uint8)
    Vq = np.ascontiguousarray(Vq, dtype=np.uint8)
    out = np.empty((M, H * D) if o_token_major else (H, M, D), np.float16)
    lib().orc_attention_q8_0(_p(Q), _p(Kq), _p(Vq), _p(out), H, M, D, scale, int(o_token_major),
                             nthreads or threads())
    return out


def layer(fmt: int, X, Wq, Wk, Wv, Wo, Wg, Wu, Wd, H: int, D: int, N_mlp: int, scale: float,
          intermediates: bool = False, nthreads: int | None = None):
    X = np.ascontiguousarray(X, dtype=np.float16)
    M, dm = X.shape
    HD = H * D
    Ws = [np.ascontiguousarray(w, dtype=np.uint8) for w in (Wq, Wk, Wv, Wo, Wg, Wu, Wd)]
    out = np.empty((M, dm), np.float16)
    inter = {
        "Q": np.empty((H, M, D), np.float16), "K": np.empty((H, M, D), np.float16),
        "V": np.empty((H, M, D), np.float16), "O": np.empty((M, HD), np.float16),
        "Xmid": np.empty((M, dm), np.float16), "S": np.empty((M, N_mlp), np.float16),
    }
    ip = [(_p(inter[k]) if intermediates else None) for k in ("Q", "K", "V", "O", "Xmid", "S")]
    rc = lib().orc_layer(fmt, _p(X), *[_p(w) for w in Ws], _p(out), M, dm, H, D, N_mlp, scale, *ip,
                         nthreads or threads())
    assert rc == 0, rc
    return (out, inter) if intermediates else out


def attention_gqa(Q, K, V, scale: float, o_token_major: bool = False, nthreads: int | None = None):
    """Q [H, M, D], K/V [Hkv, M, D]: query head h reads KV head h // (H // Hkv)."""
    Q, K, V = (np.ascontiguousarray(a, dtype=np.float16) for a in (Q, K, V))
    H, M, D = Q.shape
    out = np.empty((M, H * D) if o_token_major else (H, M, D), np.float16)
    rc = lib().orc_attention_gqa(_p(Q), _p(K), _p(V), _p(out), H, K.shape[0], M, D, scale, int(o_token_major),
                                 nthreads or threads())
    assert rc == 0, rc
    return out


def attention_q8_0_gqa(Q, Kq, Vq, Hkv: int, scale: float, o_token_major: bool = False,
                       nthreads: int | None = None):
    Q = np.ascontiguousarray(Q, dtype=np.float16)
    H, M, D = Q.shape
    Kq = np.ascontiguousarray(Kq, dtype=np.uint8)
    Vq = np.ascontiguousarray(Vq, dtype=np.uint8)
    out = np.empty((M, H * D) if o_token_major else (H, M, D), np.float16)
    rc = lib().orc_attention_q8_0_gqa(_p(Q), _p(Kq), _p(Vq), _p(out), H, Hkv, M, D, scale, int(o_token_major),
                                      nthreads or threads())
    assert rc == 0, rc
    return out


def rmsnorm(X, w, eps: float = 1e-5, norm_type: int = 1) -> np.ndarray:
    X = np.ascontiguousarray(X, dtype=np.float16)
    w = np.ascontiguousarray(w, dtype=np.float16)
    M, D = X.shape
    out = np.empty_like(X)
    rc = lib().orc_rmsnorm(_p(X), _p(w), _p(out), M, D, eps, norm_type)
    assert rc == 0, rc
    return out


def rope(T, theta: float = 10000.0, offset: int = 0, traditional: bool = False) -> np.ndarray:
    """RoPE of T [H, M, D] (returns a new array)."""
    T = np.array(T, dtype=np.float16, copy=True, order="C")
    H, M, D = T.shape
    rc = lib().orc_rope(_p(T), H, M, D, theta, offset, int(traditional))
    assert rc == 0, rc
    return T


def layer_ex(fmt: int, X, w_attn, Wq, Wk, Wv, Wo, w_ffn, Wg, Wu, Wd, Hq: int, Hkv: int, D: int, N_mlp: int,
             scale: float, norm_type: int = 1, eps: float = 1e-5, rope: bool = True, theta: float = 10000.0,
             offset: int = 0, traditional: bool = False, nthreads: int | None = None) -> np.ndarray:
    X = np.ascontiguousarray(X, dtype=np.float16)
    M, dm = X.shape
    na = None if w_attn is None else np.ascontiguousarray(w_attn, dtype=np.float16)
    nf = None if w_ffn is None else np.ascontiguousarray(w_ffn, dtype=np.float16)
    Ws = [np.ascontiguousarray(w, dtype=np.uint8) for w in (Wq, Wk, Wv, Wo, Wg, Wu, Wd)]
    out = np.empty((M, dm), np.float16)
    rc = lib().orc_layer_ex(fmt, _p(X), _p(na) if na is not None else None, *[_p(w) for w in Ws[:4]],
                            _p(nf) if nf is not None else None, *[_p(w) for w in Ws[4:]], _p(out), M, dm, Hq, Hkv,
                            D, N_mlp, scale, norm_type, eps, int(rope), theta, offset, int(traditional),
                            nthreads or threads())
    assert rc == 0, rc
    return out


def attention_q8_0_rows(Qr, Kq, Vq, pos, M: int, Hkv: int, scale: float, o_token_major: bool = False,
                        nthreads: int | None = None) -> np.ndarray:
    """Causal attention over the dequantized Q8_0 K/V [Hkv, M, D] for the query
    positions `pos` only.  Qr [H, len(pos), D] holds those queries; the result
    is [H, len(pos), D] (or [len(pos), H*D] token-major)."""
    return attention_rows(Qr, dequantize_q8_0(Kq), dequantize_q8_0(Vq), pos, M, Hkv, scale, o_token_major, nthreads)


def attention_rows(Qr, Kd, Vd, pos, M: int, Hkv: int, scale: float, o_token_major: bool = False,
                   nthreads: int | None = None) -> np.ndarray:
    """attention_q8_0_rows on K / V already in fp16 (e.g. dequantized once)."""
    Qr = np.ascontiguousarray(Qr, dtype=np.float16)
    H, nr, D = Qr.shape
    pos = np.ascontiguousarray(pos, dtype=np.uint32)
    assert pos.size == nr
    Kd = np.ascontiguousarray(Kd, dtype=np.float16)
    Vd = np.ascontiguousarray(Vd, dtype=np.float16)
    assert Kd.size == Hkv * M * D
    out = np.empty((nr, H * D) if o_token_major else (H, nr, D), np.float16)
    rc = lib().orc_attention_rows(_p(Qr), _p(Kd), _p(Vd), _p(out), _p(pos), nr, H, Hkv, M, D, scale,
                                  int(o_token_major), nthreads or threads())
    assert rc == 0, rc
    return out


def layer_ex_rows(fmt: int, X, w_attn, Wq, Wk, Wv, Wo, w_ffn, Wg, Wu, Wd, pos, Hq: int, Hkv: int, D: int,
                  N_mlp: int, scale: float, norm_type: int = 1, eps: float = 1e-5, rope: bool = False,
                  theta: float = 10000.0, offset: int = 0, traditional: bool = False,
                  nthreads: int | None = None) -> np.ndarray:
    """Rows `pos` of layer_ex (the plain router layer when w_attn = w_ffn = None,
    rope = False and Hkv = Hq): [len(pos), d_model]."""
    X = np.ascontiguousarray(X, dtype=np.float16)
    M, dm = X.shape
    pos = np.ascontiguousarray(pos, dtype=np.uint32)
    na = None if w_attn is None else np.ascontiguousarray(w_attn, dtype=np.float16)
    nf = None if w_ffn is None else np.ascontiguousarray(w_ffn, dtype=np.float16)
    Ws = [np.ascontiguousarray(w, dtype=np.uint8) for w in (Wq, Wk, Wv, Wo, Wg, Wu, Wd)]
    out = np.empty((pos.size, dm), np.float16)
    rc = lib().orc_layer_ex_rows(fmt, _p(X), _p(na) if na is not None else None, *[_p(w) for w in Ws[:4]],
                                 _p(nf) if nf is not None else None, *[_p(w) for w in Ws[4:]], _p(out), _p(pos),
                                 pos.size, M, dm, Hq, Hkv, D, N_mlp, scale, norm_type, eps, int(rope), theta,
                                 offset, int(traditional), nthreads or threads())
    assert rc == 0, rc
    return out
