"""Benchmark of the MI355X quantization-router prefill path.

Metric: ms + effective TFLOPS per quantized projection at
M=33/128/2048, K=4096.  One JSON line on stdout.

  value         effective TFLOP/s (2*M*N*K / t) of the BASELINE headline
                configuration configs[1]: MLX-4bit affine, M=128, K=4096,
                N=14336 (g64 groups repacked into the router's MLX_4BIT blocks)
  per_config    ms / TFLOP/s / GB/s and roofline fractions for every BASELINE
                configuration (Q4_0 M=33, MLX M=128, Q4_K M=2048, ternary
                M=129, the Llama-3.2-1B-shaped layer and its SwiGLU and
                attention components)
  roofline      the dominant kernel of the headline configuration, timed with
                HIP events on the stream it runs on
  cpu_baseline  the CPU oracle (restated reference gold path) on a bounded row
                sample of the headline configuration, on this host's cores;
                per_config entries of cfg1, cfg3, cfg4, SwiGLU and attention
                carry their own (half the time budget each)

A step is one projection (or one layer) over one batch.  W untimed warmup
steps run eagerly; the K timed steps are captured once into a HIP graph and
replayed, so the timed region holds back-to-back kernels with no host launch
gaps.  Each timed region is one replay of exactly K steps between two events
on the stream the kernels run on; it is repeated --repeats times (default 5)
and the median per-step time is reported (single replays vary by a few
percent).  Weights rotate over enough device copies (> 512 MB) that every step
reads them from HBM, not from the 256 MB Infinity Cache.  All inputs are
resident in HBM before timing starts.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
PKG = ROOT / "m4-prefill-engine_amd"
sys.path.insert(0, str(PKG))

PEAK_MFMA_TFLOPS = 2500.0   # MI355X dense fp16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
ROTATE_BYTES = 512 << 20


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--configs", default="all", help="comma list of config names or 'all'")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--repeats", type=int, default=5, help="timed replays of the K steps (median reported)")
    ap.add_argument("--no-probes", action="store_true", help="skip the on-device HBM / MFMA ceiling probes")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    return ap.parse_args()


class Timer:
    """Times `steps` calls of fn(i) on the current stream: eager warmup, then a
    HIP-graph capture of the timed steps replayed between two events."""

    def __init__(self, bridge, warmup: int, steps: int, repeats: int = 5):
        self.b, self.warmup, self.steps, self.repeats = bridge, warmup, steps, repeats

    def run(self, fn) -> float:
        import torch

        s = torch.cuda.current_stream()
        self.b.lib.m4_bridge_set_stream(s.cuda_stream)
        for i in range(self.warmup):
            fn(i)
        torch.cuda.synchronize()
        mode = "graph"
        g = torch.cuda.CUDAGraph()
        try:
            cap = torch.cuda.Stream()
            with torch.cuda.graph(g, stream=cap):
                self.b.lib.m4_bridge_set_stream(torch.cuda.current_stream().cuda_stream)
                for i in range(self.steps):
                    fn(i)
            self.b.lib.m4_bridge_set_stream(s.cuda_stream)
            g.replay()  # upload; untimed
            torch.cuda.synchronize()
        except Exception:  # capture unsupported: eager timing
            mode = "eager"
            self.b.lib.m4_bridge_set_stream(s.cuda_stream)
            torch.cuda.synchronize()
        # REPEATS timed replays of the K steps; the median is reported (one
        # replay alone varies by a few percent from run to run)
        times = []
        for _ in range(self.repeats):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record(s)
            if mode == "graph":
                g.replay()
            else:
                for i in range(self.steps):
                    fn(i)
            e1.record(s)
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1) / self.steps)
        self.mode = mode
        self.spread = (min(times), max(times))
        return sorted(times)[len(times) // 2]  # ms per step


def rotated(t, nbytes_each: int):
    """Device copies of t so that the set spans > ROTATE_BYTES."""
    import torch

    n = max(2, min(64, math.ceil(ROTATE_BYTES / max(1, nbytes_each))))
    return [t] + [t.clone() for _ in range(n - 1)]


def rotated_sets(Ws):
    """Copies of a layer's weight set so that the sets span > ROTATE_BYTES."""
    total = sum(w.numel() for w in Ws)
    n = max(2, min(64, math.ceil(ROTATE_BYTES / max(1, total))))
    return [Ws] + [[w.clone() for w in Ws] for _ in range(n - 1)]


def check(rc: int, what: str):
    if rc != 0:
        raise RuntimeError(f"{what} failed with status {rc}")


def bench_projection(b, timer, name, fmt, M, K, N, seed):
    import torch

    import synth

    Xn = synth.activations(M, K, seed)
    X = torch.from_numpy(Xn).cuda()
    Wn = (synth.quantized_weights(fmt, N, K, seed + 1) if fmt < 4 or fmt == synth.MLX_4BIT_G64
          else synth.random_blocks(fmt, N, K, seed + 1))
    W0 = torch.from_numpy(Wn).cuda()
    Ws = rotated(W0, W0.numel())
    Y = torch.empty(M, N, dtype=torch.float16, device="cuda")
    lib = b.lib
    xp, yp, xb, yb = X.data_ptr(), Y.data_ptr(), X.numel() * 2, Y.numel() * 2
    wps = [w.data_ptr() for w in Ws]
    wb = W0.numel()

    # formats beyond the reference's 0..5 go through the kernel-name entry point
    fn = lib.m4_bridge_dispatch_gemm if fmt < 6 else lib.m4_bridge_dispatch_router_gemm

    def step(i):
        check(fn(xp, xb, wps[i % len(wps)], wb, yp, yb, fmt, M, K, N), name)

    ms = timer.run(step)
    flops = 2.0 * M * N * K
    bytes_ = X.numel() * 2 + wb + Y.numel() * 2
    tf = flops / (ms * 1e-3) / 1e12
    gbs = bytes_ / (ms * 1e-3) / 1e9
    return {
        "name": name, "format": fmt, "M": M, "K": K, "N": N, "ms": round(ms, 5), "tflops": round(tf, 2),
        "gbs": round(gbs, 1), "frac_mfma": round(tf / PEAK_MFMA_TFLOPS, 4), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
        "flops": flops, "bytes": bytes_, "weight_copies": len(Ws), "timing": timer.mode,
    }, (Xn, Wn)


def bench_host_buffers(b, name, fmt, M, K, N, seed, calls: int = 10):
    """The headline projection with host buffers (the reference's callers pass
    unified-memory host pointers): every call copies X and W in over PCIe,
    runs, and copies Y back at synchronize.  Eager, wall-clock per call; this
    is the PCIe-inclusive rate, never `value`.  Pageable (numpy) and pinned
    (torch pin_memory) host memory."""
    import torch

    import synth

    Xn = synth.activations(M, K, seed)
    Wn = synth.quantized_weights(fmt, N, K, seed + 1)
    out = {"name": name, "format": fmt, "M": M, "K": K, "N": N, "calls": calls}
    bytes_ = Xn.nbytes + Wn.nbytes + M * N * 2
    for kind in ("pageable", "pinned"):
        if kind == "pageable":
            X, W, Y = Xn, Wn, np.empty((M, N), np.float16)
            ptr = lambda a: a.ctypes.data  # noqa: E731
        else:
            X = torch.from_numpy(Xn).pin_memory()
            W = torch.from_numpy(Wn).pin_memory()
            Y = torch.empty(M, N, dtype=torch.float16).pin_memory()
            ptr = lambda a: a.data_ptr()  # noqa: E731
        xp, wp, yp = ptr(X), ptr(W), ptr(Y)

        def call():
            check(b.lib.m4_bridge_dispatch_gemm(xp, Xn.nbytes, wp, Wn.nbytes, yp, M * N * 2, fmt, M, K, N), name)
            b.lib.m4_bridge_synchronize()

        for _ in range(2):
            call()
        t0 = time.perf_counter()
        for _ in range(calls):
            call()
        ms = (time.perf_counter() - t0) * 1e3 / calls
        out[f"{kind}_ms"] = round(ms, 4)
        out[f"{kind}_gbs"] = round(bytes_ / (ms * 1e-3) / 1e9, 1)
        out[f"{kind}_tflops"] = round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 2)
    out["bytes_over_pcie"] = bytes_
    return out


def bench_swiglu(b, timer, M, K, N, seed):
    import torch

    import synth

    Xn, Wgn, Wun = synth.activations(M, K, seed), synth.quantized_weights(0, N, K, seed + 1), \
        synth.quantized_weights(0, N, K, seed + 2)
    X, Wg, Wu = (torch.from_numpy(a).cuda() for a in (Xn, Wgn, Wun))
    Out = torch.empty(M, N, dtype=torch.float16, device="cuda")
    lib = b.lib
    # gate + up weights rotate over copies spanning > 512 MB (HBM, not MALL)
    pairs = list(zip(rotated(Wg, 2 * Wg.numel()), rotated(Wu, 2 * Wu.numel())))
    wb = Wg.numel()

    def step(i):
        g, u = pairs[i % len(pairs)]
        check(lib.m4_bridge_dispatch_swiglu(X.data_ptr(), X.numel() * 2, g.data_ptr(), wb, u.data_ptr(), wb,
                                            Out.data_ptr(), Out.numel() * 2, 0, M, N, K), "swiglu")

    ms = timer.run(step)
    flops = 4.0 * M * N * K + 4.0 * M * N  # brick3_swiglu_bench.mm:489
    tf = flops / (ms * 1e-3) / 1e12
    return {"name": "swiglu_q4_0", "M": M, "K": K, "N_mlp": N, "ms": round(ms, 5), "tflops": round(tf, 2),
            "frac_mfma": round(tf / PEAK_MFMA_TFLOPS, 4), "weight_copies": len(pairs), "timing": timer.mode}, \
        (Xn, Wgn, Wun)


def bench_attention(b, timer, H, M, D, seed):
    import torch

    rng = np.random.default_rng(seed)
    Qn, Kn, Vn = (rng.standard_normal((H, M, D)).astype(np.float16) for _ in range(3))
    Q, Kf, Vf = (torch.from_numpy(a).cuda() for a in (Qn, Kn, Vn))
    nb = H * M * D // 32
    Kq = torch.empty(nb * 34, dtype=torch.uint8, device="cuda")
    Vq = torch.empty(nb * 34, dtype=torch.uint8, device="cuda")
    lib = b.lib
    check(lib.m4_bridge_quantize_kv_q8_0(Kf.data_ptr(), Kf.numel() * 2, Kq.data_ptr(), Kq.numel(), nb), "q8")
    check(lib.m4_bridge_quantize_kv_q8_0(Vf.data_ptr(), Vf.numel() * 2, Vq.data_ptr(), Vq.numel(), nb), "q8")
    O = torch.empty(H, M, D, dtype=torch.float16, device="cuda")
    args = (Q.data_ptr(), Q.numel() * 2, Kq.data_ptr(), Kq.numel(), Vq.data_ptr(), Vq.numel(), O.data_ptr(),
            O.numel() * 2, H, M, D, 1.0 / math.sqrt(D), 0)

    def step(i):
        check(lib.m4_bridge_dispatch_flash_attn_q8_0(*args), "attention")

    ms = timer.run(step)
    flops = 2.0 * H * M * (M + 1) * D  # brick4_attn_bench.mm:475
    tf = flops / (ms * 1e-3) / 1e12
    return {"name": "flash_attn_q8_0", "H": H, "M": M, "D": D, "ms": round(ms, 5), "tflops": round(tf, 2),
            "frac_mfma": round(tf / PEAK_MFMA_TFLOPS, 4), "timing": timer.mode}, (Qn, Kn, Vn)


def bench_layer(b, timer, M, dm, H, D, Nm, seed):
    import torch

    import synth

    X = torch.from_numpy(synth.activations(M, dm, seed)).cuda()
    shapes = [(H * D, dm)] * 3 + [(dm, H * D), (Nm, dm), (Nm, dm), (dm, Nm)]
    Ws = [torch.from_numpy(synth.quantized_weights(0, n, k, seed + 1 + i)).cuda() for i, (n, k) in enumerate(shapes)]
    Xo = torch.empty(M, dm, dtype=torch.float16, device="cuda")
    lib = b.lib
    sets = rotated_sets(Ws)

    def step(i):
        ptrs = [X.data_ptr()] + [w.data_ptr() for w in sets[i % len(sets)]] + [Xo.data_ptr()]
        check(lib.m4_bridge_prefill_layer(*ptrs, 0, M, dm, H, D, Nm, 1.0 / math.sqrt(D)), "layer")

    ms = timer.run(step)
    HD = H * D
    flops = 2.0 * M * dm * HD * 4 + 2.0 * M * dm * Nm * 3 + 2.0 * H * M * (M + 1) * D
    tf = flops / (ms * 1e-3) / 1e12
    return {"name": "layer_llama32_1b_q4_0_q8kv", "M": M, "d_model": dm, "H": H, "D": D, "N_mlp": Nm,
            "weight_copies": len(sets), "ms": round(ms, 5), "tflops": round(tf, 2), "frac_mfma": round(tf / PEAK_MFMA_TFLOPS, 4),
            "tokens_per_s": round(M / (ms * 1e-3), 1), "timing": timer.mode}


def bench_layer_ex(b, timer, M, dm, Hq, Hkv, D, Nm, seed):
    """The full Llama-3.2-1B block (RMSNorm, RoPE, grouped-query attention with
    Hkv = 8, Q4_0 weights, Q8_0 KV) through m4_bridge_prefill_layer_ex."""
    import torch

    import synth

    X = torch.from_numpy(synth.activations(M, dm, seed)).cuda()
    shapes = [(Hq * D, dm), (Hkv * D, dm), (Hkv * D, dm), (dm, Hq * D), (Nm, dm), (Nm, dm), (dm, Nm)]
    Ws = [torch.from_numpy(synth.quantized_weights(0, n, k, seed + 1 + i)).cuda() for i, (n, k) in enumerate(shapes)]
    na = torch.ones(dm, dtype=torch.float16, device="cuda")
    nf = torch.ones(dm, dtype=torch.float16, device="cuda")
    Xo = torch.empty(M, dm, dtype=torch.float16, device="cuda")
    lib = b.lib
    sets = rotated_sets(Ws)

    def step(i):
        ws = sets[i % len(sets)]
        ptrs = ([X.data_ptr(), na.data_ptr()] + [w.data_ptr() for w in ws[:4]] + [nf.data_ptr()] +
                [w.data_ptr() for w in ws[4:]] + [Xo.data_ptr()])
        check(lib.m4_bridge_prefill_layer_ex(*ptrs, 0, M, dm, Hq, Hkv, D, Nm, 1.0 / math.sqrt(D), 1, 1e-5, 1,
                                             500000.0, 0, 0), "layer_ex")

    ms = timer.run(step)
    flops = (2.0 * M * dm * (Hq + 2 * Hkv) * D + 2.0 * M * Hq * D * dm + 2.0 * M * dm * Nm * 3 +
             2.0 * Hq * M * (M + 1) * D)
    tf = flops / (ms * 1e-3) / 1e12
    return {"name": "block_llama32_1b_gqa8_rmsnorm_rope", "M": M, "d_model": dm, "Hq": Hq, "Hkv": Hkv, "D": D,
            "N_mlp": Nm, "weight_copies": len(sets), "ms": round(ms, 5), "tflops": round(tf, 2), "frac_mfma": round(tf / PEAK_MFMA_TFLOPS, 4),
            "tokens_per_s": round(M / (ms * 1e-3), 1), "timing": timer.mode}


def bench_rmsnorm(b, timer, M, D, seed):
    import torch

    X = torch.randn(M, D, dtype=torch.float16, device="cuda")
    w = torch.ones(D, dtype=torch.float16, device="cuda")
    Y = torch.empty_like(X)
    lib = b.lib
    args = (X.data_ptr(), X.numel() * 2, w.data_ptr(), D * 2, Y.data_ptr(), Y.numel() * 2, M, D, 1e-5, 1)

    def step(i):
        check(lib.m4_bridge_rmsnorm(*args), "rmsnorm")

    ms = timer.run(step)
    gbs = (2.0 * M * D * 2 + D * 2) / (ms * 1e-3) / 1e9
    return {"name": "rmsnorm", "M": M, "D": D, "ms": round(ms, 5), "gbs": round(gbs, 1),
            "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "timing": timer.mode}


def bench_rope(b, timer, H, M, D, seed):
    import torch

    T = torch.randn(H, M, D, dtype=torch.float16, device="cuda")
    lib = b.lib

    def step(i):
        check(lib.m4_bridge_rope(T.data_ptr(), T.numel() * 2, H, M, D, 500000.0, 0, 0), "rope")

    ms = timer.run(step)
    gbs = 2.0 * T.numel() * 2 / (ms * 1e-3) / 1e9
    return {"name": "rope", "H": H, "M": M, "D": D, "ms": round(ms, 5), "gbs": round(gbs, 1),
            "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "timing": timer.mode}


def bench_fp16_reference(timer, name, M, K, N):
    """Calibration point, not a router kernel: the vendor library's unquantized
    fp16 GEMM (torch.matmul -> hipBLASLt) of the same shape, weights rotated the
    same way.  It shows what an fp16 GEMM without any decode reaches here."""
    import torch

    X = torch.randn(M, K, dtype=torch.float16, device="cuda")
    W0 = (torch.randn(N, K, dtype=torch.float16, device="cuda") * 0.02)
    Ws = rotated(W0, W0.numel() * 2)
    Y = torch.empty(M, N, dtype=torch.float16, device="cuda")

    def step(i):
        torch.matmul(X, Ws[i % len(Ws)].t(), out=Y)

    ms = timer.run(step)
    tf = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    return {"name": name, "M": M, "K": K, "N": N, "ms": round(ms, 5), "tflops": round(tf, 2),
            "frac_mfma": round(tf / PEAK_MFMA_TFLOPS, 4), "timing": timer.mode,
            "note": "unquantized fp16 torch.matmul (hipBLASLt) reference, not part of the router path"}


def bench_copy(timer, nbytes: int):
    """Device-to-device copy of a known size: the calibration point for the
    FETCH_SIZE / WRITE_SIZE counters (bytes moved = nbytes read + nbytes written)."""
    import torch

    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)

    def step(i):
        dst.copy_(src)

    ms = timer.run(step)
    return {"name": "copy_calib", "bytes": nbytes, "ms": round(ms, 5),
            "gbs": round(2.0 * nbytes / (ms * 1e-3) / 1e9, 1), "timing": timer.mode}


TRAFFIC_PROFILE = ROOT / "profiles" / "hbm_traffic_router_kernels.md"
# Sources of the headline kernel: a traffic figure measured on other
# versions of these files is stale and is not reported.
KERNEL_SOURCES = ("qr_gemm.hip", "qr_gemm_host.hip", "qr_gemm_shapes.h", "qr_decode.h", "qr_device.h",
                  "qr_formats.h", "qr_kernels.h")


def kernel_digest() -> str:
    import hashlib

    h = hashlib.sha256()
    for name in KERNEL_SOURCES:
        h.update((PKG / "csrc" / name).read_bytes())
    return h.hexdigest()[:16]


def traffic_from_profile(name: str):
    """HBM bytes per launch of the headline kernel, as measured by the
    rocprofv3 FETCH_SIZE / WRITE_SIZE runs summarised in TRAFFIC_PROFILE
    (copy-calibrated), with the digest of the kernel sources it was measured
    on.  Returns (bytes or None, note)."""
    try:
        lines = TRAFFIC_PROFILE.read_text().splitlines()
    except OSError:
        return None, "no traffic profile"
    digest = next((ln.split(":", 1)[1].strip() for ln in lines if ln.startswith("kernel_sources_sha256_16:")), None)
    value = next((int(ln.split(":", 1)[1]) for ln in lines if ln.startswith(f"traffic_bytes_per_launch {name}:")),
                 None)
    if value is None:
        return None, "no traffic figure for " + name
    now = kernel_digest()
    if digest != now:
        return None, f"stale: profile measured on kernel sources {digest}, these are {now}"
    return value, f"rocprofv3 FETCH_SIZE + WRITE_SIZE, kernel sources {now}"


def probes(b):
    """On-device ceilings (the reference's roofline probes): HBM read and copy
    GB/s over 1 GiB, dense fp16 MFMA TFLOP/s and the clock it ran at, with
    low-entropy and with random operands."""
    import ctypes

    r, c, t, g = (ctypes.c_double() for _ in range(4))
    out = {}
    if b.lib.m4_probe_hbm_bandwidth(1 << 30, 5, ctypes.byref(r), ctypes.byref(c)) == 0:
        out.update(hbm_read_gbs=round(r.value, 1), hbm_copy_gbs=round(c.value, 1),
                   hbm_read_frac_of_peak=round(r.value / PEAK_HBM_GBS, 4))
    if b.lib.m4_probe_mfma_f16(4096, 5, ctypes.byref(t), ctypes.byref(g)) == 0:
        out.update(mfma_f16_tflops=round(t.value, 1), mfma_clock_ghz=round(g.value, 3),
                   mfma_frac_of_peak=round(t.value / PEAK_MFMA_TFLOPS, 4))
    # random operands: the ceiling real data reaches (power-limited clock)
    if b.lib.m4_probe_mfma_f16_random(4096, 5, ctypes.byref(t), ctypes.byref(g)) == 0:
        out.update(mfma_f16_random_tflops=round(t.value, 1), mfma_random_clock_ghz=round(g.value, 3),
                   mfma_random_frac_of_peak=round(t.value / PEAK_MFMA_TFLOPS, 4))
    return out


def _oracle():
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle_bindings as ob

    return ob


def cpu_rows(run_rows, M: int, seconds: float, row_work=None):
    """Runs run_rows(rows) on growing, evenly spread row samples of an M-row
    job until ~`seconds` of CPU work, and extrapolates the time of the whole
    job by work: rows, or sum(row_work(i)) where rows cost unequal work
    (causal attention: row i attends i + 1 keys).  Returns (seconds spent,
    estimated seconds for all M rows, rows run)."""
    work = (lambda r: float(np.sum(row_work(r)))) if row_work else (lambda r: float(len(r)))
    full = work(np.arange(M))
    n, spent, done, rows_run = 1, 0.0, 0.0, 0
    while spent < seconds:
        rows = np.unique(np.linspace(0, M - 1, min(n, M)).astype(np.int64))
        t0 = time.perf_counter()
        run_rows(rows)
        spent += time.perf_counter() - t0
        done += work(rows)
        rows_run += len(rows)
        n *= 2
    return spent, spent / done * full, rows_run


def cpu_entry(value_tf: float, spent: float, est: float, rows: int, what: str, threads: int):
    return {"value": round(value_tf, 6), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"{rows} rows of {what}, evenly spread over M and repeated in growing blocks, "
                      f"{spent:.1f} s of CPU work, extrapolated to the whole job by its row work; "
                      f"double accumulation, one task per row",
            "ms_full_est": round(est * 1e3, 1)}


def cpu_projection(fmt, X, Wn, N, seconds: float, what: str):
    """The oracle (CPU restatement of the reference's gold projection,
    cpu_gold_reference.h:15-198) on a row sample of a projection."""
    ob = _oracle()
    M, K = X.shape
    threads = ob.threads()
    spent, est, rows = cpu_rows(lambda r: ob.gemm(fmt, np.ascontiguousarray(X[r]), Wn, N, nthreads=threads), M,
                                seconds)
    return cpu_entry(2.0 * M * N * K / est / 1e12, spent, est, rows, what, threads)


def cpu_swiglu(X, Wg, Wu, N, seconds: float):
    """The SwiGLU gold (brick3_swiglu_bench.mm:49-99) on a row sample."""
    ob = _oracle()
    M, K = X.shape
    threads = ob.threads()
    spent, est, rows = cpu_rows(lambda r: ob.swiglu(0, np.ascontiguousarray(X[r]), Wg, Wu, N, nthreads=threads), M,
                                seconds)
    return cpu_entry((4.0 * M * N * K + 4.0 * M * N) / est / 1e12, spent, est, rows,
                     f"the SwiGLU M={M} K={K} N={N}", threads)


def cpu_attention(Q, K, V, seconds: float):
    """The causal attention gold over the Q8_0 cache (brick4_attn_bench.mm:
    70-119, on the dequantized K / V as brick4_attn_bench.mm:241-255) on a
    query-row sample; row i costs i + 1 keys."""
    ob = _oracle()
    H, M, D = Q.shape
    threads = ob.threads()
    # the Q8_0 cache, dequantized once before timing (the reference's gold
    # runs on the dequantized K / V)
    Kd, Vd = (ob.dequantize_q8_0(ob.quantize_q8_0(a)).reshape(H, M, D) for a in (K, V))
    scale = 1.0 / math.sqrt(D)
    run = lambda r: ob.attention_rows(np.ascontiguousarray(Q[:, r]), Kd, Vd, r, M, H, scale,  # noqa: E731
                                      nthreads=threads)
    spent, est, rows = cpu_rows(run, M, seconds, row_work=lambda r: (np.asarray(r) + 1) * H)
    return cpu_entry(2.0 * H * M * (M + 1) * D / est / 1e12, spent, est, rows,
                     f"causal attention H={H} M={M} D={D} (all heads per sampled query row)", threads)


def main():
    a = parse()
    if a.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 (multi-GPU sharding is "
                                   "design-only, see DESIGN.md)"}))
        sys.exit(2)
    import torch

    import m4_bridge

    b = m4_bridge.HIPBridge.get_instance(os.environ.get("M4_BRIDGE_LIB_PATH") or PKG / "libm4_bridge.so")
    assert b.init(), b.last_error()
    timer = Timer(b, a.warmup, a.steps, a.repeats)
    want = None if a.configs == "all" else set(a.configs.split(","))

    def on(name):
        return want is None or name in want

    per = {}
    head_inputs = None
    cpu_inputs = {}
    if on("cfg2_mlx_m128"):
        per["cfg2_mlx_m128"], head_inputs = bench_projection(b, timer, "cfg2_mlx_m128", 1, 128, 4096, 14336, 20)
    if on("cfg2_mlx_g64_m128"):
        per["cfg2_mlx_g64_m128"], _ = bench_projection(b, timer, "cfg2_mlx_g64_m128", 8, 128, 4096, 14336, 20)
    if on("cfg1_q4_0_m33"):
        per["cfg1_q4_0_m33"], cpu_inputs["cfg1_q4_0_m33"] = bench_projection(b, timer, "cfg1_q4_0_m33", 0, 33, 4096,
                                                                              4096, 10)
    if on("cfg3_q4_k_m2048"):
        per["cfg3_q4_k_m2048"], cpu_inputs["cfg3_q4_k_m2048"] = bench_projection(b, timer, "cfg3_q4_k_m2048", 2, 2048,
                                                                                  4096, 4096, 30)
    if on("cfg4_ternary_m129"):
        per["cfg4_ternary_m129"], cpu_inputs["cfg4_ternary_m129"] = bench_projection(b, timer, "cfg4_ternary_m129", 3,
                                                                                      129, 2048, 8192, 40)
    # every router format at the north-star shape M = 2048, K = 4096 (Q4_K is
    # cfg3 above); the 3/5-bit formats only when named
    for fmt, tag in ((0, "q4_0"), (1, "mlx"), (3, "ternary"), (4, "var_rate"), (5, "exl3")):
        name = f"m2048_k4096_{tag}"
        if (want is None and fmt < 4) or (want is not None and name in want):
            per[name], _ = bench_projection(b, timer, name, fmt, 2048, 4096, 4096, 60 + fmt)
    for name, (M, K, N) in (("ref_fp16_gemm_m128_k4096_n14336", (128, 4096, 14336)),
                            ("ref_fp16_gemm_m2048_k4096_n4096", (2048, 4096, 4096))):
        if on(name):
            per[name] = bench_fp16_reference(timer, name, M, K, N)
    if on("cfg2_host_buffers"):
        per["cfg2_host_buffers"] = bench_host_buffers(b, "cfg2_host_buffers", 1, 128, 4096, 14336, 20)
    if want is not None and "copy_calib" in want:
        per["copy_calib"] = bench_copy(timer, 256 << 20)
    if on("cfg5_swiglu"):
        per["cfg5_swiglu"], cpu_inputs["cfg5_swiglu"] = bench_swiglu(b, timer, 2048, 2048, 8192, 50)
    if on("cfg5_attention"):
        per["cfg5_attention"], cpu_inputs["cfg5_attention"] = bench_attention(b, timer, 32, 2048, 64, 51)
    if on("attention_d128"):  # the same shape at the Llama-3-8B head width
        per["attention_d128"], _ = bench_attention(b, timer, 32, 2048, 128, 56)
    if on("cfg5_layer"):
        per["cfg5_layer"] = bench_layer(b, timer, 2048, 2048, 32, 64, 8192, 52)
    if on("block_full"):
        per["block_full"] = bench_layer_ex(b, timer, 2048, 2048, 32, 8, 64, 8192, 53)
    if on("rmsnorm"):
        per["rmsnorm"] = bench_rmsnorm(b, timer, 2048, 2048, 54)
    if on("rope"):
        per["rope"] = bench_rope(b, timer, 32, 2048, 64, 55)

    head = per.get("cfg2_mlx_m128") or next(iter(per.values()))
    traffic, traffic_note = (traffic_from_profile("cfg2_mlx_m128") if "cfg2_mlx_m128" in per
                             else (None, "headline not run"))
    out = {
        "metric": "ms + effective TFLOPS per quantized projection at M=33/128/2048, K=4096",
        "value": head["tflops"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": head["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: seeded N(0,1) activations, N(0,0.02) weights quantized per BASELINE configs",
        "config": {"workload": "MLX-4bit affine projection M=128 K=4096 N=14336 (BASELINE configs[1])",
                   "M": 128, "K": 4096, "N": 14336, "format": "MLX_4BIT (g64 repacked to 32-blocks)"},
        "roofline": {"bound": "mfma", "achieved": head["tflops"], "peak": PEAK_MFMA_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(head["tflops"] / PEAK_MFMA_TFLOPS, 4), "traffic": traffic,
                     "traffic_note": traffic_note,
                     "kernel": "gemm_rb_kernel<MLX_4BIT, 4, 1, 4, 1, 2> (128x64 tiles, two K groups and a stager wave; one kernel)", "hbm_frac": head.get("frac_hbm")},
        "per_config": per,
    }
    if not a.no_probes:
        out["probes"] = probes(b)
    if not a.no_cpu_baseline:
        # the CPU gold beside each configuration (rank 0, one GPU, bounded samples)
        if head_inputs is not None:
            X, Wn = head_inputs
            out["cpu_baseline"] = cpu_projection(1, X, Wn, 14336, a.cpu_seconds,
                                                 "the headline MLX projection M=128 K=4096 N=14336")
            per["cfg2_mlx_m128"]["cpu_baseline"] = out["cpu_baseline"]
        side = a.cpu_seconds / 2
        for name, fmt, N in (("cfg1_q4_0_m33", 0, 4096), ("cfg3_q4_k_m2048", 2, 4096), ("cfg4_ternary_m129", 3, 8192)):
            if name in cpu_inputs:
                X, Wn = cpu_inputs[name]
                per[name]["cpu_baseline"] = cpu_projection(fmt, X, Wn, N, side, f"{name} (M={X.shape[0]}, "
                                                           f"K={X.shape[1]}, N={N})")
        if "cfg5_swiglu" in cpu_inputs:
            per["cfg5_swiglu"]["cpu_baseline"] = cpu_swiglu(*cpu_inputs["cfg5_swiglu"], 8192, side)
        if "cfg5_attention" in cpu_inputs:
            per["cfg5_attention"]["cpu_baseline"] = cpu_attention(*cpu_inputs["cfg5_attention"], side)
    b.synchronize()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
