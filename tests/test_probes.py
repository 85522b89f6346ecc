"""On-device roofline probes (m4_probe_hbm_bandwidth, m4_probe_mfma_f16).

The reference measures its own memory-bandwidth and FMA ceilings
(quant_router_kernels.metal:71-104, timed by bench_universal_router.mm:
645-717); the probes here do the same for HBM and the matrix pipe.  CPU:
argument validation, which returns before any device call.  GPU: the
measured figures are positive and physically plausible for an MI355X
(read bandwidth below the 8 TB/s HBM3E peak, matrix throughput below the
2.5 PF dense fp16 peak, shader clock between 0.5 and 3 GHz).
"""
from __future__ import annotations

import ctypes

import pytest

import m4_bridge


@pytest.fixture(scope="module")
def lib(libpath):
    return m4_bridge.load_library(libpath)


def test_probe_arguments_are_checked_before_device_work(lib):
    r, c = ctypes.c_double(), ctypes.c_double()
    assert lib.m4_probe_hbm_bandwidth(1 << 26, 1, None, ctypes.byref(c)) == -2
    assert lib.m4_probe_hbm_bandwidth(1 << 26, 1, ctypes.byref(r), None) == -2
    assert lib.m4_probe_hbm_bandwidth(1 << 10, 1, ctypes.byref(r), ctypes.byref(c)) == -4  # below 1 MiB
    assert lib.m4_probe_hbm_bandwidth(1 << 26, 0, ctypes.byref(r), ctypes.byref(c)) == -4
    t, g = ctypes.c_double(), ctypes.c_double()
    assert lib.m4_probe_mfma_f16(4096, 1, None, ctypes.byref(g)) == -2
    assert lib.m4_probe_mfma_f16(4096, 1, ctypes.byref(t), None) == -2
    assert lib.m4_probe_mfma_f16(16, 1, ctypes.byref(t), ctypes.byref(g)) == -4  # fewer than 64 rounds
    assert lib.m4_probe_mfma_f16(4096, 0, ctypes.byref(t), ctypes.byref(g)) == -4
    assert lib.m4_probe_mfma_f16_random(4096, 1, None, ctypes.byref(g)) == -2
    assert lib.m4_probe_mfma_f16_random(4098, 1, ctypes.byref(t), ctypes.byref(g)) == -4  # not a multiple of 4
    assert lib.m4_probe_mfma_f16_random(16, 1, ctypes.byref(t), ctypes.byref(g)) == -4


@pytest.mark.gpu
def test_probes_measure_plausible_ceilings(bridge):
    lib = bridge.lib
    r, c = ctypes.c_double(), ctypes.c_double()
    # 1 GiB: well past the 256 MB Infinity Cache, so the read pass cannot be
    # served from it after the copy pass
    print("probe: hbm 1 GiB x 2", flush=True)
    assert lib.m4_probe_hbm_bandwidth(1 << 30, 2, ctypes.byref(r), ctypes.byref(c)) == 0
    assert 500.0 < r.value < 8000.0, r.value   # GB/s, below the HBM3E peak
    assert 500.0 < c.value < 8000.0, c.value
    t, g = ctypes.c_double(), ctypes.c_double()
    print("probe: mfma 1024 rounds x 2", flush=True)
    assert lib.m4_probe_mfma_f16(1024, 2, ctypes.byref(t), ctypes.byref(g)) == 0
    assert 100.0 < t.value < 2500.0, t.value   # TFLOP/s, below the dense fp16 peak
    assert 0.5 < g.value < 3.0, g.value        # GHz
    tr, gr = ctypes.c_double(), ctypes.c_double()
    print("probe: mfma random operands 1024 rounds x 2", flush=True)
    assert lib.m4_probe_mfma_f16_random(1024, 2, ctypes.byref(tr), ctypes.byref(gr)) == 0
    assert 100.0 < tr.value < 2500.0, tr.value
    assert 0.5 < gr.value < 3.0, gr.value
