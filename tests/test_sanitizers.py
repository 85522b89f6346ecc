"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU).

The host-only sources of the library -- the GGUF parser (qr_gguf.cpp), the
registry (qr_registry.cpp), argument validation and the host-range probe
(qr_host.cpp) -- and the CPU oracle (oracle/oracle.c) are compiled with
-fsanitize=address,undefined -fno-sanitize-recover=all beside the driver
tests/c/sanitize_host.cpp, which feeds the GGUF parser well-formed files,
every truncation, seeded byte flips and garbage from exact-size heap copies,
and calls every oracle entry point on small inputs.  Any report aborts the
driver.  The GGUF parser follows the reference loader's behaviour
(core/weights/gguf_loader.h:46-129).
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "m4-prefill-engine_amd" / "csrc"
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]


def test_host_code_under_asan_ubsan(tmp_path):
    cc, cxx = shutil.which("gcc"), shutil.which("g++")
    if not cc or not cxx:
        pytest.skip("no host C/C++ compiler")
    objs = []
    for src in (CSRC / "qr_gguf.cpp", CSRC / "qr_registry.cpp", CSRC / "qr_host.cpp",
                ROOT / "tests" / "c" / "sanitize_host.cpp"):
        o = tmp_path / (src.stem + ".o")
        subprocess.run([cxx, "-std=c++17", "-Wall", *SAN, "-c", str(src), "-o", str(o)], check=True)
        objs.append(str(o))
    o = tmp_path / "oracle.o"
    subprocess.run([cc, "-std=c11", "-D_GNU_SOURCE", "-ffp-contract=off", "-Wall", *SAN, "-c",
                    str(ROOT / "oracle" / "oracle.c"), "-o", str(o)], check=True)
    objs.append(str(o))
    exe = tmp_path / "sanitize_host"
    subprocess.run([cxx, *SAN, *objs, "-o", str(exe), "-lm", "-lpthread"], check=True)
    env = dict(os.environ, ASAN_OPTIONS="abort_on_error=0:halt_on_error=1:detect_leaks=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600, env=env)
    if r.returncode != 0 and "LeakSanitizer does not work under ptrace" in r.stderr:
        env["ASAN_OPTIONS"] = "abort_on_error=0:halt_on_error=1:detect_leaks=0"
        r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600, env=env)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "sanitize_host: ok" in r.stdout
