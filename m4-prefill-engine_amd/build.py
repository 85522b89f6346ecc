"""Builds libm4_bridge.so (HIP kernels for gfx950 + the C-ABI) in this directory.

Usage: python build.py [-j JOBS]   (also called by __graft_entry__.build()).
Every source is compiled each call; objects go to _build/.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT = HERE / "libm4_bridge.so"
BUILD = HERE / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# (source, object stem, extra flags).  The tiled projection kernel is built
# once per format (0..8) so its instantiations compile in parallel.
SOURCES = ([("qr_gemm.hip", f"qr_gemm_f{f}", (f"-DQR_GEMM_FORMAT={f}",)) for f in range(9)] +
           [(s, s.rsplit(".", 1)[0], ()) for s in ("qr_gemm_host.hip", "qr_gemm_skinny.hip", "qr_dequant.hip",
                                                   "qr_attention.hip", "qr_norm_rope.hip", "qr_probe.hip", "qr_bridge.cpp", "qr_host.cpp", "qr_registry.cpp",
                                                   "qr_gguf.cpp")])

COMMON = ["-O3", "-fPIC", "-std=c++17", "--offload-arch=gfx950", "-ffp-contract=on",
          "-fvisibility=hidden", "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
          "-Wno-unused-lambda-capture"]
# Packed-fp32 VALU ops are disabled for device code (they have produced
# silently wrong results on these parts); the host pass ignores the flag.
DEVICE = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _fresh(obj: Path, src: str) -> bool:
    """Object newer than its source and every header (incremental builds)."""
    if not obj.exists():
        return False
    t = obj.stat().st_mtime
    deps = [CSRC / src, *CSRC.glob("*.h"), *(HERE.parent / "include").glob("*.h"), HERE / "build.py"]
    return all(d.stat().st_mtime < t for d in deps)


def _compile(unit: tuple, build_dir: Path = BUILD, extra: tuple = (), incremental: bool = False) -> Path:
    src, stem, defs = unit
    obj = build_dir / (stem + ".o")
    if incremental and not extra and _fresh(obj, src):
        return obj
    cmd = [HIPCC, *COMMON, *DEVICE, *defs, *extra, "-x", "hip", "-c", str(CSRC / src), "-o", str(obj)]
    if src.endswith(".cpp"):
        cmd = [HIPCC, *COMMON, *defs, *extra, "-x", "hip", "-c", str(CSRC / src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src}\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(jobs: int = 8, verbose: bool = False, out: Path = OUT, build_dir: Path = BUILD,
          extra: tuple = (), incremental: bool = False) -> Path:
    """Compile every source (optionally with extra compiler flags, e.g. -D
    tuning macros) and link `out`.  incremental: skip objects that are newer
    than their source and every header."""
    build_dir.mkdir(parents=True, exist_ok=True)
    # slowest units first so the pool stays busy
    order = sorted(SOURCES, key=lambda u: u[1] not in ("qr_gemm_f4", "qr_gemm_f5", "qr_gemm_f2"))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, build_dir, tuple(extra), incremental), order))
    cmd = [HIPCC, "-shared", "-fPIC", "--offload-arch=gfx950", "-o", str(out), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    # A shared library links with undefined symbols; a kernel whose host stub
    # the compiler dropped would only fail when the library is loaded.
    u = subprocess.run(["nm", "-u", "-C", str(out)], capture_output=True, text=True)
    missing = [l.strip() for l in u.stdout.splitlines() if "qr::" in l or "m4_" in l]
    if missing:
        raise RuntimeError("undefined library symbols after link:\n" + "\n".join(missing[:20]))
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    j = int(sys.argv[sys.argv.index("-j") + 1]) if "-j" in sys.argv else 4
    build(j, verbose=True, incremental="--incremental" in sys.argv)
