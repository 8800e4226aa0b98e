"""Build libtaomate_h3_amd.so (gfx950) from csrc/ with hipcc, in-tree.

    python taomate-h3_amd/build.py

The library exports only the C ABI of include/taomate_h3_amd.h.  Every HIP
source is compiled for gfx950 with packed-FP32 instruction selection off.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libtaomate_h3_amd.so"
# Measurement kernels of bench.py's `ceilings` object, kept out of the product library.
CEILINGS_SRC = "ceilings.hip"
CEILINGS_LIB = PKG / "libh3q_ceilings.so"
SOURCES = ["act_quant.hip", "head_quant.hip", "norm_quant.hip", "swiglu_quant.hip", "gemm.hip", "gemm_w4.hip", "gemm_skinny.hip", "capi.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the gfx950 library)")


def _quiet(text: str) -> str:
    # hipcc's host pass does not know the GPU-only feature flag; drop that note.
    return "\n".join(l for l in text.splitlines() if "packed-fp32-ops" not in l)


def _compile(cc: str, src: str, obj: Path) -> subprocess.CompletedProcess:
    cmd = [cc, *HIPCC_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    return subprocess.run(cmd, capture_output=True, text=True)


def build(verbose: bool = False) -> Path:
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    cc = hipcc()
    objects = [objdir / (src + ".o") for src in SOURCES]
    # One hipcc per source, at most as many at once as there are CPUs (8 here).
    workers = max(1, min(len(SOURCES), os.cpu_count() or 1, 8))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        results = list(pool.map(lambda so: _compile(cc, *so), zip(SOURCES, objects)))
    for src, res in zip(SOURCES, results):
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{_quiet(res.stderr)}")
        if verbose and _quiet(res.stderr).strip():
            print(_quiet(res.stderr), file=sys.stderr)
    _link(cc, [str(o) for o in objects], LIB)
    ceil_obj = objdir / (CEILINGS_SRC + ".o")
    res = _compile(cc, CEILINGS_SRC, ceil_obj)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {CEILINGS_SRC}:\n{_quiet(res.stderr)}")
    _link(cc, [str(ceil_obj)], CEILINGS_LIB)
    return LIB


def _link(cc: str, objects: list[str], out: Path) -> None:
    tmp = out.with_suffix(".so.tmp")
    cmd = [cc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *objects]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of {out.name} failed:\n{_quiet(res.stderr)}")
    os.replace(tmp, out)


if __name__ == "__main__":
    print(build(verbose=True))
