"""Builds libmx_sampler.so for gfx950 in-tree (metallix_amd/_build/).

The library is the HIP sampler behind include/mx_sampler.h.  hipcc
cross-compiles for gfx950 without a GPU, so this runs in the build container
as well as on the GPU box.
"""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = BUILD / "libmx_sampler.so"

# -ffp-contract=off: no FMA contraction, so f32/f64 arithmetic rounds step by
# step as the reference's does.  Denormals are kept.  Packed FP32 is off.
HIPCC_FLAGS = [
    "-O3",
    "--offload-arch=gfx950",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (Path(cand).exists() or cand == "hipcc"):
            return cand
    raise RuntimeError("hipcc not found")


def _compile(src: Path, obj: Path, verbose: bool) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", str(ROOT / "include"), "-c", "-o", str(obj), str(src)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name} ({res.returncode}):\n{res.stderr[-4000:]}")


def build_library(verbose: bool = False) -> Path:
    """Compiles every csrc/*.hip for gfx950 (in parallel) and links the library."""
    from concurrent.futures import ThreadPoolExecutor

    BUILD.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    objs = [BUILD / (s.stem + ".o") for s in srcs]
    with ThreadPoolExecutor(max_workers=min(4, len(srcs))) as ex:
        for f in [ex.submit(_compile, s, o, verbose) for s, o in zip(srcs, objs)]:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed ({res.returncode}):\n{res.stderr[-4000:]}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build_library(verbose=True))
