"""Build librmoe.so in-tree with hipcc for gfx950.

Usage: ``python raon-npu_amd/build.py`` (or ``__graft_entry__.build()``).  Every
``csrc/*.hip`` file is compiled to an object under ``_build/`` and linked into
``raon-npu_amd/librmoe.so``.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "librmoe.so"
ARCH = "gfx950"

# -ffp-contract=off: the kernels restate NumPy arithmetic in which a product and a
# sum are two roundings; fused multiply-adds are written explicitly where wanted.
# The packed-fp32 feature is switched off for device code (hipcc's host pass warns
# that it does not know the feature; that is harmless).
COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain is required to build librmoe.so")


def _compile(src: Path, build_dir: Path = BUILD, defines: tuple[str, ...] = ()) -> Path:
    obj = build_dir / (src.stem + ".o")
    cmd = [hipcc(), *COMMON, *(f"-D{d}" for d in defines), "-I", str(PKG.parent / "include"), "-c", str(src),
           "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = True, out_dir: Path | None = None, defines: tuple[str, ...] = ()) -> Path:
    """Compile every HIP source and link librmoe.so; returns the library path.

    By default the library is built in-tree (the product).  ``out_dir`` builds a variant
    elsewhere with extra preprocessor ``defines`` (e.g. the decode timeline build,
    ``RMOE_DECODE_TIMELINE``), leaving the in-tree library untouched."""
    build_dir = BUILD if out_dir is None else Path(out_dir) / "_build"
    lib = LIB if out_dir is None else Path(out_dir) / "librmoe.so"
    build_dir.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = max(1, min(len(sources), int(os.environ.get("MAX_JOBS", "8"))))
    with cf.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(lambda src: _compile(src, build_dir, tuple(defines)), sources))
    tmp = lib.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib} from {len(sources)} sources", flush=True)
    return lib


if __name__ == "__main__":
    build()
    sys.exit(0)
