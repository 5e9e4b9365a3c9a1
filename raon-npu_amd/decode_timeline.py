"""Per-layer timeline of the persistent decode stack (a measurement tool, not the product).

Usage (repo root, GPU box):  python raon-npu_amd/decode_timeline.py [--build-only] [--out DIR]

Builds a variant of librmoe.so with ``RMOE_DECODE_TIMELINE`` defined (the decode stack
stores the device clock, s_memrealtime at 100 MHz, at fixed points of every layer; the
product library has no stamps) into ``DIR`` (default ``_build_timeline`` beside this file),
runs four launches of the 48-layer BASELINE stack on that library, and prints, per event,
the median and the maximum over workgroups of the time since the layer's first ``ready``,
averaged over layers 1..46.  Build the variant on the CPU host first (``--build-only``);
the GPU run then only loads it.
"""

from __future__ import annotations

import argparse
import ctypes
import sys
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
EVENTS = [
    (0, "ready seen"),
    (12, "first pass of partial logits in LDS"),
    (1, "x and partial logits in LDS, summed"),
    (13, "selection keys written"),
    (2, "routing done (ranked)"),
    (14, "first gate/up tile dot product (wave 0)"),
    (15, "gate/up waves summed (barrier)"),
    (3, "gate/up unit done, h published"),
    (4, "down waves hold their h"),
    (5, "down tiles in LDS"),
    (6, "down tile dot products done (wave 1)"),
    (7, "down partials summed (barrier)"),
    (8, "d stored as tagged words"),
    (9, "combiner holds every slot's d"),
    (10, "combiner has stored its x band"),
    (11, "combiner has published ready"),
]
LAYERS, GROUPS, NEV = 48, 256, 16


def build_variant(out: Path) -> Path:
    sys.path.insert(0, str(PKG))
    import build as B

    return B.build(verbose=True, out_dir=out, defines=("RMOE_DECODE_TIMELINE",))


def run(lib_path: Path) -> None:
    sys.path.insert(0, str(ROOT))
    from __graft_entry__ import load_package

    load_package()
    import raon_npu_amd._lib as L

    L.LIB_PATH = lib_path  # the timeline build, loaded instead of the in-tree library
    import torch

    import bench
    from raon_npu_amd.device import Context
    from raon_npu_amd.geometry import BASELINE

    ctx = Context(0)
    layers = bench.build_stack(ctx, BASELINE, LAYERS, 0)
    gen = torch.Generator(device="cuda").manual_seed(7)
    x = (torch.randn(4, BASELINE.hidden, device="cuda", generator=gen) * bench.STACK_HIDDEN_STD)
    x = x.to(torch.bfloat16).view(torch.int16)
    out = torch.empty_like(x)
    ctx.reserve_decode_stack(layers)
    stream = torch.cuda.Stream()
    for i in range(4):
        ctx.decode_stack_dev(layers, x[i], out[i], residual=True, stream=stream)
    torch.cuda.synchronize()
    lib = L.load()
    fn = lib.rmoe_debug_stack_timeline
    fn.argtypes = [ctypes.POINTER(ctypes.c_ulonglong), ctypes.c_size_t]
    buf = np.zeros((LAYERS, GROUPS, NEV), np.uint64)
    rc = fn(buf.ctypes.data_as(ctypes.POINTER(ctypes.c_ulonglong)), buf.size)
    if rc != 0:
        raise RuntimeError(f"rmoe_debug_stack_timeline returned {rc}")
    b = buf.astype(np.int64)
    rows, nxt = [], []
    for l in range(1, LAYERS - 1):
        t0 = b[l, :, 0][b[l, :, 0] > 0].min()
        r = []
        for ev, _ in EVENTS:
            v = b[l, :, ev]
            v = v[v > 0]
            r.append(((np.median(v) - t0) / 100.0, (v.max() - t0) / 100.0) if len(v) else (np.nan, np.nan))
        rows.append(r)
        n = b[l + 1, :, 0]
        nxt.append((n[n > 0].min() - t0) / 100.0)
    m = np.nanmean(np.array(rows), axis=0)
    print(f"decode stack timeline, 48-layer BASELINE stack, medians over workgroups averaged over layers 1..46")
    print(f"{'event':44s} {'median':>9s} {'max':>9s}   (us from the layer's first ready)")
    for (ev, name), (med, mx) in zip(EVENTS, m):
        print(f"{name:44s} {med:9.2f} {mx:9.2f}")
    print(f"{'next layer first ready':44s} {np.mean(nxt):9.2f}")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--out", type=Path, default=PKG / "_build_timeline")
    ap.add_argument("--build-only", action="store_true")
    args = ap.parse_args()
    lib = args.out / "librmoe.so"
    if args.build_only or not lib.exists():
        build_variant(args.out)
    if not args.build_only:
        run(lib)
    return 0


if __name__ == "__main__":
    sys.exit(main())
