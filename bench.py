#!/usr/bin/env python3
"""Benchmark of the quantized-MoE hot path on one MI355X.

Default workload: 48 stacked MoE layers of the BASELINE
shape (H=2048, I=768, 128 routed experts + 1 shared, softmax top-8, SwiGLU, q4nx
weights N(0, 0.02)), residual add between layers, batch 1.  One step = one token
through all 48 layers in ONE persistent launch (router on the device, 8 routed +
shared experts, ordered fp32 combine, residual).  Weights are synthesized and
quantized on the GPU (seeded per layer); inputs are random N(0, 0.25^2) hidden states,
one per step, resident in HBM.

Printed: one JSON line with tokens/s, the roofline of the dominant kernel (the
persistent decode kernel: 48 x 27,066,368 algorithmic bytes per launch), the
prefill grouped GEMM (config 5) and the NumPy oracle (the reference CPU path)
timed on a bounded sample on this host.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

# Scale of the random hidden states of the 48-layer stack.  The stack adds each layer's
# MoE output to its input with no normalisation and SwiGLU is quadratic in its input: with
# N(0, 0.02) weights the stream grows by ~0.34 sigma^2 per layer, so N(0, 1) states
# overflow to non-finite values after ~20 layers (and route every token to experts 0..7
# from there on), while N(0, 0.25^2) states stay finite through 48 layers.
STACK_HIDDEN_STD = 0.25
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
# HBM bytes per launch of the decode stack kernel and of the lm_head GEMV: each run
# measures them itself (measure_traffic: rocprofv3 FETCH_SIZE and WRITE_SIZE passes over
# child `bench.py --profile-pass` runs, calibrated against a 512 MiB copy).  These are the
# figures of the committed counter profile (profiles/decode_prefill_hbm_counters.txt),
# reported instead only when rocprofv3 is absent, a pass fails, or --no-traffic is given.
DECODE_TRAFFIC_BYTES = 1338163081
LM_HEAD_TRAFFIC_BYTES = 749714547


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256, help="timed decode steps (tokens); exactly this many")
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the oracle CPU sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--prefill-tokens", type=int, default=6700)
    ap.add_argument("--prefill-reps", type=int, default=10)
    ap.add_argument("--zipf-tau", type=float, default=0.02)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-lm-head", action="store_true", help="skip the lm_head bfp16 GEMV measurement")
    ap.add_argument("--no-configs", action="store_true", help="skip configs 1-3 and the weights-d layer")
    ap.add_argument("--no-weights-d", action="store_true", help="skip the weights-d layer rows of 'configs'")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the in-run rocprofv3 FETCH_SIZE/WRITE_SIZE passes (roofline.traffic then comes "
                         "from the committed counter profile)")
    ap.add_argument("--profile-pass", action="store_true",
                    help="short run for hardware counters: 2 decode launches, 1 prefill layer and a "
                         "512 MiB device copy (the calibration kernel of known size); prints no JSON")
    ap.add_argument("--profile-configs", action="store_true",
                    help="short run for hardware counters of configs 1-3: a 512 MiB device copy twice "
                         "(calibration), then 20 config-1 GEMVs, 10 config-2 1-layer decode launches and 5 "
                         "config-3 prefill layers, eager, one at a time; prints no JSON")
    ap.add_argument("--build-timeline", action="store_true",
                    help="build the timeline variant of librmoe.so (RMOE_DECODE_TIMELINE) into --timeline-dir "
                         "and exit (CPU host; no GPU needed)")
    ap.add_argument("--timeline", action="store_true",
                    help="per-layer timeline of the 48-layer decode stack from the timeline variant library "
                         "(built beforehand with --build-timeline); prints a table, no JSON")
    ap.add_argument("--timeline-dir", type=Path, default=ROOT / "_build_timeline")
    return ap.parse_args()


def build_stack(ctx, geom, n_layers: int, seed: int):
    import torch

    layers = []
    for li in range(n_layers):
        lyr = ctx.create_layer(li, geom)
        lyr.synthesize(seed * 1000 + li, 0.02)
        gen = torch.Generator(device="cuda").manual_seed(seed * 1000 + li)
        rw = (torch.randn(geom.n_routed, geom.hidden, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
        lyr.set_router(rw.contiguous(), score="softmax")
        lyr.reserve(1)
        layers.append(lyr)
    return layers


def decode_graph(ctx, layers, x_pool, out_pool, stream, n_launch: int):
    """A HIP graph of n_launch decode steps: step i carries token x_pool[i % P] through
    every layer in ONE persistent launch and writes out_pool[i % P]."""
    import torch

    P = x_pool.shape[0]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        ctx.decode_stack_dev(layers, x_pool[0], out_pool[0], residual=True, stream=stream)  # warm
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=stream):
            for i in range(n_launch):
                ctx.decode_stack_dev(layers, x_pool[i % P], out_pool[i % P], residual=True, stream=stream)
    return g


def warm_graph(g, stream, min_ms: float = 40.0, max_replays: int = 400) -> None:
    """Untimed replays of g until ~min_ms of work has run: the GPU's clocks rise under
    sustained load, and a short timed window right after a pause measures the ramp (a
    config-5 prefill layer times 1.10 ms on its first replays and 0.96 ms once warm)."""
    import time as _time

    import torch

    torch.cuda.synchronize()
    t0 = _time.perf_counter()
    for _ in range(max_replays):
        with torch.cuda.stream(stream):
            g.replay()
        torch.cuda.synchronize()
        if (_time.perf_counter() - t0) * 1e3 >= min_ms:
            break


def time_graph(g, n: int, stream) -> float:
    """Seconds for n replays, timed with events recorded on the replay stream."""
    import torch

    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(n):
            g.replay()
        end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3


def zipf_bias(n: int, tau: float, seed: int):
    """Selection bias b_e = tau * log p_e with p_e proportional to rank_e^-1.1 (seeded ranks)."""
    import numpy as np

    rng = np.random.default_rng(seed)
    ranks = rng.permutation(n) + 1
    p = ranks.astype(np.float64) ** -1.1
    p /= p.sum()
    return (tau * np.log(p)).astype(np.float32)


def prefill_bench(ctx, geom, T: int, seed: int, reps: int, tau: float, stream):
    """one MoE layer prefill of T tokens with Zipf(1.1) expert popularity.
    Returns (seconds per layer, FLOPs per layer, expert histogram)."""
    import numpy as np
    import torch

    lyr = ctx.create_layer(1000, geom)
    lyr.synthesize(seed * 1000 + 999, 0.02)
    gen = torch.Generator(device="cuda").manual_seed(seed * 1000 + 999)
    rw = (torch.randn(geom.n_routed, geom.hidden, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
    lyr.set_router(rw.contiguous(), bias=zipf_bias(geom.n_routed, tau, seed), score="softmax")
    lyr.reserve(T)
    x = torch.randn(T, geom.hidden, device="cuda", generator=gen).to(torch.bfloat16).view(torch.int16)
    out = torch.empty_like(x)
    ids = torch.empty((T, geom.top_k), dtype=torch.int32, device="cuda")
    wts = torch.empty((T, geom.top_k), dtype=torch.float32, device="cuda")
    with torch.cuda.stream(stream):
        lyr.moe_prefill_dev(x, T, out, ids_dev=ids, wts_dev=wts, stream=stream)
    torch.cuda.synchronize()
    hist = np.bincount(ids.cpu().numpy().reshape(-1), minlength=geom.n_routed)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(g, stream=stream):
            lyr.moe_prefill_dev(x, T, out, ids_dev=ids, wts_dev=wts, stream=stream)
        g.replay()
    warm_graph(g, stream)
    secs = time_graph(g, reps, stream) / reps
    flops = T * (geom.top_k + 1) * geom.flops_per_assignment + 2 * T * geom.hidden * geom.n_routed
    lyr.free()
    return secs, flops, hist


def lm_head_bench(ctx, stream, seed: int, n: int = 50):
    """The released model's lm_head GEMV (npu/backend.py:703-719): bfp16ebs8 [260096, 2560],
    749 MB, one token.  Synthetic GEMV bytes (uniform int8 mantissas, exponent 118) uploaded
    through rmoe_matrix_upload_bfp16; n launches captured in one graph."""
    import numpy as np
    import torch

    M, K = 260096, 2560
    nbytes = M * K * 9 // 8
    rng = np.random.default_rng(seed + 11)
    buf = rng.integers(0, 256, nbytes, dtype=np.uint8)
    buf.reshape(-1, 144)[:, :16] = 118
    mat = ctx.upload_matrix(buf, M, K, fmt="bfp16")
    del buf
    mat.reserve(1)
    x = torch.randn(1, K, device="cuda").to(torch.bfloat16).view(torch.int16)
    y = torch.empty(1, M, dtype=torch.int16, device="cuda")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        mat.linear_dev(x, 1, y, stream=stream)
        with torch.cuda.graph(g, stream=stream):
            for _ in range(n):
                mat.linear_dev(x, 1, y, stream=stream)
        g.replay()
    warm_graph(g, stream, min_ms=20.0)
    secs = time_graph(g, 1, stream) / n
    mat.free()
    gbs = nbytes / secs / 1e9
    return {"workload": "lm_head bfp16ebs8 GEMV [260096, 2560], 1 token (linear_bfp16_kernel)",
            "us_per_launch": round(secs * 1e6, 2), "bytes_per_launch": nbytes, "GBps": round(gbs, 1),
            "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "traffic": LM_HEAD_TRAFFIC_BYTES}


def graph_us(fn, n: int, stream) -> float:
    """Microseconds per call of fn() (a device-side launch sequence), n calls in one graph."""
    import torch

    with torch.cuda.stream(stream):
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(g, stream=stream):
            for _ in range(n):
                fn()
        g.replay()
    warm_graph(g, stream, min_ms=20.0)
    return time_graph(g, 1, stream) / n * 1e6


def roofline(bound: str, work: float, seconds: float, kernel: str, per: str, traffic=None) -> dict:
    """The roofline block of one workload: `work` algorithmic bytes (hbm) or FLOPs (mfma) per
    launch (or per layer, `per`) over its measured duration, against MI355X's peak."""
    if bound == "hbm":
        achieved, peak, unit = work / seconds / 1e9, HBM_PEAK_GBS, "GB/s"
    else:
        achieved, peak, unit = work / seconds / 1e12, MFMA_BF16_PEAK_TFLOPS, "TFLOP/s"
    return {"bound": bound, "kernel": kernel, "per": per, "work": work, "us": round(seconds * 1e6, 3),
            "achieved": round(achieved, 1), "peak": peak, "unit": unit, "frac": round(achieved / peak, 4),
            "traffic": traffic}


# HBM bytes per launch of the configs 1-3 workloads: each default run measures them itself
# (measure_config_traffic: rocprofv3 FETCH_SIZE and WRITE_SIZE over a child
# `bench.py --profile-configs`, calibrated against a 512 MiB copy).  These are the figures
# of the committed counter profile (profiles/configs123_hbm_counters.txt), reported instead
# only when rocprofv3 is absent, a pass fails, or --no-traffic is given.
CONFIG_TRAFFIC_BYTES = {"config1_gemv": 1059270, "config2_decode_layer": 28544825, "config3_prefill_445": 466689316}


class ConfigWorkloads:
    """SURVEY configs 1-3 on the device: one q4nx GEMV [768, 2048] (config 1), one BASELINE
    decode layer in a 1-layer persistent launch (config 2) and one BASELINE prefill layer of
    445 tokens (config 3), each a callable that queues one launch (sequence) on `stream`."""

    def __init__(self, ctx, layers, geom, seed: int, stream):
        import torch

        self.geom, self.stream = geom, stream
        gen = torch.Generator(device="cuda").manual_seed(seed + 21)
        # config 1: one q4nx GEMV, W [768, 2048] (the down width of a BASELINE expert), x 1 x 2048
        w = torch.randn(768, 2048, device="cuda", generator=gen) * 0.02
        self.mat = ctx.quantize_matrix(w, 768, 2048)
        del w
        self.mat.reserve(1)
        self.x = torch.randn(1, 2048, device="cuda", generator=gen).to(torch.bfloat16).view(torch.int16)
        self.y = torch.empty(1, 768, dtype=torch.int16, device="cuda")
        # config 2: one decode layer (router + 8 routed + shared + combine), one persistent launch
        self.layer0 = layers[0]
        self.ctx = ctx
        self.x1 = torch.randn(geom.hidden, device="cuda", generator=gen).to(torch.bfloat16).view(torch.int16)
        self.o1 = torch.empty_like(self.x1)
        # config 3: prefill of 445 tokens, router without selection bias (near-uniform routing)
        self.T = 445
        self.layer0.reserve(self.T)
        self.xp = torch.randn(self.T, geom.hidden, device="cuda", generator=gen).to(torch.bfloat16).view(torch.int16)
        self.op = torch.empty_like(self.xp)

    def config1(self):
        self.mat.linear_dev(self.x, 1, self.y, stream=self.stream)

    def config2(self):
        self.ctx.decode_stack_dev([self.layer0], self.x1, self.o1, residual=True, stream=self.stream)

    def config3(self):
        self.layer0.moe_prefill_dev(self.xp, self.T, self.op, stream=self.stream)

    # algorithmic work per launch (SURVEY 8(d) figures)
    CONFIG1_BYTES = 990208  # weights 983,040 + x 4,096 + y 3,072

    def config3_flops(self) -> int:
        g = self.geom
        return self.T * (g.top_k + 1) * g.flops_per_assignment + 2 * self.T * g.hidden * g.n_routed

    def config3_bytes(self) -> int:
        """Every expert's weights (445 x 8 routes leave no expert unused) + the router + x in and out."""
        g = self.geom
        return g.n_experts * g.expert_bytes + g.router_bytes + 2 * self.T * g.hidden * 2

    def free(self):
        self.mat.free()


def configs_bench(ctx, layers, geom, seed: int, stream, weights_d: bool = True) -> dict:
    """SURVEY configs 1-3 (the other rows of the measurement table) and one weights-d MoE
    layer at the released model's shapes; each timed as back-to-back launches in a graph,
    with its roofline block (algorithmic bytes or FLOPs over the measured time)."""
    import numpy as np
    import torch

    from raon_npu_amd.geometry import RAON_1_MINI

    out = {}
    wl = ConfigWorkloads(ctx, layers, geom, seed, stream)
    gen = torch.Generator(device="cuda").manual_seed(seed + 22)
    us = graph_us(wl.config1, 1000, stream)
    b = wl.CONFIG1_BYTES
    out["config1_gemv"] = {"workload": "q4nx GEMV [768, 2048] x 1 token, 1000 launches in a graph",
                           "us_per_launch": round(us, 3), "GBps": round(b / us / 1e3, 1),
                           "frac_hbm_peak": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                           "roofline": roofline("hbm", b, us / 1e6, "linear_lane_kernel<16>", "launch",
                                                CONFIG_TRAFFIC_BYTES["config1_gemv"])}
    out["_config1_bytes"] = wl.mat.download()
    us = graph_us(wl.config2, 200, stream)
    b = geom.decode_bytes()
    out["config2_decode_layer"] = {"workload": "one BASELINE decode layer, batch 1 (1-layer persistent launch)",
                                   "us_per_layer": round(us, 3), "GBps": round(b / us / 1e3, 1),
                                   "frac_hbm_peak": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                                   "roofline": roofline("hbm", b, us / 1e6, "decode_stack_kernel (1 layer)", "launch",
                                                        CONFIG_TRAFFIC_BYTES["config2_decode_layer"])}
    ctx.reserve_decode_stack(layers)
    us = graph_us(wl.config3, 20, stream)
    fl = wl.config3_flops()
    wb = geom.n_experts * geom.expert_bytes
    out["config3_prefill_445"] = {"workload": "one BASELINE prefill layer, 445 tokens, softmax top-8 routing",
                                  "ms_per_layer": round(us / 1e3, 4), "tflops": round(fl / us / 1e6, 2),
                                  "weight_GBps": round(wb / us / 1e3, 1),
                                  "frac_hbm_peak": round(wb / us / 1e3 / HBM_PEAK_GBS, 4),
                                  "roofline": roofline("hbm", wl.config3_bytes(), us / 1e6,
                                                       "prefill layer (router, top-k, dispatch, grouped GEMMs, combine)",
                                                       "layer", CONFIG_TRAFFIC_BYTES["config3_prefill_445"]),
                                  "mfma": roofline("mfma", fl, us / 1e6, "prefill layer", "layer")}
    wl.free()
    if not weights_d:
        return out
    # weights-d layer: moe_b1 (q4nx) + moe_b2 (bfp16) at H=2560, I=1088, 128+1 experts, top-6
    g = RAON_1_MINI
    rng = np.random.default_rng(seed + 23)
    dl = ctx.create_layer_d(1001, g)
    b1 = rng.integers(0, 256, g.n_routed * g.gu_bytes, dtype=np.uint8)
    blk = b1.reshape(-1, 5120)
    sc = rng.uniform(5e-4, 2e-3, (blk.shape[0], 256)).astype(np.float32)
    blk[:, :512] = (sc.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(-1, 512)
    blk[:, 512:1024] = ((-7.5 * sc).view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(-1, 512)
    dl.upload_d(1, 0, b1)
    del b1, blk
    b2 = rng.integers(0, 256, (g.n_routed + 1) * dl.dn_expert_bytes, dtype=np.uint8)
    b2.reshape(-1, 144)[:, :16] = 118
    dl.upload_d(2, 0, b2)
    del b2
    dl.reserve(1)
    xd = torch.randn(g.hidden, device="cuda", generator=gen).to(torch.bfloat16).view(torch.int16)
    od = torch.empty_like(xd)
    ids = torch.tensor(rng.choice(g.n_routed, g.top_k, replace=False), dtype=torch.int32, device="cuda")
    wts = torch.full((g.top_k,), 1.0 / g.top_k, dtype=torch.float32, device="cuda")
    us = graph_us(lambda: dl.moe_experts_dev(xd, ids, wts, od, stream=stream), 200, stream)
    b = g.top_k * (dl.gu_expert_bytes + dl.dn_expert_bytes)
    # the same layer's grouped prefill contract for a chunk of 256 tokens (host entry point,
    # uploads and read-back included, as moe_experts_grouped serves RaonModel.prefill)
    Tg = 256
    xg = np.asarray(rng.standard_normal((Tg, g.hidden)), np.float32)
    xg = ((xg.view(np.uint32) + 0x8000) >> 16).astype(np.uint16)
    idg = np.stack([rng.choice(g.n_routed, g.top_k, replace=False) for _ in range(Tg)]).astype(np.int32)
    wg = np.full((Tg, g.top_k), 1.0 / g.top_k, np.float32)
    sg = ((np.asarray(rng.standard_normal((Tg, 2 * g.inter)), np.float32).view(np.uint32) + 0x8000) >> 16).astype(np.uint16)
    dl.reserve(Tg)
    dl.moe_experts_grouped(xg, idg, wg, sg)
    t0 = time.perf_counter()
    for _ in range(3):
        dl.moe_experts_grouped(xg, idg, wg, sg)
    gsec = (time.perf_counter() - t0) / 3
    # the same call on device-resident operands, 10 back-to-back calls in one graph
    import torch as _t

    xgd = _t.from_numpy(xg.view(np.int16)).cuda()
    idgd = _t.from_numpy(idg).cuda()
    wgd = _t.from_numpy(wg).cuda()
    sgd = _t.from_numpy(sg.view(np.int16)).cuda()
    rgd = _t.empty(Tg, g.hidden, dtype=_t.int16, device="cuda")
    sdd = _t.empty(Tg, g.hidden, dtype=_t.int16, device="cuda")
    gus = graph_us(lambda: dl.moe_experts_grouped_dev(xgd, idgd, wgd, sgd, rgd, sdd, stream=stream), 10, stream)
    wbytes = g.n_routed * (dl.gu_expert_bytes + dl.dn_expert_bytes) + dl.dn_expert_bytes
    out["weights_d_grouped_256"] = {
        "workload": "released-model MoE layer from weights-d bundles, moe_experts_grouped of 256 tokens "
                    "(routed sums + shared down): device-resident in a graph, and as the host call incl. copies",
        "ms_per_layer": round(gus / 1e3, 4), "tokens_per_s": round(Tg / gus * 1e6, 1),
        "weight_GBps": round(wbytes / gus / 1e3, 1), "frac_hbm_peak": round(wbytes / gus / 1e3 / HBM_PEAK_GBS, 4),
        "host_call_ms_per_layer": round(gsec * 1e3, 3)}
    out["weights_d_moe_experts"] = {
        "workload": "released-model MoE layer from weights-d bundles (q4nx moe_b1 + bfp16 moe_b2, H=2560, "
                    "I=1088), 6 routed experts of one token (decode_gate_up_band_kernel + decode_down_band_kernel)",
        "us_per_layer": round(us, 3), "bytes": b, "GBps": round(b / us / 1e3, 1),
        "frac_hbm_peak": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}
    dl.free()
    return out


def _blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info

        return max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:
        return 1


def _timed_loop(fn, budget_s: float, min_n: int = 2) -> tuple[float, int]:
    """Seconds per call of fn() over at least min_n calls and about budget_s seconds."""
    n, t0 = 0, time.perf_counter()
    while True:
        fn(n)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s and n >= min_n:
            return el / n, n


def cpu_legs(layer0, geom, cfg1_bytes: bytes, args) -> dict:
    """The reference CPU path restated by the oracle (test infrastructure), timed on this
    host's cores beside the GPU figures, in two variants:

    * "per_call_dequant" -- reference-faithful: the selected experts' q4nx bytes are
      parsed and dequantized when used, with the DWeights LRU of 32 experts
      (npu/backend.py:940-1058, 1246-1273), then NumpyBackend's fp32 GEMVs
      (host/backend.py:402-417, 466-510) and RaonModel._moe_token (host/raon.py:1288-1330);
    * "predequantized" -- the CPU's best case: every expert held as fp32 (dequantized
      before timing), the same token-serial GEMVs.

    Each with all BLAS threads and with one.  Configs 1-3 use the layer-0 weights of the
    decode stack, config 4 extrapolates a token-layer x48 (every layer costs the same), and
    config 5 is timed once with per-expert GEMMs over the whole 6,700-token batch
    (pre-dequantized) -- the reference CPU path itself is token-serial and is given per
    token instead.  Returns per-config figures and the headline (config 4) baseline."""
    import numpy as np
    import torch
    from threadpoolctl import threadpool_limits

    from oracle import moe as om
    from oracle.bf16 import f32_to_bf16
    from oracle.q4nx import dequantize_grouped, dequantize_simple, parse_gemv

    nthr = _blas_threads()
    hostinfo = {"os_cpu_count": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)), "blas_threads": nthr}
    budget = args.cpu_seconds
    rng = np.random.default_rng(args.seed + 31)
    out: dict = {"host": hostinfo}

    # config 1: one q4nx GEMV [768, 2048] (990,208 algorithmic bytes per call)
    x1 = f32_to_bf16(rng.standard_normal(2048).astype(np.float32))
    w_pre = dequantize_simple(*parse_gemv(cfg1_bytes, K=2048, M=768))
    c1 = {}
    for tag, threads in (("all_threads", nthr), ("one_thread", 1)):
        with threadpool_limits(threads):
            per_i, _ = _timed_loop(lambda i: om.linear(dequantize_simple(*parse_gemv(cfg1_bytes, K=2048, M=768)), x1),
                                   budget / 12)
            per_p, _ = _timed_loop(lambda i: om.linear(w_pre, x1), budget / 12, min_n=20)
        c1[tag] = {"per_call_dequant": {"us_per_call": round(per_i * 1e6, 1), "GBps": round(990208 / per_i / 1e9, 3)},
                   "predequantized": {"us_per_call": round(per_p * 1e6, 1), "GBps": round(990208 / per_p / 1e9, 3)}}
    out["config1"] = c1

    # the layer: router from build_stack's seed, experts read back from the device
    gen = torch.Generator(device="cuda").manual_seed(args.seed * 1000)
    rw = (torch.randn(geom.n_routed, geom.hidden, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
    router = rw.view(torch.int16).cpu().numpy().view(np.uint16)
    spec = om.RouterSpec(router, geom.top_k, score="softmax")
    wf = spec.weight_f32()
    parts = [layer0.download_expert(e) for e in range(geom.n_experts)]
    gu_all, dn_all = b"".join(p[0] for p in parts), b"".join(p[1] for p in parts)
    del parts
    xs = f32_to_bf16(rng.standard_normal((445, geom.hidden)).astype(np.float32))

    def token(bank, i):
        x = xs[i % xs.shape[0]]
        o, *_ = om.moe_token(bank, spec, x, None, None, shared_id=geom.shared_id, router_w_f32=wf)
        return o

    # variant (i): per-call dequant with an LRU of 32 experts
    faithful = {}
    for tag, threads, bud in (("all_threads", nthr, budget), ("one_thread", 1, budget / 2)):
        bank = om.ExpertBank(gu_all, dn_all, geom.n_experts, geom.hidden, geom.inter, cache=32)
        with threadpool_limits(threads):
            per, n = _timed_loop(lambda i: token(bank, i), bud)
        faithful[tag] = (per, n)
    # variant (ii): every expert dequantized to fp32 before timing
    bank_pre = om.ExpertBank(gu_all, dn_all, geom.n_experts, geom.hidden, geom.inter, cache=geom.n_experts)
    for e in range(geom.n_experts):
        gu = bank_pre.gate_up[e * bank_pre.gu_bytes:(e + 1) * bank_pre.gu_bytes]
        w = dequantize_grouped(*parse_gemv(gu, K=geom.hidden, M=2 * geom.inter))
        dn = bank_pre.down[e * bank_pre.dn_bytes:(e + 1) * bank_pre.dn_bytes]
        d = dequantize_grouped(*parse_gemv(dn, K=geom.inter_pad, M=geom.hidden))[:, : geom.inter]
        bank_pre._cache[e] = (np.ascontiguousarray(w[: geom.inter]), np.ascontiguousarray(w[geom.inter:]),
                              np.ascontiguousarray(d))
    with threadpool_limits(nthr):
        t0 = time.perf_counter()
        for i in range(xs.shape[0]):  # config 3 in full: 445 tokens, token-serial
            token(bank_pre, i)
        pre_all = ((time.perf_counter() - t0) / xs.shape[0], xs.shape[0])
    with threadpool_limits(1):
        pre_one = _timed_loop(lambda i: token(bank_pre, i), budget / 4)
    pre = {"all_threads": pre_all, "one_thread": pre_one}

    layer_bytes = geom.decode_bytes()
    fl3 = 445 * (geom.top_k + 1) * geom.flops_per_assignment + 2 * 445 * geom.hidden * geom.n_routed

    def per_layer(per, n, how):
        return {"us_per_layer": round(per * 1e6, 1), "GBps": round(layer_bytes / per / 1e9, 4), "tokens": n,
                "timed": how}

    out["config2"] = {tag: {"per_call_dequant": per_layer(*faithful[tag], "token sample"),
                            "predequantized": per_layer(*pre[tag], "445 tokens" if tag == "all_threads"
                                                        else "token sample")} for tag in faithful}

    def prefill(per, n, how):
        return {"ms_per_layer": round(per * 445 * 1e3, 2), "tflops": round(fl3 / (per * 445) / 1e12, 6),
                "timed": how}

    out["config3"] = {tag: {"per_call_dequant": prefill(*faithful[tag], f"{faithful[tag][1]} tokens, x445"),
                            "predequantized": prefill(*pre[tag], "all 445 tokens" if tag == "all_threads"
                                                      else f"{pre[tag][1]} tokens, x445")} for tag in faithful}
    out["config4"] = {tag: {"per_call_dequant": {"tokens_per_s": round(1.0 / (faithful[tag][0] * args.layers), 5)},
                            "predequantized": {"tokens_per_s": round(1.0 / (pre[tag][0] * args.layers), 5)}}
                      for tag in faithful}

    # config 5 once: 6,700 Zipf-routed tokens, per-expert GEMMs on the pre-dequantized bank
    T5 = args.prefill_tokens
    zspec = om.RouterSpec(router, geom.top_k, score="softmax", bias=zipf_bias(geom.n_routed, args.zipf_tau, args.seed))
    x5 = f32_to_bf16(rng.standard_normal((T5, geom.hidden)).astype(np.float32))
    fl5 = T5 * (geom.top_k + 1) * geom.flops_per_assignment + 2 * T5 * geom.hidden * geom.n_routed
    with threadpool_limits(nthr):
        t0 = time.perf_counter()
        om.prefill_layer(bank_pre, zspec, x5, geom.shared_id, None, None, batched=True)
        s5 = time.perf_counter() - t0
    out["config5"] = {"all_threads": {
        "predequantized_grouped_gemm": {"ms_per_layer": round(s5 * 1e3, 1), "tflops": round(fl5 / s5 / 1e12, 5),
                                        "timed": "once, whole batch"},
        "per_call_dequant": {"ms_per_layer": round(faithful["all_threads"][0] * T5 * 1e3, 1),
                             "tflops": round(fl5 / (faithful["all_threads"][0] * T5) / 1e12, 7),
                             "timed": f"{faithful['all_threads'][1]} tokens, x{T5} (token-serial reference path)"}}}
    per_f, n_f = faithful["all_threads"]
    headline = {
        "value": round(1.0 / (per_f * args.layers), 5),
        "unit": "tokens/s",
        "cores": nthr,
        "kind": "port",
        "sample": (f"NumPy oracle of the reference CPU path (route_token + moe_experts + shared + combine, "
                   f"per-call dequant with the DWeights LRU of 32) on {n_f} tokens through layer 0 "
                   f"({per_f * 1e3:.1f} ms per token-layer, {nthr} BLAS threads), extrapolated x{args.layers} layers; "
                   f"one thread: {faithful['one_thread'][0] * 1e3:.1f} ms per token-layer; host "
                   f"os.cpu_count()={hostinfo['os_cpu_count']}, usable CPUs {hostinfo['affinity_cpus']}"),
        "one_thread_value": round(1.0 / (faithful["one_thread"][0] * args.layers), 5),
        "predequantized_value": round(1.0 / (pre["all_threads"][0] * args.layers), 5),
        **hostinfo,
    }
    return {"headline": headline, "configs": out}


def calibration_copy(n_copies: int = 2) -> None:
    """A plain device copy of 512 MiB, n_copies times: its FETCH_SIZE / WRITE_SIZE per
    dispatch calibrate the counters against a known byte count."""
    import torch

    n = 512 * 1024 * 1024
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(n_copies):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def profile_configs(ctx, layers, geom, args, stream) -> int:
    """Configs 1-3 for per-dispatch hardware counters: the calibration copy, then each
    config's launch sequence a fixed number of times, eagerly, one at a time."""
    import torch

    calibration_copy()
    wl = ConfigWorkloads(ctx, layers[:1], geom, args.seed, stream)
    ctx.reserve_decode_stack(layers[:1])
    for name, fn, n in (("config1", wl.config1, 20), ("config2", wl.config2, 10), ("config3", wl.config3, 5)):
        for _ in range(n):
            with torch.cuda.stream(stream):
                fn()
            torch.cuda.synchronize()
        log(f"profile configs: {name} x{n} done")
    wl.free()
    ctx.close()
    return 0


def profile_pass(ctx, layers, geom, args, stream, gen) -> int:
    """A short, fixed sequence of kernels for per-dispatch hardware counters: a plain
    device copy of 512 MiB (twice; its FETCH_SIZE / WRITE_SIZE per dispatch calibrate the
    counters against a known byte count), two decode launches of the 48-layer stack, one
    prefill layer of config 5 and the lm_head GEMV."""
    import torch

    calibration_copy()
    x = (torch.randn(2, geom.hidden, device="cuda", generator=gen) * STACK_HIDDEN_STD).to(torch.bfloat16)
    x = x.view(torch.int16)
    out = torch.empty_like(x)
    ctx.reserve_decode_stack(layers)
    for i in range(2):
        ctx.decode_stack_dev(layers, x[i], out[i], residual=True, stream=stream)
    torch.cuda.synchronize()
    if not args.no_prefill:
        prefill_bench(ctx, geom, args.prefill_tokens, args.seed, 1, args.zipf_tau, stream)
    if not args.no_lm_head:
        lm_head_bench(ctx, stream, args.seed, n=2)
    torch.cuda.synchronize()
    log("profile pass done: copy 512 MiB x2, decode stack x2, prefill x1, lm_head GEMV")
    ctx.close()
    return 0


def _kind_profile_pass(name: str) -> str:
    """Kernel kind of a dispatch of `bench.py --profile-pass`."""
    return "stack" if "decode_stack" in name else "lm_head" if "linear_bfp16" in name else "copy"


# Kernel kinds of a dispatch of `bench.py --profile-configs` (the first match counts;
# other dispatches, such as the weight synthesis, are left out).
_CONFIG_KINDS = (("copyBuffer", "copy"), ("CopyBuffer", "copy"), ("linear_lane_kernel", "config1"),
                 ("decode_stack_kernel", "config2"), ("router_prep_kernel", "c3_router"),
                 ("topk_kernel", "c3_topk"), ("dispatch_scatter_kernel", "c3_scatter"),
                 ("grouped_gemm_kernel", "c3_gemm"), ("h_unify_kernel", "c3_unify"), ("combine_kernel", "c3_combine"))


def _kind_profile_configs(name: str) -> str | None:
    return next((k for pat, k in _CONFIG_KINDS if pat in name), None)


def _counter_pass(counter: str, out_dir: Path, child_args: list[str], kind_of, timeout_s: float,
                  regex: str | None = None) -> dict | None:
    """One rocprofv3 counter pass over a child `bench.py <child_args>` (this script, run
    as a separate process; this process only waits).  Returns {kernel kind: [per-dispatch
    counter sums, in dispatch order]} with the kinds that kind_of gives the kernel names
    (None: left out), or None when the pass did not produce its CSV."""
    import csv
    import subprocess
    from collections import defaultdict

    cmd = ["rocprofv3", "--pmc", counter] + (["--kernel-include-regex", regex] if regex else []) + [
        "--output-format", "csv", "-d", str(out_dir), "-o", "run", "--",
        sys.executable, str(ROOT / "bench.py")] + child_args
    # The pass runs in a process group of its own, so that a pass that overruns is ended
    # together with the profiled child (rocprofv3 starts the program as its own child).
    import signal

    try:
        proc = subprocess.Popen(cmd, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL, start_new_session=True)
    except OSError as e:
        log(f"traffic pass {counter}: {type(e).__name__}: {e}")
        return None
    try:
        proc.wait(timeout=timeout_s)
    except subprocess.TimeoutExpired:
        os.killpg(proc.pid, signal.SIGKILL)
        proc.wait()
        log(f"traffic pass {counter}: no result within {timeout_s:.0f} s; the pass was ended")
        return None
    csvs = sorted(out_dir.rglob("run_counter_collection.csv"))
    if not csvs:
        log(f"traffic pass {counter}: rocprofv3 exited {proc.returncode} without counter output")
        return None
    per = defaultdict(float)
    names = {}
    with open(csvs[0], newline="") as f:
        for row in csv.DictReader(f):
            if row.get("Counter_Name") != counter:
                continue
            d = int(row["Dispatch_Id"])
            per[d] += float(row["Counter_Value"])
            names[d] = row["Kernel_Name"]
    out = defaultdict(list)
    for d in sorted(per):
        kind = kind_of(names[d])
        if kind is not None:
            out[kind].append(per[d])
    # rocprofv3 can end with a fault of its own after a complete run; complete CSVs count.
    return dict(out) if out.get("copy") else None


def _calibrated_passes(child_args: list[str], kind_of, regex: str | None, tag: str) -> dict | None:
    """FETCH_SIZE, then WRITE_SIZE over the child, each per-dispatch value scaled to bytes
    by what the same counter reads for the child's 512 MiB calibration copy (its two
    largest copy dispatches).  {counter: {kind: [bytes per dispatch]}, counter + "_factor": f}."""
    import statistics
    import tempfile

    res = {}
    with tempfile.TemporaryDirectory(prefix=f"rmoe_traffic_{tag}_") as td:
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            r = _counter_pass(counter, Path(td) / counter, child_args, kind_of, 90.0, regex)
            if r is None:
                return None
            factor = 512 * 1024 * 1024 / statistics.median(sorted(r["copy"])[-2:])
            res[counter] = {k: [v * factor for v in vals] for k, vals in r.items()}
            res[counter + "_factor"] = factor
    return res


def measure_traffic(args) -> dict | None:
    """HBM bytes per launch of the decode stack and of the lm_head GEMV, measured in this
    run: rocprofv3 FETCH_SIZE, then WRITE_SIZE, each over a child `bench.py --profile-pass`
    (a 512 MiB device copy twice, two decode launches of the 48-layer stack, the lm_head
    GEMV), each scaled by what the same counter reads for the copy of known size (512 MiB
    read, 512 MiB written).  None when rocprofv3 is absent or a pass fails."""
    import shutil
    import statistics

    if shutil.which("rocprofv3") is None:
        log("traffic: rocprofv3 not found; roofline.traffic falls back to the committed figure")
        return None
    child = ["--profile-pass", "--no-prefill", "--seed", str(args.seed), "--layers", str(args.layers)] + (
        ["--no-lm-head"] if args.no_lm_head else [])
    res = _calibrated_passes(child, _kind_profile_pass, "decode_stack|linear_bfp16|copy|Copy", "stack")
    if res is None or "stack" not in res["FETCH_SIZE"] or "stack" not in res["WRITE_SIZE"]:
        return None
    med = {c: {k: statistics.median(v) for k, v in res[c].items()} for c in ("FETCH_SIZE", "WRITE_SIZE")}
    out = {
        "stack": med["FETCH_SIZE"]["stack"] + med["WRITE_SIZE"]["stack"],
        "fetch_factor": res["FETCH_SIZE_factor"],
        "write_factor": res["WRITE_SIZE_factor"],
    }
    if "lm_head" in med["FETCH_SIZE"] and "lm_head" in med["WRITE_SIZE"]:
        out["lm_head"] = med["FETCH_SIZE"]["lm_head"] + med["WRITE_SIZE"]["lm_head"]
    return out


def measure_config_traffic(args) -> dict | None:
    """HBM bytes per launch of configs 1-3, measured in this run like measure_traffic but
    over a child `bench.py --profile-configs --layers 1` (the calibration copy, then 20
    config-1 GEMVs, 10 config-2 1-layer decode launches and 5 config-3 prefill layers, one at
    a time): config 1 and 2 the median dispatch of their kernel, config 3 the sum over its
    kernels of their median dispatch (the grouped GEMM's gate/up and down dispatches
    alternate).  None when rocprofv3 is absent or a pass fails."""
    import shutil
    import statistics

    if shutil.which("rocprofv3") is None:
        return None
    res = _calibrated_passes(["--profile-configs", "--layers", "1", "--seed", str(args.seed)],
                             _kind_profile_configs, None, "configs")
    if res is None:
        return None
    out = {}
    c3_kinds = ("c3_router", "c3_topk", "c3_scatter", "c3_unify", "c3_combine")
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        r = res[c]
        if not all(k in r for k in ("config1", "config2", "c3_gemm") + c3_kinds) or len(r["c3_gemm"]) < 2:
            log(f"traffic: the configs pass of {c} lacks a kernel; configs keep the committed figures")
            return None
        med = {k: statistics.median(v) for k, v in r.items()}
        gemm = r["c3_gemm"]
        c3 = sum(med[k] for k in c3_kinds) + statistics.median(gemm[0::2]) + statistics.median(gemm[1::2])
        for name, v in (("config1_gemv", med["config1"]), ("config2_decode_layer", med["config2"]),
                        ("config3_prefill_445", c3)):
            out[name] = out.get(name, 0.0) + v
    return out


# Timeline stamps of the decode stack's timeline build (event index, meaning); the
# product library has none.  One wave per workgroup stores s_memrealtime (100 MHz).
TIMELINE_EVENTS = [
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
TIMELINE_SHAPE = (48, 256, 16)  # layers, workgroups, events of the device buffer


def build_timeline(out_dir: Path) -> Path:
    """The timeline variant of librmoe.so (RMOE_DECODE_TIMELINE) under out_dir."""
    sys.path.insert(0, str(ROOT / "raon-npu_amd"))
    import build as B

    return B.build(verbose=True, out_dir=out_dir, defines=("RMOE_DECODE_TIMELINE",))


def timeline(lib_path: Path, seed: int) -> int:
    """Four launches of the 48-layer BASELINE stack on the timeline library; prints, per
    event, the median and the maximum over workgroups of the time since the layer's first
    `ready`, averaged over layers 1..46, and the start of the next layer."""
    import ctypes

    import numpy as np

    if not lib_path.exists():
        log(f"{lib_path} is missing: build it first with --build-timeline")
        return 2
    from __graft_entry__ import load_package

    load_package()
    import raon_npu_amd._lib as L

    L.LIB_PATH = lib_path  # the timeline build instead of the in-tree library
    import torch

    from raon_npu_amd.device import Context
    from raon_npu_amd.geometry import BASELINE

    nl, ng, ne = TIMELINE_SHAPE
    ctx = Context(0)
    layers = build_stack(ctx, BASELINE, nl, seed)
    gen = torch.Generator(device="cuda").manual_seed(seed + 7)
    x = (torch.randn(4, BASELINE.hidden, device="cuda", generator=gen) * STACK_HIDDEN_STD).to(torch.bfloat16)
    x = x.view(torch.int16)
    out = torch.empty_like(x)
    ctx.reserve_decode_stack(layers)
    stream = torch.cuda.Stream()
    for i in range(4):
        ctx.decode_stack_dev(layers, x[i], out[i], residual=True, stream=stream)
    torch.cuda.synchronize()
    fn = L.load().rmoe_debug_stack_timeline
    fn.argtypes = [ctypes.POINTER(ctypes.c_ulonglong), ctypes.c_size_t]
    buf = np.zeros((nl, ng, ne), np.uint64)
    rc = fn(buf.ctypes.data_as(ctypes.POINTER(ctypes.c_ulonglong)), buf.size)
    if rc != 0:
        raise RuntimeError(f"rmoe_debug_stack_timeline returned {rc}")
    b = buf.astype(np.int64)
    rows, nxt = [], []
    for l in range(1, nl - 1):
        t0 = b[l, :, 0][b[l, :, 0] > 0].min()
        r = []
        for ev, _ in TIMELINE_EVENTS:
            v = b[l, :, ev]
            v = v[v > 0]
            r.append(((np.median(v) - t0) / 100.0, (v.max() - t0) / 100.0) if len(v) else (np.nan, np.nan))
        rows.append(r)
        n = b[l + 1, :, 0]
        nxt.append((n[n > 0].min() - t0) / 100.0)
    m = np.nanmean(np.array(rows), axis=0)
    print("decode stack timeline, 48-layer BASELINE stack, medians over workgroups averaged over layers 1..46")
    print(f"{'event':44s} {'median':>9s} {'max':>9s}   (us from the layer's first ready)")
    for (ev, name), (med, mx) in zip(TIMELINE_EVENTS, m):
        print(f"{name:44s} {med:9.2f} {mx:9.2f}")
    print(f"{'next layer first ready':44s} {np.mean(nxt):9.2f}", flush=True)
    # The same events per workgroup role (the unit dealing of the stack kernel: workgroup g
    # holds GU unit g when g < n_gu, GU units of the shared slot are the last nhb of them, and
    # the combiner of band b is the workgroup whose first DN unit is (slot 0, band b), i.e.
    # workgroup (n_gu + b) mod G).
    geom = BASELINE
    S, nhb, nb2 = geom.top_k + geom.n_shared, geom.inter // 32, geom.hidden // 64
    n_gu = S * nhb
    G = int((b[1, :, 0] > 0).sum())
    comb = {(n_gu + i) % G for i in range(nb2)}
    roles = [
        ("gate/up, routed slot", [w for w in range(G) if w < n_gu - nhb]),
        ("gate/up, shared slot (from LDS)", [w for w in range(G) if n_gu - nhb <= w < n_gu]),
        ("band combiners (no gate/up)", [w for w in range(G) if w >= n_gu and w in comb]),
        ("others (one down unit only)", [w for w in range(G) if w >= n_gu and w not in comb]),
    ]
    print("per workgroup role: median / max over the role's workgroups, averaged over layers 1..46")
    for rname, wgs in roles:
        if not wgs:
            continue
        print(f"  {rname} ({len(wgs)} workgroups)")
        for ev, name in TIMELINE_EVENTS:
            med, mx = [], []
            for l in range(1, nl - 1):
                t0 = b[l, :, 0][b[l, :, 0] > 0].min()
                v = b[l, wgs, ev]
                v = v[v > 0]
                if len(v):
                    med.append((np.median(v) - t0) / 100.0)
                    mx.append((v.max() - t0) / 100.0)
            if med:
                print(f"    {name:42s} {np.mean(med):9.2f} {np.mean(mx):9.2f}")
    sys.stdout.flush()
    ctx.close()
    return 0


def main() -> int:
    args = parse_args()
    if args.build_timeline:
        build_timeline(args.timeline_dir)
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (this build runs on a single "
              f"MI355X; the multi-GPU expert-parallel layout is a design in DESIGN.md)", file=sys.stderr)
        return 2
    import torch

    if args.timeline:
        return timeline(args.timeline_dir / "librmoe.so", args.seed)
    from __graft_entry__ import load_package

    load_package()
    from raon_npu_amd.device import Context
    from raon_npu_amd.geometry import BASELINE

    geom = BASELINE
    t_setup = time.perf_counter()
    ctx = Context(0)
    layers = build_stack(ctx, geom, args.layers, args.seed)
    log(f"stack of {args.layers} layers ready ({args.layers * (geom.n_experts * geom.expert_bytes + geom.router_bytes) / 1e9:.2f} GB) "
        f"in {time.perf_counter() - t_setup:.1f}s")

    stream = torch.cuda.Stream()
    gen = torch.Generator(device="cuda").manual_seed(args.seed + 7)
    if args.profile_pass:
        return profile_pass(ctx, layers, geom, args, stream, gen)
    if args.profile_configs:
        return profile_configs(ctx, layers, geom, args, stream)
    K, W = max(1, args.steps), max(0, args.warmup)
    P = min(32, K)  # distinct tokens, resident in HBM; launch i carries token i % P
    x_pool = (torch.randn(P, geom.hidden, device="cuda", generator=gen) * STACK_HIDDEN_STD).to(torch.bfloat16)
    x_pool = x_pool.view(torch.int16)
    out_pool = torch.empty_like(x_pool)
    ctx.reserve_decode_stack(layers)
    g = decode_graph(ctx, layers, x_pool, out_pool, stream, K)
    gw = decode_graph(ctx, layers, x_pool, out_pool, stream, W) if W else None
    log(f"decode graphs captured: {W} warmup + {K} timed steps (one persistent launch per step)")
    if gw is not None:
        with torch.cuda.stream(stream):
            gw.replay()
    torch.cuda.synchronize()
    secs = time_graph(g, 1, stream)
    steps = K
    tok_s = steps / secs
    ms_per_step = secs * 1e3 / steps
    bytes_per_token = args.layers * geom.decode_bytes()
    log(f"decode: {tok_s:.1f} tok/s, {ms_per_step:.4f} ms/token, {bytes_per_token * tok_s / 1e9:.1f} GB/s")
    # The timed launches' outputs must equal eager launches on the same tokens.
    check_ids = sorted({0, P - 1})
    eager = torch.empty_like(x_pool[0])
    with torch.cuda.stream(stream):
        for i in check_ids:
            ctx.decode_stack_dev(layers, x_pool[i], eager, residual=True, stream=stream)
            torch.cuda.synchronize()
            if not torch.equal(eager, out_pool[i]):
                raise RuntimeError(f"decode step {i}: timed graph output differs from an eager launch")
    if not torch.isfinite(out_pool.view(torch.bfloat16).float()).all():
        raise RuntimeError("the residual stream overflowed: non-finite decode outputs")
    log(f"timed outputs of tokens {check_ids} equal eager launches; all outputs finite")
    # The dominant kernel is the persistent decode kernel itself (one launch per step):
    # its average duration is the step time measured above.
    per_launch = secs / steps
    nbytes = bytes_per_token
    achieved = nbytes / per_launch / 1e9

    prefill = None
    if not args.no_prefill:
        psec, pflops, hist = prefill_bench(ctx, geom, args.prefill_tokens, args.seed, args.prefill_reps, args.zipf_tau,
                                           stream)
        tflops = pflops / psec / 1e12
        prefill = {
            "workload": f"BASELINE config 5: {args.prefill_tokens} tokens, Zipf(1.1) routing (selection bias tau={args.zipf_tau})",
            "ms_per_layer": round(psec * 1e3, 4),
            "flops_per_layer": pflops,
            "tflops": round(tflops, 2),
            "frac_bf16_peak": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "expert_tokens_max": int(hist.max()),
            "expert_tokens_min": int(hist.min()),
            "experts_over_1000": int((hist > 1000).sum()),
            "experts_under_10": int((hist < 10).sum()),
        }
        log(f"prefill {args.prefill_tokens} tokens: {psec * 1e3:.3f} ms/layer, {tflops:.1f} TFLOP/s "
            f"(hist max {hist.max()} min {hist.min()})")

    configs = None
    if not args.no_configs:
        configs = configs_bench(ctx, layers, geom, args.seed, stream, weights_d=not args.no_weights_d)
        for k, v in configs.items():
            if not k.startswith("_"):
                log(f"{k}: {v}")

    lm_head = None
    if not args.no_lm_head:
        lm_head = lm_head_bench(ctx, stream, args.seed)
        log(f"lm_head bfp16 GEMV: {lm_head['us_per_launch']} us, {lm_head['GBps']} GB/s")

    cpu = None
    if not args.no_cpu:
        cfg1 = configs.pop("_config1_bytes", None) if configs else None
        if cfg1 is None:
            import torch as _t

            w = _t.randn(768, 2048, device="cuda", generator=_t.Generator(device="cuda").manual_seed(args.seed + 21)) * 0.02
            m = ctx.quantize_matrix(w, 768, 2048)
            cfg1 = m.download()
            m.free()
        legs = cpu_legs(layers[0], geom, cfg1, args)
        cpu = legs["headline"]
        if configs:
            c = legs["configs"]
            configs["config1_gemv"]["cpu"] = c["config1"]
            configs["config2_decode_layer"]["cpu"] = c["config2"]
            configs["config3_prefill_445"]["cpu"] = c["config3"]
        cpu["configs"] = {k: legs["configs"][k] for k in ("config4", "config5")}
        if prefill is not None:
            prefill["cpu"] = legs["configs"]["config5"]
        log(f"cpu baseline: {cpu['value']} tok/s ({cpu['cores']} BLAS threads; one thread {cpu['one_thread_value']}, "
            f"pre-dequantized {cpu['predequantized_value']})")
    elif configs:
        configs.pop("_config1_bytes", None)

    # HBM traffic per launch, measured in this run by counter passes over child processes
    # (this process holds its buffers and waits); the committed figures otherwise.
    traffic, traffic_src = (DECODE_TRAFFIC_BYTES if args.layers == 48 else None), "committed counter profile"
    if not args.no_traffic and args.layers == 48:
        torch.cuda.synchronize()
        t_tr = time.perf_counter()
        tr = measure_traffic(args)
        if tr is not None:
            traffic, traffic_src = int(tr["stack"]), "rocprofv3 FETCH_SIZE + WRITE_SIZE, this run"
            if lm_head is not None and "lm_head" in tr:
                lm_head["traffic"] = int(tr["lm_head"])
                lm_head["traffic_source"] = traffic_src
            log(f"traffic: decode stack {traffic / 1e9:.4f} GB per launch ({traffic / nbytes:.3f}x the algorithmic "
                f"bytes), factors {tr['fetch_factor']:.1f} / {tr['write_factor']:.1f} B per counter unit, "
                f"{time.perf_counter() - t_tr:.0f} s")
    if lm_head is not None and "traffic_source" not in lm_head:
        lm_head["traffic_source"] = "committed counter profile"
    if configs:
        ctr = None
        if not args.no_traffic:
            torch.cuda.synchronize()
            t_tr = time.perf_counter()
            ctr = measure_config_traffic(args)
            if ctr is not None:
                log("traffic: configs 1-3 " + ", ".join(f"{k} {v / 1e6:.2f} MB" for k, v in ctr.items()) +
                    f" per launch, {time.perf_counter() - t_tr:.0f} s")
        for name in CONFIG_TRAFFIC_BYTES:
            if name in configs:
                rl = configs[name]["roofline"]
                if ctr is not None:
                    rl["traffic"] = int(ctr[name])
                rl["traffic_source"] = ("rocprofv3 FETCH_SIZE + WRITE_SIZE, this run" if ctr is not None
                                        else "committed counter profile")

    line = {
        "metric": "MoE decode tokens/s (48-layer q4nx stack, batch 1); prefill grouped-GEMM TFLOP/s in 'prefill'",
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) q4nx weights generated on the GPU; N(0,0.25^2) hidden states)",
        "config": {
            "workload": "BASELINE config 4: 48-layer decode, batch 1",
            "layers": args.layers,
            "hidden": geom.hidden,
            "moe_intermediate": geom.inter,
            "experts": f"{geom.n_routed} routed + {geom.n_shared} shared, softmax top-{geom.top_k}",
            "weights": "q4nx (5 bits/weight)",
            "activation": "SwiGLU, bf16 activations, fp32 accumulate",
            "bytes_per_token": bytes_per_token,
            "sustained_GBps": round(bytes_per_token * tok_s / 1e9, 1),
            "stack_roofline_frac": round(bytes_per_token * tok_s / 1e9 / HBM_PEAK_GBS, 4),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_stack_kernel (48 layers per launch)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "bytes_per_launch": nbytes,
            "us_per_launch": round(per_launch * 1e6, 3),
        },
        "cpu_baseline": cpu,
        "prefill": prefill,
        "lm_head": lm_head,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
