"""GPU: llama.cpp Q4_K tensors converted to q4nx on the device (quant/gguf_q4k.py:160-233).

The conversion is bit-exact against the oracle (codes kept, group parameters RTNE bf16
of the exact products, NaN -> 0x7FC0): compared as pack_gemv bytes.  GEMV and a decode
MoE layer built from converted tensors are then checked against the fp32 oracle with
the BASELINE bars (max-abs 1e-2, rel-L2 1e-3).
"""

from __future__ import annotations

import numpy as np
import pytest

import raon_npu_amd.geometry as G
from oracle import moe as om
from oracle import q4k
from oracle.bf16 import bf16_to_f32, f32_to_bf16
from oracle.q4nx import dequantize_simple, pack_gemv

from moe_fixtures import compare_bf16, random_tokens, routing_margin

pytestmark = pytest.mark.gpu


def _q4k_tensor(M: int, K: int, seed: int, special: bool = False) -> np.ndarray:
    """Random block_q4_K bytes of a row-major [M, K] tensor with finite d / dmin in the
    range of real models; ``special`` plants fp16 NaN, inf, subnormal, zero and negative
    d / dmin values in a few blocks."""
    rng = np.random.default_rng(seed)
    n = M * K // 256
    b = rng.integers(0, 256, size=(n, 144), dtype=np.uint8)
    # |w| ~ 0.05 as in real Q4_K exports (d * sc * 15 and dmin * mn of a few hundredths)
    b[:, 0:2] = (rng.uniform(2e-5, 2e-4, n) * rng.choice([-1, 1], n)).astype("<f2").view(np.uint8).reshape(n, 2)
    b[:, 2:4] = rng.uniform(1e-5, 4e-4, n).astype("<f2").view(np.uint8).reshape(n, 2)
    if special:
        vals = np.array([np.nan, np.inf, -np.inf, 6e-8, 0.0, -0.0, -1.5, 65504.0], dtype="<f2")
        for i, v in enumerate(vals):
            b[3 * i, 0:2] = np.array([v], dtype="<f2").view(np.uint8)
            b[3 * i + 1, 2:4] = np.array([v], dtype="<f2").view(np.uint8)
    return b


@pytest.mark.parametrize("M,K,special", [(128, 256, True), (256, 2048, False), (2176, 2560, False)])
def test_q4k_conversion_bit_exact(gpu_ctx, M, K, special):
    raw = _q4k_tensor(M, K, M + K, special)
    mat = gpu_ctx.upload_matrix(raw, M, K, fmt="q4k")
    assert mat.fmt == "q4nx"
    codes, scales, mins = q4k.matrix_to_q4nx(raw, M, K)
    want = pack_gemv(codes, scales, mins)
    got = mat.download()
    assert got == want
    mat.free()


def test_q4k_linear_matches_oracle(gpu_ctx):
    M, K = 2560, 2560  # an lm_head-wide slice: the real lm_head is [260096, 2560]
    raw = _q4k_tensor(M, K, 11)
    codes, scales, mins = q4k.matrix_to_q4nx(raw, M, K)
    wf = dequantize_simple(codes, scales, mins)
    rng = np.random.default_rng(12)
    x = f32_to_bf16(rng.standard_normal((3, K)).astype(np.float32))
    mat = gpu_ctx.upload_matrix(raw, M, K, fmt="q4k")
    y = mat.linear(x)
    ref = np.stack([om.linear(wf, x[t]) for t in range(3)])
    err, rel, same = compare_bf16(y, ref)
    print(f"q4k linear max-abs {err:.3e} rel-L2 {rel:.3e} bit-identical {same:.4f} "
          f"(|y| rms {np.sqrt(np.mean(bf16_to_f32(ref).astype(np.float64) ** 2)):.3e})")
    assert err <= 1e-2 and rel <= 1e-3 and same >= 0.99
    mat.free()


def test_q4k_rejects_bad_shapes(gpu_ctx):
    """Contract violations raise ValueError, as the reference's loaders do."""
    raw = _q4k_tensor(128, 256, 13)
    with pytest.raises(ValueError):
        gpu_ctx.upload_matrix(raw[:-1], 128, 256, fmt="q4k")
    with pytest.raises(ValueError):
        gpu_ctx.upload_matrix(raw, 128, 300, fmt="q4k")


def test_moe_layer_from_q4k_experts(gpu_ctx):
    """Experts from ffn_{gate,up,down}_exps-style Q4_K tensors: the device holds exactly
    the oracle's conversion, and a decode layer routes bit-exactly and matches the oracle."""
    from raon_npu_amd.backend import GpuBackend

    geom = G.MoeGeometry(hidden=512, inter=256, n_routed=8, n_shared=1, top_k=2)
    ne = geom.n_experts
    gate = _q4k_tensor(ne * geom.inter, geom.hidden, 21)
    up = _q4k_tensor(ne * geom.inter, geom.hidden, 22)
    down = _q4k_tensor(ne * geom.hidden, geom.inter, 23)
    rng = np.random.default_rng(24)
    router = f32_to_bf16(rng.normal(0.0, 0.05, (geom.n_routed, geom.hidden)).astype(np.float32))
    be = GpuBackend(context=gpu_ctx)
    lyr = be.register_moe_layer_q4k(960, geom, gate, up, down, router_weight=router, score="softmax")
    lyr.reserve(4)
    gu_parts, dn_parts = [], []
    pg, pd = geom.inter * geom.hidden // 256 * 144, geom.hidden * geom.inter // 256 * 144
    for e in range(ne):
        cg, sg, mg = q4k.matrix_to_q4nx(gate[e * pg // 144:(e + 1) * pg // 144], geom.inter, geom.hidden)
        cu, su, mu = q4k.matrix_to_q4nx(up[e * pg // 144:(e + 1) * pg // 144], geom.inter, geom.hidden)
        cd, sd, md = q4k.matrix_to_q4nx(down[e * pd // 144:(e + 1) * pd // 144], geom.hidden, geom.inter)
        gu_parts.append(pack_gemv(np.concatenate([cg, cu]), np.concatenate([sg, su]), np.concatenate([mg, mu])))
        dn_parts.append(pack_gemv(cd, sd, md))
        got_gu, got_dn = lyr.download_expert(e)
        assert got_gu == gu_parts[-1] and got_dn == dn_parts[-1], e
    bank = om.ExpertBank(b"".join(gu_parts), b"".join(dn_parts), ne, geom.hidden, geom.inter, geom.inter_pad,
                         cache=ne)
    spec = om.RouterSpec(router, geom.top_k, score="softmax")
    xs = random_tokens(4, geom.hidden, 25)
    for t in range(4):
        out, ids, _ = lyr.moe_decode(xs[t])
        ref, top, _, _ = om.moe_token(bank, spec, xs[t], None, None, shared_id=geom.shared_id)
        if routing_margin(xs[t], spec) > 1e-6:
            assert sorted(ids.tolist()) == sorted(top.tolist())
        a, b = bf16_to_f32(out).astype(np.float64), bf16_to_f32(ref).astype(np.float64)
        err = np.abs(a - b).max()
        rel = np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)
        print(f"q4k layer token {t}: max-abs {err:.3e} rel-L2 {rel:.3e} (|out| rms {np.sqrt(np.mean(b ** 2)):.3e})")
        assert err <= 1e-2 and rel <= 1e-3
    lyr.free()
