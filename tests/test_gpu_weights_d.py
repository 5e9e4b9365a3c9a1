"""GPU: weights-d MoE layers (q4nx moe_b1 gate/up, bfp16 moe_b2 down) and the loader.

The device holds exactly the bundle bytes (download round trips), and the routed sum
(``moe_experts``, host/backend.py:466-510 as NpuBackend.moe_experts serves it on the real
model, npu/backend.py:5029-5322), the grouped prefill contract (npu/backend.py:4845-4979)
and the shared expert served through ``linear`` (RaonModel._moe_token, host/raon.py:
1288-1330) match the fp32 oracle over ``DWeights``-style dequantization within the
BASELINE bars (max-abs 1e-2, rel-L2 1e-3).  The loader test builds a one-layer
weights-d directory at the real model's shapes (H=2560, I=1088, 128+1 experts, top-6).
"""

from __future__ import annotations

import numpy as np
import pytest

import raon_npu_amd.geometry as G
from oracle import bfp16 as B
from oracle import moe as om
from oracle.bf16 import bf16_to_f32, f32_to_bf16
from oracle.q4nx import pack_gemv, quantize

from moe_fixtures import check_grouped_dev, compare_bf16, random_tokens
from weights_d_fixtures import manifest_entry, random_bfp16_bundle, random_q4nx_bundle, write_bundle, write_manifest

pytestmark = pytest.mark.gpu


def _small_d_bundles(geom, seed):
    """moe_b1 / moe_b2 / shared_gu of a small layer, quantized from N(0, 0.02) weights
    with the oracle's q4nx and bfp16 packers (down columns past I are zero)."""
    rng = np.random.default_rng(seed)
    b1 = [pack_gemv(*quantize(rng.normal(0, 0.02, (2 * geom.inter, geom.hidden)).astype(np.float32)))
          for _ in range(geom.n_routed)]
    b2 = []
    for _ in range(geom.n_routed + 1):
        d = np.zeros((geom.hidden, geom.inter_pad), np.float32)
        d[:, : geom.inter] = rng.normal(0, 0.02, (geom.hidden, geom.inter))
        b2.append(B.pack_gemv(d))
    sgu = B.pack_gemv(rng.normal(0, 0.02, (2 * geom.inter, geom.hidden)).astype(np.float32))
    router = f32_to_bf16(rng.normal(0, 0.05, (geom.n_routed, geom.hidden)).astype(np.float32))
    return b"".join(b1), b"".join(b2), sgu, router


@pytest.fixture(scope="module")
def small_d(gpu_ctx):
    from raon_npu_amd.backend import GpuBackend

    geom = G.MoeGeometry(hidden=512, inter=320, n_routed=8, n_shared=1, top_k=3)
    b1, b2, sgu, router = _small_d_bundles(geom, 41)
    be = GpuBackend(context=gpu_ctx)
    lyr = be.register_moe_layer_d(970, geom, b1, b2, shared_gu=sgu, router_weight=router, score="sigmoid",
                                  scaling=2.5)
    lyr.reserve(16)
    bank = om.DExpertBank(b1, b2, geom.n_routed, geom.hidden, geom.inter, shared_gu=sgu, cache=16)
    yield be, lyr, geom, bank, (b1, b2, sgu, router)
    lyr.free()


def test_d_layer_round_trip(small_d):
    be, lyr, geom, bank, (b1, b2, sgu, _) = small_d
    gb, db = lyr.gu_expert_bytes, lyr.dn_expert_bytes
    assert db == geom.hidden * geom.inter_pad * 9 // 8
    for e in (0, 5, geom.n_routed):
        gu, dn = lyr.download_expert(e)
        assert dn == b2[e * db:(e + 1) * db]
        assert gu == (b"" if e == geom.n_routed else b1[e * gb:(e + 1) * gb])


@pytest.mark.parametrize("betas", [(4.0, 25.0), (None, None)])
def test_d_layer_moe_experts(small_d, betas):
    be, lyr, geom, bank, _ = small_d
    rng = np.random.default_rng(42)
    xs = random_tokens(4, geom.hidden, 43)
    for t in range(4):
        ids = rng.choice(geom.n_routed, geom.top_k, replace=False)
        w = rng.uniform(0.1, 1.0, geom.top_k).astype(np.float32)
        got = be.moe_experts(970, xs[t], ids, w, *betas)
        ref = om.moe_experts(bank, xs[t], ids, w, *betas)
        err, rel, same = compare_bf16(got, ref)
        print(f"d-layer moe_experts token {t} betas {betas}: max-abs {err:.3e} rel-L2 {rel:.3e} identical {same:.4f}")
        assert err <= 1e-2 and rel <= 1e-3


def test_d_layer_shared_expert_via_linear(small_d):
    """RaonModel._moe_token's shared path: linear(gate), linear(up), host SiTU, linear(down)."""
    be, lyr, geom, bank, _ = small_d
    pfx = "model.layers.970.moe.shared_experts"
    x = random_tokens(1, geom.hidden, 44)[0]
    g = be.linear(f"{pfx}.gate_proj.weight", x)
    u = be.linear(f"{pfx}.up_proj.weight", x)
    sg, su, sd = bank.expert(geom.n_routed)
    for got, w in ((g, sg), (u, su)):
        err, rel, _ = compare_bf16(got, om.linear(w, x))
        assert err <= 1e-2 and rel <= 1e-3
    act = f32_to_bf16(om.situ_glu(g, u))
    down = be.linear(f"{pfx}.down_proj.weight", act)
    err, rel, same = compare_bf16(down, om.linear(sd, act))
    print(f"shared down via linear: max-abs {err:.3e} rel-L2 {rel:.3e} identical {same:.4f}")
    assert down.shape == (geom.hidden,) and err <= 1e-2 and rel <= 1e-3
    # fp32 input gives fp32 output (host/backend.py:9-14)
    assert be.linear(f"{pfx}.down_proj.weight", bf16_to_f32(act)).dtype == np.float32


def test_d_layer_grouped(small_d):
    be, lyr, geom, bank, _ = small_d
    T = 11
    rng = np.random.default_rng(45)
    x = random_tokens(T, geom.hidden, 46)
    ids = np.stack([rng.choice(geom.n_routed, geom.top_k, replace=False) for _ in range(T)]).astype(np.int64)
    w = rng.uniform(0.1, 1.0, (T, geom.top_k)).astype(np.float32)
    sg, su, _ = bank.expert(geom.n_routed)
    sgu = np.stack([np.concatenate([om.linear(sg, x[t]), om.linear(su, x[t])]) for t in range(T)])
    routed, sdown = be.moe_experts_grouped(970, x, ids, w, sgu)
    r_ref, s_ref = om.moe_experts_grouped(bank, x, ids, w, sgu, geom.n_routed)
    for got, ref, what in ((routed, r_ref, "routed"), (sdown, s_ref, "shared_down")):
        err, rel, same = compare_bf16(got, ref)
        print(f"d-layer grouped {what}: max-abs {err:.3e} rel-L2 {rel:.3e} identical {same:.4f}")
        assert err <= 1e-2 and rel <= 1e-3
    # The grouped MFMA path and the per-token decode kernels agree within the same bar.
    err, rel, _ = compare_bf16(routed[3], be.moe_experts(970, x[3], ids[3], w[3]))
    assert err <= 1e-2 and rel <= 1e-3
    # the device-resident form equals the host call, eagerly and under graph replay
    check_grouped_dev(be, 970, x, ids, w, sgu)


def test_d_layer_rejects_what_it_cannot_serve(small_d, gpu_ctx):
    be, lyr, geom, bank, (b1, b2, _, _) = small_d
    x = random_tokens(1, geom.hidden, 47)[0]
    with pytest.raises(ValueError, match="weights-d"):
        lyr.moe_decode(x)
    with pytest.raises(ValueError, match="weights-d"):
        gpu_ctx.decode_stack([lyr], x)
    with pytest.raises(ValueError):
        lyr.upload_d(1, geom.n_routed - 1, b1[: 2 * lyr.gu_expert_bytes])  # past the last routed expert
    with pytest.raises(ValueError):
        lyr.upload_d(2, 0, b2[:-1])
    with pytest.raises(ValueError):
        lyr.upload_experts(b1, b2)
    with pytest.raises(ValueError):
        be.moe_experts(970, x, np.array([0, 0, 1]), np.ones(3, np.float32))
    # the router still runs on a weights-d layer (sigmoid + scaling)
    ids, wts, logits = lyr.route(x)
    spec = om.RouterSpec(small_d[4][3], geom.top_k, score="sigmoid", scaling=2.5)
    top, w_ref, _ = om.route_token(x, spec)
    assert sorted(ids[0].tolist()) == sorted(np.asarray(top).tolist())


def test_load_weights_d_real_shapes(gpu_ctx, tmp_path, small_d):
    """One MoE layer of the released model's bundle shapes, loaded from a directory with a
    manifest (require_complete=False: the other bundles are absent), then served."""
    from raon_npu_amd import weights_d as W
    from raon_npu_amd.backend import GpuBackend

    comps, bundles = W.canonical_specs()
    rng = np.random.default_rng(48)
    data = {
        "L01/moe_b1": random_q4nx_bundle(W.canonical_size(bundles["L01/moe_b1"])[0], rng),
        "L01/moe_b2": random_bfp16_bundle(W.canonical_size(bundles["L01/moe_b2"])[0], rng),
        "L01/shared_gu": random_bfp16_bundle(W.canonical_size(bundles["L01/shared_gu"])[0], rng),
    }
    entries = []
    for name, buf in data.items():
        sha = write_bundle(tmp_path, bundles[name], buf)
        entries.append(manifest_entry(bundles[name], comps, bundles[name].rel_file, sha))
    write_manifest(tmp_path, entries)

    be = GpuBackend(context=gpu_ctx)
    info = be.load_weights_d(tmp_path, require_complete=False)
    assert set(info["loaded"]) == set(data)
    lyr = be.layer(1)
    assert lyr.d_layout and lyr.geom.top_k == 6
    assert lyr.download_expert(77)[1] == data["L01/moe_b2"][77 * 3686400:78 * 3686400].tobytes()
    bank = om.DExpertBank(data["L01/moe_b1"], data["L01/moe_b2"], 128, 2560, 1088, shared_gu=data["L01/shared_gu"],
                          cache=8)
    x = random_tokens(2, 2560, 49)
    for t in range(2):
        ids = rng.choice(128, 6, replace=False)
        w = rng.uniform(0.05, 0.4, 6).astype(np.float32)
        got = be.moe_experts(1, x[t], ids, w)
        err, rel, same = compare_bf16(got, om.moe_experts(bank, x[t], ids, w))
        print(f"weights-d L01 moe_experts token {t}: max-abs {err:.3e} rel-L2 {rel:.3e} identical {same:.4f}")
        assert err <= 1e-2 and rel <= 1e-3
        # Another layer's activations (a narrower layer: its rows land in this layer's
        # padding columns of the shared scratch) must not leak into this layer's down
        # input: the random moe_b2 bytes here have non-zero weights in those columns.
        sbe, _, sgeom, _, _ = small_d
        sbe.moe_experts(970, random_tokens(1, sgeom.hidden, 50 + t)[0], np.arange(sgeom.top_k),
                        np.ones(sgeom.top_k, np.float32))
        assert np.array_equal(be.moe_experts(1, x[t], ids, w), got)
    # The grouped MFMA path at the real shapes: I = 1088 leaves the last gate/up n-tile
    # partial, and the bfp16 down K is padded to 1280 with non-zero padding weights.
    # Routes are drawn from 12 experts so that the oracle dequantizes few of them.
    T = 48
    xg = random_tokens(T, 2560, 56)
    gids = np.stack([rng.choice(12, 6, replace=False) for _ in range(T)]).astype(np.int64)
    gw = rng.uniform(0.05, 0.4, (T, 6)).astype(np.float32)
    gsgu = random_tokens(T, 2 * 1088, 57)
    routed, sdown = be.moe_experts_grouped(1, xg, gids, gw, gsgu)
    r_ref, s_ref = om.moe_experts_grouped_batched(bank, xg, gids, gw, gsgu, 128)
    for got, ref, what in ((routed, r_ref, "routed"), (sdown, s_ref, "shared_down")):
        err, rel, same = compare_bf16(got, ref)
        print(f"weights-d L01 grouped T={T} {what}: max-abs {err:.3e} rel-L2 {rel:.3e} identical {same:.4f}")
        assert err <= 1e-2 and rel <= 1e-3
    sg, su, sd = bank.expert(128)
    g = be.linear("model.layers.1.moe.shared_experts.gate_proj.weight", x[0])
    act = f32_to_bf16(om.situ_glu(g, be.linear("model.layers.1.moe.shared_experts.up_proj.weight", x[0])))
    err, rel, _ = compare_bf16(be.linear("model.layers.1.moe.shared_experts.down_proj.weight", act), om.linear(sd, act))
    assert err <= 1e-2 and rel <= 1e-3
    lyr.free()

    # a corrupted byte fails the digest and leaves no layer behind
    buf = data["L01/moe_b2"].copy()
    buf[12345] ^= 1
    (tmp_path / bundles["L01/moe_b2"].rel_file).write_bytes(buf.tobytes())
    be._layers = {}
    with pytest.raises(ValueError, match="sha256 mismatch"):
        be.load_weights_d(tmp_path, require_complete=False)
    assert 1 not in be._layers
    with pytest.raises(KeyError):  # the device layer was freed too
        lyr.free()


def test_moe_experts_dev_matches_host_and_replays(small_d):
    """rmoe_moe_experts_dev: the host entry point's result from device pointers, eagerly
    and from a captured graph replayed with eager work in between (every replay checked)."""
    import torch

    be, lyr, geom, bank, _ = small_d
    rng = np.random.default_rng(51)
    xs = random_tokens(3, geom.hidden, 52)
    ids = np.stack([rng.choice(geom.n_routed, geom.top_k, replace=False) for _ in range(3)]).astype(np.int32)
    w = rng.uniform(0.1, 1.0, (3, geom.top_k)).astype(np.float32)
    want = np.stack([be.moe_experts(970, xs[t], ids[t], w[t]) for t in range(3)])
    xd = torch.from_numpy(xs.view(np.int16)).cuda()
    idd = torch.from_numpy(ids).cuda()
    wd = torch.from_numpy(w).cuda()
    od = torch.zeros_like(xd)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for t in range(3):
            lyr.moe_experts_dev(xd[t], idd[t], wd[t], od[t], stream=stream)
    torch.cuda.synchronize()
    assert np.array_equal(od.cpu().numpy().view(np.uint16), want)
    od.zero_()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(g, stream=stream):
            for t in range(3):
                lyr.moe_experts_dev(xd[t], idd[t], wd[t], od[t], stream=stream)
    for rep in range(3):
        od.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(od.cpu().numpy().view(np.uint16), want), rep
        be.moe_experts(970, xs[rep], ids[(rep + 1) % 3], w[rep])  # eager work between replays
    with pytest.raises(ValueError):
        lyr.moe_experts_dev(xd[0], idd[0][:2].contiguous(), wd[0], od[0])


def test_d_layer_grouped_many_tokens(small_d):
    """1,100 tokens: groups of ~410 rows span full 128-row tiles and a partial one of each
    tile class; the whole call matches the batched oracle, and sampled tokens match the
    per-token decode kernels within the same bar."""
    be, lyr, geom, bank, _ = small_d
    T = 1100
    rng = np.random.default_rng(53)
    x = random_tokens(T, geom.hidden, 54)
    ids = np.stack([rng.choice(geom.n_routed, geom.top_k, replace=False) for _ in range(T)]).astype(np.int64)
    w = rng.uniform(0.1, 1.0, (T, geom.top_k)).astype(np.float32)
    sgu = random_tokens(T, 2 * geom.inter, 55)
    routed, sdown = be.moe_experts_grouped(970, x, ids, w, sgu)
    for t in (0, 517, 1099):
        err, rel, _ = compare_bf16(routed[t], be.moe_experts(970, x[t], ids[t], w[t]))
        assert err <= 1e-2 and rel <= 1e-3, t
    r_ref, s_ref = om.moe_experts_grouped_batched(bank, x, ids, w, sgu, geom.n_routed)
    for got, ref, what in ((routed, r_ref, "routed"), (sdown, s_ref, "shared_down")):
        err, rel, same = compare_bf16(got, ref)
        print(f"d-layer grouped T={T} {what}: max-abs {err:.3e} rel-L2 {rel:.3e} identical {same:.4f}")
        assert err <= 1e-2 and rel <= 1e-3


def test_d_layer_grouped_ignores_down_padding(gpu_ctx):
    """moe_b2's columns past I are padding whose bytes are not guaranteed: here they hold
    values ~1e30 (block exponents far above the real ones).  The bfp16 down GEMM shifts
    each weight row by the largest exponent of its real columns only, and the h columns
    past I are zero, so the result equals the oracle, which reads columns < I."""
    from raon_npu_amd.backend import GpuBackend

    geom = G.MoeGeometry(hidden=512, inter=320, n_routed=8, n_shared=1, top_k=3)
    rng = np.random.default_rng(61)
    b1, _, sgu, router = _small_d_bundles(geom, 62)
    b2 = []
    for _ in range(geom.n_routed + 1):
        d = np.empty((geom.hidden, geom.inter_pad), np.float32)
        d[:, : geom.inter] = rng.normal(0, 0.02, (geom.hidden, geom.inter))
        d[:, geom.inter:] = rng.normal(0, 1e30, (geom.hidden, geom.inter_pad - geom.inter))
        b2.append(B.pack_gemv(d))
    b2 = b"".join(b2)
    be = GpuBackend(context=gpu_ctx)
    lyr = be.register_moe_layer_d(971, geom, b1, b2, shared_gu=sgu, router_weight=router, score="sigmoid",
                                  scaling=2.5)
    try:
        bank = om.DExpertBank(b1, b2, geom.n_routed, geom.hidden, geom.inter, shared_gu=sgu, cache=16)
        T = 40
        x = random_tokens(T, geom.hidden, 63)
        ids = np.stack([rng.choice(geom.n_routed, geom.top_k, replace=False) for _ in range(T)]).astype(np.int64)
        w = rng.uniform(0.1, 1.0, (T, geom.top_k)).astype(np.float32)
        sgu_rows = random_tokens(T, 2 * geom.inter, 64)
        routed, sdown = be.moe_experts_grouped(971, x, ids, w, sgu_rows)
        r_ref, s_ref = om.moe_experts_grouped(bank, x, ids, w, sgu_rows, geom.n_routed)
        for got, ref, what in ((routed, r_ref, "routed"), (sdown, s_ref, "shared_down")):
            assert np.all(np.isfinite(bf16_to_f32(got))), what
            err, rel, same = compare_bf16(got, ref)
            print(f"d-layer grouped, garbage padding, {what}: max-abs {err:.3e} rel-L2 {rel:.3e} identical {same:.4f}")
            assert err <= 1e-2 and rel <= 1e-3
    finally:
        lyr.free()
