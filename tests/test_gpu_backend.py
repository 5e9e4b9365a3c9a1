"""GPU: the drop-in boundary -- GpuBackend driven as RaonModel / Engine drive a backend.

Mirrors npu/test_backend_small.py:190-222 (the NPU backend equals the NumPy backend on the
same weights): here GpuBackend against the oracle's restatement of NumpyBackend, with the
reference's conventions -- uint16 bf16 in/out, fp32 in gives fp32 out, ValueError for
contract violations, KeyError for unknown weights, linear_batch byte-identical to stacked
linear.  Outputs within max-abs 1e-2 / rel-L2 1e-3 of the fp32 oracle; routing exact.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import bfp16 as B
from oracle import moe as om
from oracle.bf16 import bf16_to_f32, f32_to_bf16
from oracle.q4nx import dequantize_simple, pack_gemv, quantize

from moe_fixtures import check_bf16, check_grouped_dev, compare_bf16, make_layer, random_tokens, routing_margin

pytestmark = pytest.mark.gpu

GEOM_ARGS = dict(hidden=512, inter=256, n_routed=16, n_shared=1, top_k=4)


@pytest.fixture(scope="module")
def be():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from raon_npu_amd.backend import GpuBackend

    b = GpuBackend(0)
    yield b
    b.ctx.close()


@pytest.fixture(scope="module")
def dense(be):
    """A q4nx 'dense_gu'-like bundle [384, 512] served as two components, and a bfp16 bundle."""
    rng = np.random.default_rng(3)
    w = rng.normal(0, 0.02, (384, 512)).astype(np.float32)
    c, s, m = quantize(w)
    be.register_bundle("dense_gu", pack_gemv(c, s, m), 384, 512)
    be.register_component("gate", "dense_gu", 0, 256)
    be.register_component("up", "dense_gu", 256, 384)
    wb = rng.normal(0, 0.02, (256, 512)).astype(np.float32)
    blob = B.pack_gemv(wb)
    be.register_bundle("o_proj", blob, 256, 512, fmt="bfp16_gemv")
    return dequantize_simple(c, s, m), B.dequantize_packed(blob, 512, 256)


@pytest.fixture(scope="module")
def moe(be):
    from raon_npu_amd.geometry import MoeGeometry

    geom = MoeGeometry(**GEOM_ARGS)
    syn = make_layer(geom, seed=11)
    be.register_moe_layer(3, geom, syn.gate_up, syn.down, router_weight=syn.router, score="softmax")
    return geom, syn, syn.bank()


def test_linear_components_and_dtypes(be, dense):
    wq, _ = dense
    x = random_tokens(1, 512, 1)[0]
    y = be.linear("gate", x)
    assert y.dtype == np.uint16 and y.shape == (256,)
    err, rel, _ = compare_bf16(y, om.linear(wq[:256], x))
    assert err <= 1e-2 and rel <= 1e-3
    yu = be.linear("up", x)
    np.testing.assert_array_equal(yu, be.linear("dense_gu", x)[256:])
    # fp32 input -> fp32 output holding bf16 values (host/backend.py:9-14)
    xf = bf16_to_f32(x)
    yf = be.linear("gate", xf)
    assert yf.dtype == np.float32
    np.testing.assert_array_equal(f32_to_bf16(yf), y)


def test_linear_batch_is_stacked_linear(be, dense):
    xs = random_tokens(5, 512, 2)
    yb = be.linear_batch("gate", xs)
    ys = np.stack([be.linear("gate", xs[t]) for t in range(5)])
    np.testing.assert_array_equal(yb, ys)


def test_linear_bfp16_bundle(be, dense):
    _, wb = dense
    xs = random_tokens(3, 512, 4)
    y = be.linear_batch("o_proj", xs)
    err, rel, same = compare_bf16(y, om.linear(wb, xs))
    assert err <= 1e-2 and rel <= 1e-3 and same >= 0.99


def test_bundle_reuse_rule(be, dense):
    """npu/backend.py:3652-3663: the same input object in the same step reuses the bundle."""
    x = random_tokens(1, 512, 5)[0]
    be.set_step(7)
    a = be.linear("gate", x)
    n = be.call_counts["linear_gpu"]
    b = be.linear("up", x)  # same bundle, same step, same object -> sliced from the cache
    np.testing.assert_array_equal(b, be.linear("dense_gu", x)[256:])
    assert be.call_counts["linear_gpu"] == n + 2
    be.set_step(8)
    np.testing.assert_array_equal(be.linear("gate", x), a)
    be.reset()


def test_errors_follow_the_reference(be, dense, moe):
    with pytest.raises(KeyError):
        be.linear("no_such_weight", random_tokens(1, 512, 6)[0])
    with pytest.raises(ValueError):
        be.linear("gate", random_tokens(1, 256, 6)[0])  # wrong width
    with pytest.raises(ValueError):
        be.register_bundle("bad", b"\0" * 10, 128, 256, fmt="q8")
    with pytest.raises(ValueError):
        be.layer(99)
    with pytest.raises(NotImplementedError):
        be.mla_attend()
    assert "gate" in be and "dense_gu" in be and "nope" not in be


def test_moe_experts_matches_oracle(be, moe):
    geom, syn, bank = moe
    spec = syn.router_spec()
    xs = random_tokens(6, geom.hidden, 21)
    for t in range(6):
        top, wts, _ = om.route_token(xs[t], spec)
        for gb, vb in ((4.0, 25.0), (None, None)):
            got = be.moe_experts(3, xs[t], top, wts, gb, vb)
            want = om.moe_experts(bank, xs[t], top, wts, gb, vb)
            err, rel, _ = compare_bf16(got, want)
            assert err <= 1e-2 and rel <= 1e-3, (t, gb, err, rel)
    with pytest.raises(ValueError):
        be.moe_experts(3, xs[0], top, wts, shared_gu=np.zeros(3, np.uint16))


def test_route_matches_oracle(be, moe):
    geom, syn, _ = moe
    spec = syn.router_spec()
    xs = random_tokens(16, geom.hidden, 22)
    top, wts, logits = be.route(3, xs)
    for t in range(16):
        rt, rw, rl = om.route_token(xs[t], spec)
        np.testing.assert_allclose(logits[t], rl, rtol=1e-5, atol=1e-6)
        if routing_margin(xs[t], spec) > 1e-6:
            np.testing.assert_array_equal(top[t], rt)
            np.testing.assert_allclose(wts[t], rw, rtol=1e-5, atol=1e-7)


def test_moe_experts_grouped_matches_oracle(be, moe):
    geom, syn, bank = moe
    spec = syn.router_spec()
    T = 37
    xs = random_tokens(T, geom.hidden, 23)
    routes = [om.route_token(xs[t], spec) for t in range(T)]
    top = np.stack([r[0] for r in routes]).astype(np.int64)
    wts = np.stack([r[1] for r in routes]).astype(np.float32)
    sgu = np.stack([om.shared_gate_up(bank, geom.shared_id, xs[t]) for t in range(T)])
    routed, sdown = be.moe_experts_grouped(3, xs, top, wts, sgu, 4.0, 25.0)
    r_ref, s_ref = om.moe_experts_grouped(bank, xs, top, wts, sgu, geom.shared_id, 4.0, 25.0)
    for got, want in ((routed, r_ref), (sdown, s_ref)):
        err, rel, _ = compare_bf16(got, want)
        assert err <= 1e-2 and rel <= 1e-3, (err, rel)
    # each grouped row equals the per-token path within the same bar
    one = be.moe_experts(3, xs[5], top[5], wts[5], 4.0, 25.0)
    err, rel, _ = compare_bf16(routed[5], one)
    assert err <= 1e-2 and rel <= 1e-3
    # the device-resident form equals the host call, eagerly and under graph replay
    check_grouped_dev(be, 3, xs, top, wts, sgu, 4.0, 25.0)


def test_grouped_validation(be, moe):
    """npu/backend.py:4864-4897."""
    geom, _, _ = moe
    T = 3
    x = random_tokens(T, geom.hidden, 24)
    top = np.tile(np.arange(geom.top_k), (T, 1))
    w = np.full((T, geom.top_k), 0.25, np.float32)
    sgu = np.zeros((T, 2 * geom.inter), np.uint16)
    bad = [
        dict(x=x.astype(np.float32)),
        dict(x=x[:, :-2]),
        dict(top_ids=top[:, :-1]),
        dict(top_ids=np.where(top == 1, geom.n_routed, top)),
        dict(top_ids=np.where(top == 1, 0, top)),  # duplicate expert
        dict(top_weights=w.astype(np.float64)),
        dict(shared_gu=sgu[:, :-1]),
    ]
    for b in bad:
        args = dict(x=x, top_ids=top, top_weights=w, shared_gu=sgu)
        args.update(b)
        with pytest.raises(ValueError):
            be.moe_experts_grouped(3, args["x"], args["top_ids"], args["top_weights"], args["shared_gu"])


def test_hooks_and_flags(be, moe):
    geom, _, _ = moe
    x = random_tokens(1, geom.hidden, 25)[0]
    assert be.moe_prestart_shared(3, x) is None
    assert be.moe_abort_prestart_shared() is None
    assert be.prefetch_linears([]) is None
    assert be.prefill_shared_precompute is True and be.prefill_grouped_moe is True
    assert be.preload(4) is None


# ------------------------------------------------- RaonModel's call sequences --
def _pfx(layer: int) -> str:
    return f"model.layers.{layer}.moe"


def test_shared_expert_components_are_views(be, moe):
    """register_moe_layer serves the shared expert (expert n_routed of the bundles) under
    the names RaonModel calls, in place: the views download to the uploaded bytes."""
    geom, syn, bank = moe
    gu_view = be._bundles["L03/shared_gate_up"]
    dn_view = be._bundles["L03/shared_down"]
    e = geom.shared_id
    assert gu_view.download() == syn.gate_up[e * geom.gu_bytes:(e + 1) * geom.gu_bytes]
    assert dn_view.download() == syn.down[e * geom.dn_bytes:(e + 1) * geom.dn_bytes]
    x = random_tokens(1, geom.hidden, 30)[0]
    g, u, d = bank.expert(e)
    for name, w, xi in ((f"{_pfx(3)}.shared_experts.gate_proj.weight", g, x),
                        (f"{_pfx(3)}.shared_experts.up_proj.weight", u, x),
                        (f"{_pfx(3)}.shared_experts.down_proj.weight", d, x[: geom.inter])):
        err, rel, same = compare_bf16(be.linear(name, xi), om.linear(w, xi))
        assert err <= 1e-2 and rel <= 1e-3, name


def test_raon_model_token_call_sequence(be, moe):
    """RaonModel._moe_token (host/raon.py:1288-1330) replayed call for call: prestart hook,
    host router (NumPy, as _route_token), moe_experts, linear of the shared gate/up/down
    names with the host SiTU-GLU between, RTNE(routed + shared)."""
    geom, syn, bank = moe
    spec = syn.router_spec()
    pfx = _pfx(3)
    for t, x in enumerate(random_tokens(5, geom.hidden, 31)):
        be.set_step(100 + t)
        be.moe_prestart_shared(3, x)
        top, w, _ = om.route_token(x, spec)
        routed = be.moe_experts(3, x, top, w, gate_beta=4.0, value_beta=25.0)
        sh_gate = be.linear(f"{pfx}.shared_experts.gate_proj.weight", x)
        sh_up = be.linear(f"{pfx}.shared_experts.up_proj.weight", x)
        sh_act = om.situ_glu(sh_gate, sh_up, 4.0, 25.0)
        shared = be.linear(f"{pfx}.shared_experts.down_proj.weight", f32_to_bf16(sh_act))
        out = f32_to_bf16(bf16_to_f32(routed) + bf16_to_f32(shared))
        ref, rtop, _, _ = om.moe_token(bank, spec, x, 4.0, 25.0, shared_id=geom.shared_id)
        assert top.tolist() == rtop.tolist()
        check_bf16(out, ref, f"_moe_token replay {t}")


def test_raon_model_prefill_call_sequence(be, moe):
    """The grouped prefill branch (host/raon.py:1565-1602) replayed: linear_batch of the
    shared gate and up names, per-token host routing, moe_experts_grouped with the
    concatenated shared_gu, RTNE(routed + shared_down)."""
    geom, syn, bank = moe
    spec = syn.router_spec()
    pfx = _pfx(3)
    T = 29
    xs = random_tokens(T, geom.hidden, 32)
    sh_gate_all = be.linear_batch(f"{pfx}.shared_experts.gate_proj.weight", xs)
    sh_up_all = be.linear_batch(f"{pfx}.shared_experts.up_proj.weight", xs)
    routes = [om.route_token(xs[t], spec) for t in range(T)]
    top_all = np.stack([r[0] for r in routes])
    w_all = np.stack([r[1] for r in routes]).astype(np.float32, copy=False)
    routed, shared_down = be.moe_experts_grouped(3, xs, top_all, w_all,
                                                 np.concatenate([sh_gate_all, sh_up_all], axis=1),
                                                 gate_beta=4.0, value_beta=25.0)
    out = f32_to_bf16(bf16_to_f32(routed) + bf16_to_f32(shared_down))
    ref, rtop, _ = om.prefill_layer(bank, spec, xs, geom.shared_id, 4.0, 25.0)
    np.testing.assert_array_equal(top_all, rtop)
    check_bf16(out, ref, "prefill branch replay")


def test_linear_batch_rejects_non_bf16(be, moe):
    """npu/backend.py:3399-3400: only a [T, K] uint16 ndarray is accepted."""
    geom, _, _ = moe
    name = f"{_pfx(3)}.shared_experts.gate_proj.weight"
    xs = random_tokens(2, geom.hidden, 33)
    for bad in (bf16_to_f32(xs), xs[0], xs.astype(np.int32), list(xs)):
        with pytest.raises(ValueError):
            be.linear_batch(name, bad)


def test_view_handles_follow_the_layer(be):
    """A view's handle goes with its layer: freed or re-created layers invalidate it."""
    from raon_npu_amd.geometry import MoeGeometry

    geom = MoeGeometry(**GEOM_ARGS)
    syn = make_layer(geom, seed=34)
    lyr = be.register_moe_layer(9, geom, syn.gate_up, syn.down)
    view = be._bundles["L09/shared_down"]
    x = random_tokens(1, geom.inter_pad, 35)
    view.linear(x)
    lyr.free()
    with pytest.raises(KeyError):
        view.linear(x)
