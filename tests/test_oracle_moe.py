"""Pins of oracle.moe: known answers, closed forms and library routines."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import moe as om
from oracle import planner as op
from oracle.bf16 import bf16_to_f32, f32_to_bf16

from moe_fixtures import make_layer, random_tokens

import raon_npu_amd.geometry as G

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())
SMALL = G.MoeGeometry(hidden=256, inter=128, n_routed=12, n_shared=1, top_k=4)


@pytest.fixture(scope="module")
def small_layer():
    return make_layer(SMALL, seed=1)


def test_silu_glu_known_answers():
    for case in GOLDEN["silu_glu"]:
        g = np.full(16, case["gate"], np.float32)
        u = np.full(16, case["up"], np.float32)
        np.testing.assert_allclose(om.swiglu(g, u), case["out"], rtol=1e-5, atol=1e-6)


def test_activations_closed_form():
    rng = np.random.default_rng(4)
    g = (rng.standard_normal(4096) * 4).astype(np.float32)
    u = (rng.standard_normal(4096) * 4).astype(np.float32)
    gd, ud = g.astype(np.float64), u.astype(np.float64)
    sig = 1 / (1 + np.exp(-gd))
    np.testing.assert_allclose(om.swiglu(g, u), gd * sig * ud, rtol=2e-6, atol=1e-30)
    situ = 3.5 * np.tanh(gd / 3.5) * sig * 19.0 * np.tanh(ud / 19.0)
    np.testing.assert_allclose(om.situ_glu(g, u, 3.5, 19.0), situ, rtol=2e-6, atol=1e-30)
    # bf16 inputs are widened exactly
    gb, ub = f32_to_bf16(g), f32_to_bf16(u)
    np.testing.assert_array_equal(om.glu(gb, ub, None, None), om.swiglu(bf16_to_f32(gb), bf16_to_f32(ub)))


def test_linear_against_float64():
    rng = np.random.default_rng(8)
    w = (rng.standard_normal((96, 512)) * 0.02).astype(np.float32)
    x = f32_to_bf16(rng.standard_normal(512).astype(np.float32))
    y = om.linear(w, x)
    exact = w.astype(np.float64) @ bf16_to_f32(x).astype(np.float64)
    # one bf16 rounding of a value within fp32 summation error of the exact product
    yf = bf16_to_f32(y).astype(np.float64)
    assert np.all(np.abs(yf - exact) <= np.abs(exact) * 2**-8 + 1e-6)
    # fp32 input stays fp32
    assert om.linear(w, bf16_to_f32(x)).dtype == np.float32


@pytest.mark.parametrize("score", ["softmax", "sigmoid"])
def test_route_token_matches_torch_topk(small_layer, score):
    rng = np.random.default_rng(12)
    bias = (rng.standard_normal(SMALL.n_routed) * 0.01).astype(np.float32)
    spec = om.RouterSpec(small_layer.router, SMALL.top_k, score=score, bias=bias, scaling=2.5)
    xs = random_tokens(32, SMALL.hidden, 13)
    for x in xs:
        top, w, logits = om.route_token(x, spec)
        lt = torch.from_numpy(logits.astype(np.float32))
        sc = torch.softmax(lt, 0) if score == "softmax" else torch.sigmoid(lt)
        np.testing.assert_allclose(om.router_scores(logits, score), sc.numpy(), rtol=1e-6, atol=1e-9)
        choice = om.router_scores(logits, score) + bias
        ref = torch.topk(torch.from_numpy(choice), SMALL.top_k).indices.numpy()
        assert top.tolist() == ref.tolist()
        assert abs(float(np.sum(w, dtype=np.float64)) - 2.5) < 1e-5


def test_combine_order_regression():
    # kernels/moe_grouped/test_planner.py:127-155: ascending id, not route order.
    ids = np.array(GOLDEN["order_regression_ids"]["ids"])
    vals = np.zeros((6, 5), np.float32)
    vals[1], vals[2], vals[3] = 1.0e8, 1.0, -1.0e8
    rows = {int(e): f32_to_bf16(vals[r]) for r, e in enumerate(ids)}
    w = np.ones(6, np.float32)
    correct = om.combine_routed(rows, ids, w)
    acc = np.zeros(5, np.float32)
    for r in range(6):
        acc += bf16_to_f32(rows[int(ids[r])]) * 1.0
    assert correct.tobytes() != f32_to_bf16(acc).tobytes()


def test_accumulate_known_answer():
    # bench/moe/test_moe_ref.py:430-437: rows 1..6 at weight 1/6 plus shared row 7 -> 10.5
    rows = {e: f32_to_bf16(np.full(8, float(e + 1), np.float32)) for e in range(6)}
    routed = om.combine_routed(rows, np.arange(6), np.full(6, 1.0 / 6.0, np.float32))
    out = f32_to_bf16(bf16_to_f32(routed) + np.float32(7.0))
    np.testing.assert_allclose(bf16_to_f32(out), 10.5, rtol=1e-6)


def test_moe_experts_properties(small_layer):
    bank = small_layer.bank()
    x = random_tokens(1, SMALL.hidden, 21)[0]
    ids = np.array([7, 2, 11, 5])
    w = np.array([0.4, 0.3, 0.2, 0.1], np.float32)
    out = om.moe_experts(bank, x, ids, w)
    perm = np.array([2, 0, 3, 1])
    assert om.moe_experts(bank, x, ids[perm], w[perm]).tobytes() == out.tobytes()
    single = om.moe_experts(bank, x, np.array([5]), np.array([1.0], np.float32))
    assert single.tobytes() == om.expert_chain(bank, 5, x, 4.0, 25.0).tobytes()


def test_grouped_equals_planner_path(small_layer):
    # Restates kernels/moe_grouped/test_planner.py:67-105 on the q4nx experts.
    bank = small_layer.bank()
    T, k = 13, SMALL.top_k
    xs = random_tokens(T, SMALL.hidden, 31)
    rng = np.random.default_rng(32)
    ids = np.stack([rng.choice(SMALL.n_routed, k, replace=False) for _ in range(T)])
    w = rng.random((T, k), dtype=np.float32)
    sgu = np.stack([om.shared_gate_up(bank, SMALL.shared_id, x) for x in xs])
    routed, sdown = om.moe_experts_grouped(bank, xs, ids, w, sgu, SMALL.shared_id, None, None)

    def run(plan, inputs, stage):
        outs = []
        for call, gathered in zip(plan.calls, inputs):
            width = 2 * SMALL.inter if stage == "b1" else SMALL.hidden
            o = np.zeros((8, 8, width), np.uint16)
            for slot, job in enumerate(call.jobs):
                if job is None:
                    continue
                g, u, d = bank.expert(job.expert)
                for row in range(len(job.assignments)):
                    xr = gathered[slot, row]
                    o[slot, row] = np.concatenate([om.linear(g, xr), om.linear(u, xr)]) if stage == "b1" else om.linear(d, xr[: SMALL.inter])
            outs.append(o)
        return outs

    p1 = op.build_plan(ids, n_routed=SMALL.n_routed)
    b1 = op.scatter_b1(p1, run(p1, op.gather_inputs(p1, xs), "b1"))
    rin, sin = op.make_b2_inputs(b1, sgu, SMALL.inter, None, None)
    p2 = op.build_plan(ids, include_shared=True, n_routed=SMALL.n_routed)
    final, shared = op.scatter_b2(p2, run(p2, op.gather_inputs(p2, rin, sin), "b2"), ids, w)
    np.testing.assert_array_equal(final, routed)
    np.testing.assert_array_equal(shared, sdown)
    # the per-expert GEMM form agrees within one bf16 rounding
    r2, s2 = om.moe_experts_grouped_batched(bank, xs, ids, w, sgu, SMALL.shared_id, None, None)
    for a, b in ((r2, routed), (s2, sdown)):
        d = np.abs(bf16_to_f32(a).astype(np.float64) - bf16_to_f32(b))
        assert d.max() < 1e-2


def test_moe_token_adds_shared(small_layer):
    lay = small_layer
    bank, spec = lay.bank(), lay.router_spec()
    x = random_tokens(1, SMALL.hidden, 41)[0]
    out, top, w, _ = om.moe_token(bank, spec, x, None, None, shared_id=SMALL.shared_id)
    routed = om.moe_experts(bank, x, top, w, None, None)
    sh = om.shared_expert(bank, SMALL.shared_id, x, None, None)
    assert out.tobytes() == f32_to_bf16(bf16_to_f32(routed) + bf16_to_f32(sh)).tobytes()
