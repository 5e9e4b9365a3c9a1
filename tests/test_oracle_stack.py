"""Pins of oracle.moe.prefill_layer and oracle.moe.residual_stack (CPU).

* ``prefill_layer`` (host/raon.py:1565-1602, grouped branch) against the token path
  (``moe_token`` per token, host/raon.py:1288-1330): byte-equal, as the reference's own
  grouped-prefill parity test requires (host/test_prefill_grouped_parity.py:42-115 asserts
  the grouped path equals the token-serial one byte for byte).
* Both against a closed form on constant-weight experts (tests/closed_form.py): every
  projection is ``c * sum(x)`` and every sum is exact, so the layer reduces to a scalar
  chain evaluated with Python floats and torch's bf16 rounding.
* The identity case: all-zero expert bundles give a zero MoE output, so the residual
  stack returns its input unchanged.
* Planted mistakes (a single rounding around the residual add, a dropped shared expert,
  gate and up swapped, the lowest-scoring experts selected) each break the closed-form
  comparison: the pins tell those plausible errors apart.
"""

from __future__ import annotations

import numpy as np
import pytest

import closed_form as cf
from moe_fixtures import make_layer, random_tokens
from oracle import moe as om
from oracle.bf16 import bf16_to_f32, f32_to_bf16
from oracle.q4nx import pack_gemv, quantize

import raon_npu_amd.geometry as G

GEOM = G.MoeGeometry(hidden=256, inter=128, n_routed=16, n_shared=1, top_k=4)


def _const_oracle_layers(n_layers: int, seed: int):
    """Constant-weight layers as oracle Layers (pack_gemv bytes of quantize(constant))."""
    g = GEOM
    consts, layers = [], []
    for li in range(n_layers):
        lay = cf.make_const_layer(g.hidden, g.inter, g.n_routed, g.top_k, seed + li)
        gu = b"".join(pack_gemv(*quantize(lay.gate_up_f32(e))) for e in range(g.n_experts))
        dn = b"".join(pack_gemv(*quantize(lay.down_f32(e, g.inter_pad))) for e in range(g.n_experts))
        bank = om.ExpertBank(gu, dn, g.n_experts, g.hidden, g.inter, g.inter_pad, cache=g.n_experts)
        layers.append(om.Layer(bank, om.RouterSpec(lay.router_bf16(), g.top_k, score="softmax"), g.shared_id))
        consts.append(lay)
    return consts, layers


@pytest.fixture(scope="module")
def const_stack():
    return _const_oracle_layers(5, 700)


def test_constant_bundles_dequantize_to_constants(const_stack):
    consts, layers = const_stack
    for lay, ol in zip(consts, layers):
        for e in (0, GEOM.n_routed):
            g, u, d = ol.bank.expert(e)
            assert np.all(g == np.float32(lay.cg[e])) and np.all(u == np.float32(lay.cu[e]))
            assert np.all(d == np.float32(lay.cd[e]))


def test_residual_stack_closed_form(const_stack):
    consts, layers = const_stack
    xs = cf.inputs(6, GEOM.hidden, 710)
    for x in xs:
        got = om.residual_stack(layers, x)
        ref = cf.residual_stack(consts, bf16_to_f32(x))
        np.testing.assert_array_equal(bf16_to_f32(got), ref)


def test_moe_token_routing_closed_form(const_stack):
    consts, layers = const_stack
    x = cf.inputs(1, GEOM.hidden, 711)[0]
    for lay, ol in zip(consts, layers):
        top, w, _ = om.route_token(x, ol.router)
        assert sorted(top.tolist()) == lay.chosen
        np.testing.assert_array_equal(w, np.full(GEOM.top_k, 1.0 / GEOM.top_k, np.float32))


def test_prefill_layer_closed_form(const_stack):
    consts, layers = const_stack
    xs = cf.inputs(9, GEOM.hidden, 712)
    for lay, ol in zip(consts[:2], layers[:2]):
        for batched in (False, True):
            out, top, w = om.prefill_layer(ol.bank, ol.router, xs, GEOM.shared_id, None, None, batched=batched)
            for t in range(xs.shape[0]):
                s = float(np.sum(bf16_to_f32(xs[t]).astype(np.float64)))
                assert np.all(bf16_to_f32(out[t]) == np.float32(cf.layer_out(lay, s))), (batched, t)
                assert sorted(top[t].tolist()) == lay.chosen


def test_prefill_layer_equals_token_path():
    """Grouped-branch prefill == token-serial _moe_token, byte for byte (random weights,
    both routers, SwiGLU and SiTU)."""
    for score, betas, seed in (("softmax", (None, None), 720), ("sigmoid", (4.0, 25.0), 721)):
        bias = (np.random.default_rng(seed).standard_normal(GEOM.n_routed) * 0.01).astype(np.float32)
        syn = make_layer(GEOM, seed=seed, score=score, bias=bias if score == "sigmoid" else None)
        bank, spec = syn.bank(), syn.router_spec()
        if score == "sigmoid":
            spec.scaling = 2.5
        xs = random_tokens(7, GEOM.hidden, seed + 1)
        out, top, w = om.prefill_layer(bank, spec, xs, GEOM.shared_id, *betas, batched=False)
        for t in range(xs.shape[0]):
            ref, rtop, rw, _ = om.moe_token(bank, spec, xs[t], *betas, shared_id=GEOM.shared_id)
            assert out[t].tobytes() == ref.tobytes(), (score, t)
            assert top[t].tolist() == rtop.tolist()
            np.testing.assert_array_equal(w[t], rw)
        # the per-expert GEMM form: same routing, outputs within one rounding of the bf16 grid
        out_b, top_b, _ = om.prefill_layer(bank, spec, xs, GEOM.shared_id, *betas, batched=True)
        np.testing.assert_array_equal(top_b, top)
        d = np.abs(bf16_to_f32(out_b).astype(np.float64) - bf16_to_f32(out))
        assert d.max() <= 1e-2


def test_zero_bundles_identity():
    """All-zero experts: every projection is 0, so prefill_layer returns zeros and the
    residual stack returns x unchanged (any router)."""
    g = GEOM
    z = np.zeros((2 * g.inter, g.hidden), np.float32)
    gu = pack_gemv(*quantize(z)) * g.n_experts
    dn = pack_gemv(*quantize(np.zeros((g.hidden, g.inter_pad), np.float32))) * g.n_experts
    bank = om.ExpertBank(gu, dn, g.n_experts, g.hidden, g.inter, g.inter_pad, cache=g.n_experts)
    syn = make_layer(g, seed=730)
    layers = [om.Layer(bank, syn.router_spec(), g.shared_id) for _ in range(3)]
    xs = random_tokens(4, g.hidden, 731)
    out, _, _ = om.prefill_layer(bank, syn.router_spec(), xs, g.shared_id, None, None)
    assert np.all(bf16_to_f32(out) == 0.0)
    for x in xs:
        assert om.residual_stack(layers, x).tobytes() == x.tobytes()


# ------------------------------------------------------------ planted mistakes --
def _stack_single_rounding(layers, x):
    h = np.asarray(x, np.uint16)
    for lyr in layers:
        top, w, _ = om.route_token(h, lyr.router, lyr.router_f32())
        routed = om.moe_experts(lyr.bank, h, top, w, None, None)
        sh = om.shared_expert(lyr.bank, lyr.shared_id, h, None, None)
        h = f32_to_bf16(bf16_to_f32(h) + (bf16_to_f32(routed) + bf16_to_f32(sh)))
    return h


def _stack_no_shared(layers, x):
    h = np.asarray(x, np.uint16)
    for lyr in layers:
        out, *_ = om.moe_token(lyr.bank, lyr.router, h, None, None, None, lyr.router_f32())
        h = f32_to_bf16(bf16_to_f32(h) + bf16_to_f32(out))
    return h


def _differs(fn, consts, layers, xs) -> bool:
    return any(not np.array_equal(bf16_to_f32(fn(layers, x)), cf.residual_stack(consts, bf16_to_f32(x))) for x in xs)


def test_planted_mistakes_break_the_closed_form(const_stack, monkeypatch):
    consts, layers = const_stack
    xs = cf.inputs(6, GEOM.hidden, 710)
    assert _differs(_stack_single_rounding, consts, layers, xs)
    assert _differs(_stack_no_shared, consts, layers, xs)
    real_glu = om.glu
    monkeypatch.setattr(om, "glu", lambda g, u, gb, vb: real_glu(u, g, gb, vb))
    assert _differs(om.residual_stack, consts, layers, xs)
    monkeypatch.setattr(om, "glu", real_glu)
    real_scores = om.router_scores
    # the lowest-scoring experts selected: another expert set
    monkeypatch.setattr(om, "router_scores", lambda lg, score: -real_scores(lg, score))
    assert _differs(om.residual_stack, consts, layers, xs[:2])
