"""GPU: the persistent decode kernel over a stack of MoE layers (BASELINE config 4 path).

One launch carries a token through every layer: router, top-k, routed + shared experts,
ordered combine and residual add per layer.  Checked against the oracle's
``residual_stack`` (routing of every layer bit-exact unless the k/k+1 selection gap is a
near-tie; hidden state within the bf16-ulp bound of the residual stream), against
layer-by-layer launches of the same kernel (bit-identical), and under HIP-graph replay.
"""

from __future__ import annotations

import numpy as np
import pytest

import raon_npu_amd.geometry as G
from oracle import moe as om
from oracle.bf16 import bf16_to_f32, f32_to_bf16

from moe_fixtures import STACK_HIDDEN_STD, LazyBank, check_bf16, make_layer, random_tokens, routing_margin

pytestmark = pytest.mark.gpu

TOL_ABS, TOL_REL = 1e-2, 1e-3
MARGIN = 1e-6


def _check_ulp(out, ref, label):
    """BASELINE bar via check_bf16: max-abs 1e-2 and rel-L2 1e-3 on every element (residual-
    stream values reach |x| >= 2; the largest ulp difference there is reported)."""
    check_bf16(out, ref, label)


def _oracle_stack(oracle_layers, x, gate_beta=None, value_beta=None):
    """Per layer: (top ids, selection margin) and the final hidden state (om.residual_stack)."""
    h = np.asarray(x, dtype=np.uint16)
    routes = []
    for lyr in oracle_layers:
        out, top, _, logits = om.moe_token(lyr.bank, lyr.router, h, gate_beta, value_beta, lyr.shared_id,
                                           lyr.router_f32())
        sc = om.router_scores(logits, lyr.router.score)
        choice = sc if lyr.router.bias is None else sc + lyr.router.bias
        s = np.sort(choice)[::-1]
        routes.append((top, float(s[lyr.router.top_k - 1] - s[lyr.router.top_k])))
        h = f32_to_bf16(bf16_to_f32(h) + bf16_to_f32(out))
    return h, routes


def _small_stack(ctx, n, base, geom=None, score="softmax", bias_seed=None, scaling=1.0):
    geom = geom or G.MoeGeometry(hidden=512, inter=256, n_routed=16, n_shared=1, top_k=4)
    layers, oracle_layers = [], []
    for li in range(n):
        bias = None
        if bias_seed is not None:
            bias = (np.random.default_rng(bias_seed + li).standard_normal(geom.n_routed) * 0.01).astype(np.float32)
        syn = make_layer(geom, seed=base + li, score=score, bias=bias)
        lyr = ctx.create_layer(base + li, geom)
        lyr.upload_experts(syn.gate_up, syn.down)
        lyr.set_router(syn.router, bias=bias, score=score, scaling=scaling)
        layers.append(lyr)
        ol = syn.oracle_layer()
        ol.router.scaling = scaling
        oracle_layers.append(ol)
    return geom, layers, oracle_layers


def test_stack_matches_oracle(gpu_ctx):
    """Eight layers of a small geometry in one launch.  The launch equals eight chained
    1-layer launches bit for bit; every 1-layer launch matches the oracle on the same
    input (routing exact, output within the bar); the first four layers also match the
    free-running oracle stack.  (Free-running over all eight layers, single bf16 rounding
    flips compound through the residual stream past rel-L2 1e-3.)"""
    import torch

    geom, layers, oracle_layers = _small_stack(gpu_ctx, 8, 1200)
    gpu_ctx.reserve_decode_stack(layers)
    xs = random_tokens(5, geom.hidden, 1210)
    s = torch.cuda.current_stream()
    for t, x in enumerate(xs):
        out, top, _ = gpu_ctx.decode_stack(layers, x, residual=True)
        h = x
        for li, (lyr, ol) in enumerate(zip(layers, oracle_layers)):
            got, ids, _ = lyr.moe_decode(h, residual=True)
            ref, rtop, _, logits = om.moe_token(ol.bank, ol.router, h, None, None, ol.shared_id, ol.router_f32())
            ref = f32_to_bf16(bf16_to_f32(h) + bf16_to_f32(ref))
            sc = om.router_scores(logits, "softmax")
            srt = np.sort(sc)[::-1]
            if srt[geom.top_k - 1] - srt[geom.top_k] > MARGIN:
                assert ids.tolist() == rtop.tolist() == top[li].tolist(), (t, li)
            _check_ulp(got, ref, f"token {t} layer {li}")
            h = got
        assert np.array_equal(out, h), f"token {t}: stack differs from chained layers"
        ref4, routes = _oracle_stack(oracle_layers[:4], x)
        out4, top4, _ = gpu_ctx.decode_stack(layers[:4], x, residual=True)
        for li, (rtop, margin) in enumerate(routes):
            if margin > MARGIN:
                assert top4[li].tolist() == rtop.tolist(), (t, li)
        _check_ulp(out4, ref4, f"4-layer stack token {t}")
    for lyr in layers:
        lyr.free()


def test_stack_equals_layer_by_layer(gpu_ctx):
    """BASELINE geometry: a 6-layer launch is bit-identical to six 1-layer launches."""
    import torch

    geom = G.BASELINE
    layers = []
    for li in range(6):
        lyr = gpu_ctx.create_layer(1300 + li, geom)
        lyr.synthesize(77 + li, 0.02)
        gen = torch.Generator(device="cuda").manual_seed(1300 + li)
        rw = (torch.randn(geom.n_routed, geom.hidden, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
        lyr.set_router(rw.contiguous(), score="softmax")
        layers.append(lyr)
    gpu_ctx.reserve_decode_stack(layers)
    x = random_tokens(3, geom.hidden, 1310)
    s = torch.cuda.current_stream()
    for t in range(3):
        h = torch.from_numpy(x[t].view(np.int16)).cuda()
        ids_l = torch.empty((6, geom.top_k), dtype=torch.int32, device="cuda")
        for li, lyr in enumerate(layers):
            nxt = torch.empty_like(h)
            lyr.moe_decode_dev(h, nxt, residual=True, ids_dev=ids_l[li], stream=s)
            h = nxt
        out = torch.empty_like(h)
        ids_s = torch.empty((6, geom.top_k), dtype=torch.int32, device="cuda")
        x_dev = torch.from_numpy(x[t].view(np.int16)).cuda()
        gpu_ctx.decode_stack_dev(layers, x_dev, out, residual=True, ids_dev=ids_s, stream=s)
        torch.cuda.synchronize()
        assert torch.equal(ids_s, ids_l)
        assert torch.equal(out, h), f"token {t}: stack differs from layer-by-layer"
    for lyr in layers:
        lyr.free()


def test_stack_baseline_matches_oracle(gpu_ctx):
    """BASELINE shape (H=2048, I=768, 128 + 1 experts, softmax top-8), 3 layers: the launch
    equals the chained 1-layer launches, and each layer matches the oracle on its input."""
    import torch

    geom = G.BASELINE
    layers, oracle_layers = [], []
    for li in range(3):
        lyr = gpu_ctx.create_layer(1400 + li, geom)
        lyr.synthesize(500 + li, 0.02)
        gen = torch.Generator(device="cuda").manual_seed(1400 + li)
        rw = (torch.randn(geom.n_routed, geom.hidden, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
        router = rw.view(torch.int16).cpu().numpy().view(np.uint16)
        lyr.set_router(router, score="softmax")
        parts = [lyr.download_expert(e) for e in range(geom.n_experts)]
        bank = om.ExpertBank(b"".join(p[0] for p in parts), b"".join(p[1] for p in parts), geom.n_experts,
                             geom.hidden, geom.inter, cache=geom.n_experts)
        oracle_layers.append(om.Layer(bank, om.RouterSpec(router, geom.top_k, score="softmax"), geom.shared_id))
        layers.append(lyr)
    gpu_ctx.reserve_decode_stack(layers)
    for t, x in enumerate(random_tokens(2, geom.hidden, 1410)):
        out, top, _ = gpu_ctx.decode_stack(layers, x, residual=True)
        h = x
        for li, (lyr, ol) in enumerate(zip(layers, oracle_layers)):
            got, ids, _ = lyr.moe_decode(h, residual=True)
            ref, routes = _oracle_stack([ol], h)
            if routes[0][1] > MARGIN:
                assert ids.tolist() == routes[0][0].tolist() == top[li].tolist(), (t, li)
            _check_ulp(got, ref, f"baseline token {t} layer {li}")
            h = got
        assert np.array_equal(out, h), f"token {t}: stack differs from chained layers"
    for lyr in layers:
        lyr.free()


def test_stack_reference_model_shape(gpu_ctx):
    """The reference model's numerics (host/raon.py:1224-1247, host/backend.py:47-62): H=2560,
    I=1088 (down input padded to 1280), top-6, sigmoid router with selection bias and
    routed_scaling_factor 2.5, SiTU-GLU; 3 layers, 16 routed + shared experts."""
    geom = G.MoeGeometry(hidden=2560, inter=1088, n_routed=16, n_shared=1, top_k=6)
    geom, layers, oracle_layers = _small_stack(gpu_ctx, 3, 1500, geom=geom, score="sigmoid", bias_seed=1550,
                                               scaling=2.5)
    gpu_ctx.reserve_decode_stack(layers)
    for t, x in enumerate(random_tokens(2, geom.hidden, 1510)):
        out, top, _ = gpu_ctx.decode_stack(layers, x, residual=True, gate_beta=4.0, value_beta=25.0)
        h = x
        for li, (lyr, ol) in enumerate(zip(layers, oracle_layers)):
            got, ids, _ = lyr.moe_decode(h, residual=True, gate_beta=4.0, value_beta=25.0)
            ref, routes = _oracle_stack([ol], h, 4.0, 25.0)
            if routes[0][1] > MARGIN:
                assert ids.tolist() == routes[0][0].tolist() == top[li].tolist(), (t, li)
            _check_ulp(got, ref, f"reference-shape token {t} layer {li}")
            h = got
        assert np.array_equal(out, h), f"token {t}: stack differs from chained layers"
    for lyr in layers:
        lyr.free()


@pytest.mark.parametrize("score,bias_seed", [("softmax", 1850), ("sigmoid", None)], ids=["softmax-bias", "sigmoid"])
def test_stack_selection_variants(gpu_ctx, score, bias_seed):
    """The selection keys outside the softmax-without-bias fast path (which ranks logits):
    softmax scores plus a selection bias, and sigmoid scores without one.  Three layers in one
    launch equal three chained 1-layer launches bit for bit, and each layer's routing and
    output match the oracle on the same input."""
    geom, layers, oracle_layers = _small_stack(gpu_ctx, 3, 1860 if bias_seed else 1880, score=score,
                                               bias_seed=bias_seed)
    gpu_ctx.reserve_decode_stack(layers)
    for t, x in enumerate(random_tokens(3, geom.hidden, 1830)):
        out, top, _ = gpu_ctx.decode_stack(layers, x, residual=True)
        h = x
        for li, (lyr, ol) in enumerate(zip(layers, oracle_layers)):
            got, ids, _ = lyr.moe_decode(h, residual=True)
            ref, routes = _oracle_stack([ol], h)
            if routes[0][1] > MARGIN:
                assert ids.tolist() == routes[0][0].tolist() == top[li].tolist(), (score, t, li)
            _check_ulp(got, ref, f"{score} token {t} layer {li}")
            h = got
        assert np.array_equal(out, h), f"{score} token {t}: stack differs from chained layers"
    for lyr in layers:
        lyr.free()


def test_stack_graph_replays_match_eager(gpu_ctx):
    """Captured in a HIP graph: every replay equals an eager launch (counters are cleared by
    the kernel itself, so replays need no memset node)."""
    import torch

    geom, layers, _ = _small_stack(gpu_ctx, 4, 1600)
    gpu_ctx.reserve_decode_stack(layers)
    xs = torch.from_numpy(random_tokens(4, geom.hidden, 1610).view(np.int16)).cuda()
    x = xs[0].clone()
    out = torch.empty_like(x)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            gpu_ctx.decode_stack_dev(layers, x, out, residual=True, stream=s)
    torch.cuda.current_stream().wait_stream(s)
    eager = torch.empty_like(x)
    for r in range(4):
        x.copy_(xs[r])
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        gpu_ctx.decode_stack_dev(layers, xs[r], eager, residual=True, stream=torch.cuda.current_stream())
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r}"
    for lyr in layers:
        lyr.free()


def test_stack_wait_timeout_is_reported(gpu_ctx):
    """A wait that gives up is reported with its workgroup, layer and hand-off.  The host
    forces it by lowering the kernel's own poll bound (every workgroup still leaves
    normally: the others see the abort flag); the context is cleared for the next launch,
    which equals the result from before."""
    from raon_npu_amd._lib import RmoeError

    geom, layers, _ = _small_stack(gpu_ctx, 3, 1900)
    gpu_ctx.reserve_decode_stack(layers)
    x = random_tokens(1, geom.hidden, 1910)[0]
    good, top, _ = gpu_ctx.decode_stack(layers, x, residual=True)
    try:
        gpu_ctx.set_stack_wait_limit(1)
        with pytest.raises(RmoeError, match=r"workgroup \d+ gave up at layer \d+ waiting for"):
            gpu_ctx.decode_stack(layers, x, residual=True)
    finally:
        gpu_ctx.set_stack_wait_limit(0)
    again, top2, _ = gpu_ctx.decode_stack(layers, x, residual=True)
    np.testing.assert_array_equal(again, good)
    np.testing.assert_array_equal(top2, top)
    for lyr in layers:
        lyr.free()


def test_stack_rejects_mixed_geometry(gpu_ctx):
    a = gpu_ctx.create_layer(1700, G.MoeGeometry(hidden=512, inter=256, n_routed=16, n_shared=1, top_k=4))
    b = gpu_ctx.create_layer(1701, G.MoeGeometry(hidden=512, inter=128, n_routed=16, n_shared=1, top_k=4))
    rng = np.random.default_rng(0)
    for lyr in (a, b):
        lyr.set_router(f32_to_bf16(rng.standard_normal((16, 512)).astype(np.float32) * 0.02), score="softmax")
    with pytest.raises(ValueError):
        gpu_ctx.reserve_decode_stack([a, b])
    with pytest.raises(KeyError):
        gpu_ctx.reserve_decode_stack([a, 123456])
    a.free()
    b.free()


# ------------------------------------------------------- config 4 at full depth --
N48 = 48


def _baseline_layers(ctx, n, base, seed):
    import torch

    geom = G.BASELINE
    layers = []
    for li in range(n):
        lyr = ctx.create_layer(base + li, geom)
        lyr.synthesize(seed + li, 0.02)
        gen = torch.Generator(device="cuda").manual_seed(seed + li)
        rw = (torch.randn(geom.n_routed, geom.hidden, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
        lyr.set_router(rw.contiguous(), score="softmax")
        layers.append(lyr)
    return geom, layers


@pytest.fixture(scope="module")
def stack48(gpu_ctx):
    """48 BASELINE-shape layers (18.3 GB of q4nx weights) on the device."""
    geom, layers = _baseline_layers(gpu_ctx, N48, 3000, 9100)
    gpu_ctx.reserve_decode_stack(layers)
    yield geom, layers
    for lyr in layers:
        lyr.free()


def _chained(layers, x_dev, stream):
    """48 one-layer launches; returns the input of every layer, the final output and ids."""
    import torch

    k = layers[0].geom.top_k
    ids = torch.empty((len(layers), k), dtype=torch.int32, device="cuda")
    h, inputs = x_dev, []
    for li, lyr in enumerate(layers):
        inputs.append(h)
        nxt = torch.empty_like(h)
        lyr.moe_decode_dev(h, nxt, residual=True, ids_dev=ids[li], stream=stream)
        h = nxt
    return inputs, h, ids


def _stack48_routers(geom, n=N48, seed=9100):
    """The router of each layer of stack48 (bf16 bit patterns), regenerated from its seed."""
    import torch

    routers = []
    for li in range(n):
        gen = torch.Generator(device="cuda").manual_seed(seed + li)
        rw = (torch.randn(geom.n_routed, geom.hidden, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
        routers.append(rw.view(torch.int16).cpu().numpy().view(np.uint16))
    return routers


def test_stack48_equals_chained_layers_and_oracle_routing(gpu_ctx, stack48):
    """One 48-layer persistent launch == 48 chained 1-layer launches bit for bit (outputs and
    routing of every layer), for four tokens; the routing of all 48 layers of every token
    equals the oracle's (host/raon.py:1224-1247) on the GPU's own layer input, apart from
    near-ties (k/k+1 gap <= 1e-6, reported); and the outputs of layers 0, 1, 23, 46 and 47
    of the first token match the oracle within the bar."""
    import torch

    geom, layers = stack48
    s = torch.cuda.current_stream()
    specs = [om.RouterSpec(r, geom.top_k, score="softmax") for r in _stack48_routers(geom)]
    wfs = [sp.weight_f32() for sp in specs]
    n_tok = 4
    xs = random_tokens(n_tok, geom.hidden, 3010, STACK_HIDDEN_STD)
    checked = ties = 0
    for t in range(n_tok):
        x_dev = torch.from_numpy(xs[t].view(np.int16)).cuda()
        inputs, h, ids_l = _chained(layers, x_dev, s)
        out = torch.empty_like(x_dev)
        ids_s = torch.empty_like(ids_l)
        gpu_ctx.decode_stack_dev(layers, x_dev, out, residual=True, ids_dev=ids_s, stream=s)
        torch.cuda.synchronize()
        assert torch.equal(ids_s, ids_l), f"token {t}: routing differs from the chained launches"
        assert torch.equal(out, h), f"token {t}: 48-layer launch differs from the chained launches"
        assert np.all(np.isfinite(bf16_to_f32(out.cpu().numpy().view(np.uint16)))), "residual stream overflowed"
        got_ids = ids_s.cpu().numpy()
        xin_all = [inp.cpu().numpy().view(np.uint16) for inp in inputs]
        for li in range(N48):
            top, _, _ = om.route_token(xin_all[li], specs[li], wfs[li])
            if routing_margin(xin_all[li], specs[li]) > MARGIN:
                assert got_ids[li].tolist() == top.tolist(), f"token {t} layer {li}"
                checked += 1
            else:
                ties += 1
        if t:
            continue
        for li in (0, 1, 23, 46, 47):
            xin = xin_all[li]
            ref, _, _, _ = om.moe_token(LazyBank(layers[li]), specs[li], xin, None, None, shared_id=geom.shared_id)
            got = (inputs[li + 1] if li + 1 < N48 else h).cpu().numpy().view(np.uint16)
            check_bf16(got, f32_to_bf16(bf16_to_f32(xin) + bf16_to_f32(ref)), f"48-stack layer {li}")
    print(f"48-layer routing: {checked} (token, layer) pairs equal the oracle, {ties} near-ties reported")
    assert checked >= n_tok * N48 - 4


def test_stack48_graph_back_to_back(gpu_ctx, stack48):
    """Four 48-layer launches back to back in one HIP graph (no host sync between them),
    each on its own token: every replay's outputs and routing equal eager single launches."""
    import torch

    geom, layers = stack48
    n = 4
    xs = torch.from_numpy(random_tokens(n, geom.hidden, 3020, STACK_HIDDEN_STD).view(np.int16)).cuda()
    outs = torch.empty_like(xs)
    ids = torch.empty((n, N48, geom.top_k), dtype=torch.int32, device="cuda")
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for i in range(n):
                gpu_ctx.decode_stack_dev(layers, xs[i], outs[i], residual=True, ids_dev=ids[i], stream=s)
    torch.cuda.current_stream().wait_stream(s)
    cur = torch.cuda.current_stream()
    eager = torch.empty_like(xs)
    eids = torch.empty_like(ids)
    for i in range(n):
        gpu_ctx.decode_stack_dev(layers, xs[i], eager[i], residual=True, ids_dev=eids[i], stream=cur)
    torch.cuda.synchronize()
    for r in range(3):
        outs.zero_()
        ids.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(outs, eager) and torch.equal(ids, eids), f"replay {r}"
        # eager work between replays
        gpu_ctx.decode_stack_dev(layers, xs[r], eager[r], residual=True, ids_dev=eids[r], stream=cur)
        torch.cuda.synchronize()


def test_stack48_closed_form(gpu_ctx):
    """48 BASELINE-shape layers of constant-weight experts (tests/closed_form.py): every sum
    is exact in any order, so the whole stack has a closed form -- the kernel must equal it
    bit for bit, with each layer routed to its chosen experts at weights 1/8."""
    import torch

    import closed_form as cf

    geom = G.BASELINE
    consts = [cf.make_const_layer(geom.hidden, geom.inter, geom.n_routed, geom.top_k, 4000 + li) for li in range(N48)]
    gu = torch.empty((2 * geom.inter, geom.hidden), dtype=torch.float32, device="cuda")
    dn = torch.empty((geom.hidden, geom.inter), dtype=torch.float32, device="cuda")
    layers = []
    try:
        for li, c in enumerate(consts):
            lyr = gpu_ctx.create_layer(3500 + li, geom)
            layers.append(lyr)
            for e in range(geom.n_experts):
                gu[: geom.inter].fill_(c.cg[e])
                gu[geom.inter:].fill_(c.cu[e])
                dn.fill_(c.cd[e])
                lyr.quantize_expert(e, gu, dn)
            lyr.set_router(c.router_bf16(), score="softmax")
        gpu_ctx.reserve_decode_stack(layers)
        xs = cf.inputs(3, geom.hidden, 4100)
        for t in range(3):
            out, top, w = gpu_ctx.decode_stack(layers, xs[t], residual=True)
            ref = cf.residual_stack(consts, bf16_to_f32(xs[t]))
            for li, c in enumerate(consts):
                assert sorted(top[li].tolist()) == c.chosen, (t, li)
            np.testing.assert_array_equal(w, np.full(w.shape, 1.0 / geom.top_k, np.float32))
            np.testing.assert_array_equal(bf16_to_f32(out), ref)
    finally:
        for lyr in layers:
            lyr.free()


def test_decode_stack_dev_rejects_bad_tensors(gpu_ctx):
    """Every tensor the kernel indexes is checked on the host before any launch."""
    import torch

    geom, layers, _ = _small_stack(gpu_ctx, 2, 1800)
    gpu_ctx.reserve_decode_stack(layers)
    x = torch.zeros(geom.hidden, dtype=torch.int16, device="cuda")
    out = torch.zeros_like(x)
    good_ids = torch.zeros((2, geom.top_k), dtype=torch.int32, device="cuda")
    for kw in (dict(x_dev=x[:-1]), dict(out_dev=torch.zeros(geom.hidden, dtype=torch.float32, device="cuda")),
               dict(ids_dev=torch.zeros(geom.top_k, dtype=torch.int32, device="cuda")),
               dict(wts_dev=torch.zeros((2, geom.top_k), dtype=torch.int32, device="cuda")),
               dict(x_dev=torch.zeros(geom.hidden, dtype=torch.int16))):
        args = dict(x_dev=x, out_dev=out, ids_dev=good_ids, wts_dev=None)
        args.update(kw)
        with pytest.raises(ValueError):
            gpu_ctx.decode_stack_dev(layers, args["x_dev"], args["out_dev"], residual=True, ids_dev=args["ids_dev"],
                                     wts_dev=args["wts_dev"])
    for lyr in layers:
        lyr.free()
