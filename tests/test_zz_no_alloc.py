"""GPU: rmoe_moe_experts_static_dev, the routed-expert decode entry point that allocates
nothing (its working memory is a static per-device array).

Called through the C ABI and compared with rmoe_moe_experts_dev (context scratch) on two
calls in a row, the second on a smaller layer; both share the decode kernels, so the
outputs are bit-identical, and they match the oracle within the BASELINE bar.  Also:
replays of a HIP graph that captured it, and the rejection of a layer whose scratch
exceeds the static array or whose slots exceed the decode kernels' shape limits.
"""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import raon_npu_amd.geometry as G
from oracle import moe as om

from moe_fixtures import check_bf16, make_layer, random_tokens

pytestmark = pytest.mark.gpu


def _static(lyr, x, ids, wts, out, stream=None, betas=(None, None)):
    """The new entry point, called through the C ABI as a ctypes binding would."""
    from raon_npu_amd import _lib
    from raon_npu_amd.device import act_code

    act, gb, vb = act_code(*betas)
    st = None if stream is None else stream.cuda_stream
    _lib.call("rmoe_moe_experts_static_dev", lyr.ctx.handle, lyr.layer, C.c_void_p(x.data_ptr()),
              C.c_void_p(ids.data_ptr()), C.c_void_p(wts.data_ptr()), int(ids.shape[0]), act, gb, vb,
              C.c_void_p(out.data_ptr()), st)


def _case(torch, lyr, geom, seed, k):
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(random_tokens(1, geom.hidden, seed)[0].view(np.int16)).cuda()
    ids = torch.tensor(rng.choice(geom.n_routed, k, replace=False), dtype=torch.int32, device="cuda")
    wts = torch.tensor(rng.random(k, dtype=np.float32), device="cuda")
    return x, ids, wts


def test_static_scratch_entry_point(gpu_ctx):
    import torch

    s = torch.cuda.current_stream()
    # call 1: BASELINE shape, k = 8
    big = gpu_ctx.create_layer(5100, G.BASELINE)
    big.synthesize(5100, 0.02)
    big.reserve(1)
    x, ids, wts = _case(torch, big, G.BASELINE, 5101, 8)
    ref = torch.empty_like(x)
    got = torch.full_like(x, 0x7FC0)
    big.moe_experts_dev(x, ids, wts, ref, None, None, stream=s)
    _static(big, x, ids, wts, got)
    torch.cuda.synchronize()
    assert torch.equal(got, ref), "static scratch differs from context scratch (BASELINE, k=8)"
    # call 2: a smaller layer (H=512, I=256) and k = 3, SiTU-GLU, on the same static array
    geom = G.MoeGeometry(hidden=512, inter=256, n_routed=16, n_shared=1, top_k=4)
    syn = make_layer(geom, seed=5102)
    small = gpu_ctx.create_layer(5102, geom)
    small.upload_experts(syn.gate_up, syn.down)
    small.reserve(1)
    x2, ids2, wts2 = _case(torch, small, geom, 5103, 3)
    ref2 = torch.empty_like(x2)
    got2 = torch.full_like(x2, 0x7FC0)
    small.moe_experts_dev(x2, ids2, wts2, ref2, 4.0, 25.0, stream=s)
    _static(small, x2, ids2, wts2, got2, betas=(4.0, 25.0))
    torch.cuda.synchronize()
    assert torch.equal(got2, ref2), "static scratch differs from context scratch (small layer, k=3)"
    want = om.moe_experts(syn.bank(), x2.cpu().numpy().view(np.uint16), ids2.cpu().numpy(), wts2.cpu().numpy(),
                          4.0, 25.0)
    check_bf16(got2.cpu().numpy().view(np.uint16), want, "static entry point vs oracle")
    # captured in a HIP graph: every replay equals the eager result
    g = torch.cuda.CUDAGraph()
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    out_g = torch.empty_like(x)
    with torch.cuda.stream(cs):
        with torch.cuda.graph(g, stream=cs):
            _static(big, x, ids, wts, out_g, stream=cs)
    torch.cuda.current_stream().wait_stream(cs)
    for r in range(3):
        out_g.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, ref), f"replay {r}"
        _static(small, x2, ids2, wts2, got2, betas=(4.0, 25.0))  # eager work on the same array between replays
        torch.cuda.synchronize()
        assert torch.equal(got2, ref2)
    big.free()
    small.free()


def test_static_scratch_rejects_oversize(gpu_ctx):
    """A layer whose decode scratch (the activations of its k slots, 16 x 8448 bf16 here)
    exceeds the 256 KiB static array is refused before any launch; so is one within the
    array whose k slots exceed the decode kernels' shape limits (LDS)."""
    import torch

    ids = torch.arange(16, dtype=torch.int32, device="cuda")
    wts = torch.ones(16, dtype=torch.float32, device="cuda")
    geom = G.MoeGeometry(hidden=256, inter=8448, n_routed=16, n_shared=1, top_k=16)
    lyr = gpu_ctx.create_layer(5104, geom)
    x = torch.zeros(geom.hidden, dtype=torch.int16, device="cuda")
    out = torch.empty_like(x)
    with pytest.raises(ValueError, match="static decode scratch"):
        _static(lyr, x, ids, wts, out)
    lyr.free()
    geom = G.MoeGeometry(hidden=4096, inter=2048, n_routed=16, n_shared=1, top_k=16)
    lyr = gpu_ctx.create_layer(5105, geom)
    x = torch.zeros(geom.hidden, dtype=torch.int16, device="cuda")
    out = torch.empty_like(x)
    with pytest.raises(ValueError, match="shape limits"):
        _static(lyr, x, ids, wts, out)
    lyr.free()
