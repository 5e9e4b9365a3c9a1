"""GPU: q4nx upload re-layout round trips and the device quantizer vs the oracle (bit-exact)."""

from __future__ import annotations

import numpy as np
import pytest

from oracle.q4nx import pack_gemv, quantize

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,K", [(128, 256), (768, 2048), (2176, 2560), (2048, 1280), (1536, 2048)])
def test_upload_download_round_trip(gpu_ctx, M, K):
    rng = np.random.default_rng(M + K)
    blob = rng.integers(0, 256, M * K * 5 // 8, dtype=np.uint8)
    # scales/mins are arbitrary bf16 bits: the layout must move every byte unchanged
    mat = gpu_ctx.upload_matrix(blob, M, K)
    assert mat.download() == blob.tobytes()
    mat.free()


def _quantize_on_gpu(gpu_ctx, w):
    import torch

    wd = torch.from_numpy(w).cuda()
    mat = gpu_ctx.quantize_matrix(wd, *w.shape)
    out = mat.download()
    mat.free()
    return out


@pytest.mark.parametrize("M,K,scale", [(128, 256, 0.02), (768, 2048, 0.02), (256, 512, 2.5), (128, 1024, 1e-30)])
def test_device_quantizer_matches_oracle(gpu_ctx, M, K, scale):
    rng = np.random.default_rng(99)
    w = (rng.standard_normal((M, K)) * scale).astype(np.float32)
    assert _quantize_on_gpu(gpu_ctx, w) == pack_gemv(*quantize(w))


def test_device_quantizer_edge_groups(gpu_ctx):
    w = np.zeros((128, 256), np.float32)
    w[:, 32:64] = 5.0
    w[:, 64:96] = -12.5
    w[:, 96:128] = np.linspace(1.0, 10.0, 32, dtype=np.float32)
    w[:, 128:160] = 0.1
    w[0, 160] = -3e38
    w[0, 161] = 3e38
    w[1:, 160:192] = np.linspace(1001.0, 1001.1, 32, dtype=np.float32)
    w[:, 192:] = np.random.default_rng(1).standard_normal((128, 64)).astype(np.float32) * 1e-40
    assert _quantize_on_gpu(gpu_ctx, w) == pack_gemv(*quantize(w))


def test_device_quantizer_rejects_non_finite(gpu_ctx):
    w = np.ones((128, 256), np.float32)
    w[3, 7] = np.nan
    with pytest.raises(ValueError, match="non-finite"):
        _quantize_on_gpu(gpu_ctx, w)


def test_expert_quantizer_pads_down_columns(gpu_ctx):
    import torch

    import raon_npu_amd.geometry as G
    from oracle.q4nx import pad

    geom = G.MoeGeometry(hidden=256, inter=192, n_routed=2, n_shared=1, top_k=1)  # Ipad = 256
    rng = np.random.default_rng(5)
    gu = (rng.standard_normal((2 * geom.inter, geom.hidden)) * 0.02).astype(np.float32)
    dn = (rng.standard_normal((geom.hidden, geom.inter)) * 0.02).astype(np.float32)
    lyr = gpu_ctx.create_layer(900, geom)
    lyr.quantize_expert(1, torch.from_numpy(gu).cuda(), torch.from_numpy(dn).cuda())
    got_gu, got_dn = lyr.download_expert(1)
    assert got_gu == pack_gemv(*quantize(gu))
    assert got_dn == pack_gemv(*quantize(pad(dn, 128, 256)[0]))
    lyr.free()
