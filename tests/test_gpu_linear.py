"""GPU: dense q4nx GEMV (``linear``) vs the oracle (BASELINE config 1 and variants).

Tolerance: max-abs 1e-2 and rel-L2 1e-3 against the fp32 oracle;
additionally >= 99% of outputs must be bit-identical bf16 (the rest differ by
fp32 summation order, one bf16 ulp).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import moe as om
from oracle.bf16 import f32_to_bf16
from oracle.q4nx import dequantize_simple, pack_gemv, quantize

from moe_fixtures import compare_bf16

pytestmark = pytest.mark.gpu


def _case(M, K, seed, std=0.02):
    rng = np.random.default_rng(seed)
    w = rng.normal(0.0, std, (M, K)).astype(np.float32)
    c, s, m = quantize(w)
    return pack_gemv(c, s, m), dequantize_simple(c, s, m), rng


def test_config1_gemv(gpu_ctx):
    # W 768x2048 N(0,0.02), x 1x2048 bf16 N(0,1), seed 0.
    blob, wf, _ = _case(768, 2048, 0)
    rng = np.random.default_rng(0)
    x = f32_to_bf16(rng.standard_normal((1, 2048)).astype(np.float32))
    mat = gpu_ctx.upload_matrix(blob, 768, 2048)
    y = mat.linear(x)
    ref = om.linear(wf, x)
    err, rel, same = compare_bf16(y, ref)
    print(f"config1 max-abs {err:.3e} rel-L2 {rel:.3e} bit-identical {same:.4f}")
    assert err <= 1e-2 and rel <= 1e-3 and same >= 0.99
    mat.free()


@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 9])
# K <= 4096 runs one workgroup per row band (linear_band_kernel); K = 5120 runs the K-split
# kernel with its partials and ordered final sum.
@pytest.mark.parametrize("M,K", [(128, 256), (1536, 2048), (2048, 768), (2176, 2560), (256, 5120)])
def test_gemv_tokens_and_shapes(gpu_ctx, T, M, K):
    blob, wf, rng = _case(M, K, M * 7 + K + T)
    x = f32_to_bf16(rng.standard_normal((T, K)).astype(np.float32))
    mat = gpu_ctx.upload_matrix(blob, M, K)
    y = mat.linear(x)
    ref = np.stack([om.linear(wf, x[t]) for t in range(T)])
    err, rel, same = compare_bf16(y, ref)
    assert err <= 1e-2 and rel <= 1e-3 and same >= 0.99, (err, rel, same)
    mat.free()


def test_gemv_input_padding(gpu_ctx):
    # npu/backend.py:3680-3684: a narrower input is zero-padded to the bundle K.
    blob, wf, rng = _case(256, 1280, 17)
    x = f32_to_bf16(rng.standard_normal((3, 1088)).astype(np.float32))
    mat = gpu_ctx.upload_matrix(blob, 256, 1280)
    y = mat.linear(x)
    xp = np.zeros((3, 1280), np.uint16)
    xp[:, :1088] = x
    ref = np.stack([om.linear(wf, r) for r in xp])
    err, rel, _ = compare_bf16(y, ref)
    assert err <= 1e-2 and rel <= 1e-3
    mat.free()


def test_gemv_extreme_inputs(gpu_ctx):
    # zero weights/inputs, large magnitudes, exact cancellations
    M, K = 128, 512
    rng = np.random.default_rng(23)
    w = rng.normal(0, 1.0, (M, K)).astype(np.float32)
    w[:8] = 0.0
    c, s, m = quantize(w)
    mat = gpu_ctx.upload_matrix(pack_gemv(c, s, m), M, K)
    wf = dequantize_simple(c, s, m)
    x = np.zeros((4, K), np.uint16)
    x[1] = f32_to_bf16(np.full(K, 3.0e3, np.float32))
    x[2] = f32_to_bf16(rng.standard_normal(K).astype(np.float32) * 1e-20)
    x[3, ::2] = f32_to_bf16(np.ones(K // 2, np.float32))
    x[3, 1::2] = f32_to_bf16(-np.ones(K // 2, np.float32))
    y = mat.linear(x)
    assert np.all(y[0] == 0)
    for t in range(1, 4):
        ref = om.linear(wf, x[t])
        a = y[t].view(np.int16).astype(np.int32)
        b = ref.view(np.int16).astype(np.int32)
        rel = np.abs(om.bf16_to_f32(y[t]) - om.bf16_to_f32(ref)) / np.maximum(np.abs(om.bf16_to_f32(ref)), 1e-30)
        assert np.mean(a == b) >= 0.95 and np.median(rel) < 1e-2
    mat.free()


# One token of a matrix with fewer than 32 row bands and 4, 8, 16 or 32 K tiles runs
# linear_lane_kernel (two lanes per K tile, x straight from memory, group sums on v_dot2).
@pytest.mark.parametrize("M,K", [(128, 512), (256, 1024), (128, 4096), (1920, 2048), (384, 2048)])
def test_gemv_single_token_lane_kernel(gpu_ctx, M, K):
    blob, wf, rng = _case(M, K, M * 11 + K)
    x = f32_to_bf16(rng.standard_normal((1, K)).astype(np.float32))
    mat = gpu_ctx.upload_matrix(blob, M, K)
    y = mat.linear(x)
    ref = om.linear(wf, x[0])[None]
    err, rel, same = compare_bf16(y, ref)
    assert err <= 1e-2 and rel <= 1e-3 and same >= 0.99, (err, rel, same)
    mat.free()


def test_gemv_single_token_extreme_inputs(gpu_ctx):
    # The extreme rows of test_gemv_extreme_inputs, one token per call (the lane kernel).
    M, K = 128, 512
    rng = np.random.default_rng(23)
    w = rng.normal(0, 1.0, (M, K)).astype(np.float32)
    w[:8] = 0.0
    c, s, m = quantize(w)
    mat = gpu_ctx.upload_matrix(pack_gemv(c, s, m), M, K)
    wf = dequantize_simple(c, s, m)
    rows = [np.zeros(K, np.uint16), f32_to_bf16(np.full(K, 3.0e3, np.float32)),
            f32_to_bf16(rng.standard_normal(K).astype(np.float32) * 1e-20)]
    alt = np.zeros(K, np.uint16)
    alt[::2] = f32_to_bf16(np.ones(K // 2, np.float32))
    alt[1::2] = f32_to_bf16(-np.ones(K // 2, np.float32))
    rows.append(alt)
    for t, xr in enumerate(rows):
        y = mat.linear(xr[None])[0]
        ref = om.linear(wf, xr)
        if t == 0:
            assert np.all(y == 0)
            continue
        a = y.view(np.int16).astype(np.int32)
        b = ref.view(np.int16).astype(np.int32)
        rel = np.abs(om.bf16_to_f32(y) - om.bf16_to_f32(ref)) / np.maximum(np.abs(om.bf16_to_f32(ref)), 1e-30)
        assert np.mean(a == b) >= 0.95 and np.median(rel) < 1e-2, t
    mat.free()
