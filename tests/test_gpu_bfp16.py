"""GPU: 9-bit bfp16ebs8 matrices -- device re-layout round trips and the GEMV vs the oracle.

Bars: the re-layout is a byte permutation (round trips bit-exact on any bytes); GEMV
outputs within max-abs 1e-2 and rel-L2 1e-3 of the fp32 oracle with >= 99% bit-identical
bf16 (the rest differ by fp32 summation order); integer-valued cases, whose sums are
exact in fp32, bit-exact.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import bfp16 as B
from oracle import moe as om
from oracle.bf16 import bf16_to_f32, f32_to_bf16

from moe_fixtures import compare_bf16

pytestmark = pytest.mark.gpu


def _packed_case(M, K, seed, std=0.02):
    rng = np.random.default_rng(seed)
    w = rng.normal(0.0, std, (M, K)).astype(np.float32)
    blob = B.pack_gemv(w)
    return blob, B.dequantize_packed(blob, K, M), rng


def _random_bytes(M, K, rng, e_lo=118, e_hi=122):
    """Arbitrary GEMV bytes: uniform int8 mantissas, exponents drawn from [e_lo, e_hi]
    (every 144-byte group starts with its 16 exponent bytes)."""
    buf = rng.integers(0, 256, M * K * 9 // 8, dtype=np.uint8)
    grp = buf.reshape(-1, B.GROUP_BYTES)
    grp[:, : B.HALF_ROWS] = rng.integers(e_lo, e_hi + 1, (grp.shape[0], B.HALF_ROWS), dtype=np.uint8)
    return buf


@pytest.mark.parametrize("M,K", [(128, 256), (256, 1280), (384, 2560)])
def test_upload_download_round_trip(gpu_ctx, M, K):
    rng = np.random.default_rng(M + K)
    w = (rng.standard_normal((M, K)) * np.exp(rng.uniform(-6, 6, (M, 1)))).astype(np.float32)
    w[5, :64] = 1e-41  # flushed blocks (e = 7, m = 0)
    blob = B.pack_gemv(w)
    mat = gpu_ctx.upload_matrix(blob, M, K, fmt="bfp16")
    assert mat.nbytes == len(blob) == M * K * 9 // 8
    assert mat.download() == blob
    mat.free()
    raw = rng.integers(0, 256, M * K * 9 // 8, dtype=np.uint8).tobytes()  # any bytes, e < 7 included
    mat = gpu_ctx.upload_matrix(raw, M, K, fmt="bfp16")
    assert mat.download() == raw
    mat.free()


def test_integer_contract_bit_exact(gpu_ctx):
    """bench/gemv_bfp16/test_bfp16_ref.py:473-486: integer weights and inputs, every sum
    exact in fp32 -> the device output equals float64 rounded once to bf16, bit for bit."""
    rng = np.random.default_rng(1234)
    w = rng.integers(-4, 5, (128, 256)).astype(np.float32)
    x = rng.integers(-4, 5, (3, 256)).astype(np.float32)
    mat = gpu_ctx.upload_matrix(B.pack_gemv(w), 128, 256, fmt="bfp16")
    y = mat.linear(f32_to_bf16(x))
    want = f32_to_bf16((x.astype(np.float64) @ w.T.astype(np.float64)).astype(np.float32))
    np.testing.assert_array_equal(y, want)
    mat.free()


def test_exponent_boundaries_through_the_kernel(gpu_ctx):
    """bench/gemv_bfp16/test_bfp16_ref.py:214-257 on the device: a raw block (not from the
    packer) with e in {0,1,6,7,127,254,255} and m in {1,-128,127,0}; one-hot inputs read
    the decoded weights back column by column (each is exact in bf16, or +-inf)."""
    M, K = 128, 256
    raw = bytearray(M * K * 9 // 8)
    exps, mants = [0, 1, 6, 7, 127, 254, 255], [1, -128, 127, 0]
    for r, e in enumerate(exps):
        raw[r] = e
    for c, m in enumerate(mants):
        for r in range(len(exps)):
            raw[16 + c * 16 + r] = m & 0xFF
    mat = gpu_ctx.upload_matrix(bytes(raw), M, K, fmt="bfp16")
    x = np.zeros((4, K), np.uint16)
    for c in range(4):
        x[c, c] = 0x3F80  # bf16 1.0
    y = bf16_to_f32(mat.linear(x))
    for r, e in enumerate(exps):
        for c, m in enumerate(mants):
            with np.errstate(over="ignore"):
                want = np.float32(m * 2.0 ** (max(e, 7) - 133))
            got = y[c, r]
            if np.isinf(want):
                assert np.isinf(got) and np.signbit(got) == np.signbit(want), (e, m, got)
            else:
                assert got == want, (e, m, got, want)
    assert np.all(y[:, len(exps):] == 0)
    mat.free()


# The real model's bfp16 shapes (npu/backend.py:122-135): moe_b2 expert down [2560, 1280],
# shared_gu [2176, 2560], o_proj [2560, 5120], mla_in [1152, 2560], q_b [7680, 768].
@pytest.mark.parametrize("T", [1, 2, 4, 5, 9])
@pytest.mark.parametrize("M,K", [(128, 256), (2560, 1280), (2176, 2560), (2560, 5120), (1152, 2560), (7680, 768)])
def test_gemv_tokens_and_shapes(gpu_ctx, T, M, K):
    blob, wf, rng = _packed_case(M, K, M * 7 + K + T)
    x = f32_to_bf16(rng.standard_normal((T, K)).astype(np.float32))
    mat = gpu_ctx.upload_matrix(blob, M, K, fmt="bfp16")
    y = mat.linear(x)
    ref = om.linear(wf, x)
    err, rel, same = compare_bf16(y, ref)
    print(f"bfp16 {M}x{K} T={T}: max-abs {err:.3e} rel-L2 {rel:.3e} bit-identical {same:.4f}")
    assert err <= 1e-2 and rel <= 1e-3 and same >= 0.99, (err, rel, same)
    mat.free()


def test_gemv_input_padding(gpu_ctx):
    """npu/backend.py:3680-3684: moe_b2 takes I = 1088 inputs zero-padded to K = 1280."""
    blob, wf, rng = _packed_case(2560, 1280, 17)
    x = f32_to_bf16(rng.standard_normal((3, 1088)).astype(np.float32))
    mat = gpu_ctx.upload_matrix(blob, 2560, 1280, fmt="bfp16")
    y = mat.linear(x)
    xp = np.zeros((3, 1280), np.uint16)
    xp[:, :1088] = x
    err, rel, same = compare_bf16(y, om.linear(wf, xp))
    assert err <= 1e-2 and rel <= 1e-3 and same >= 0.99
    mat.free()


def test_gemv_tall_matrix(gpu_ctx):
    """A tall matrix (512 row bands): few K splits, so each wave streams several tiles;
    arbitrary mantissa bytes."""
    M, K = 32768, 2560
    rng = np.random.default_rng(99)
    buf = _random_bytes(M, K, rng)
    mat = gpu_ctx.upload_matrix(buf, M, K, fmt="bfp16")
    x = f32_to_bf16(rng.standard_normal((2, K)).astype(np.float32))
    y = mat.linear(x)
    wf = B.dequantize_packed(buf, K, M)
    err, rel, same = compare_bf16(y, om.linear(wf, x))
    print(f"bfp16 {M}x{K}: max-abs {err:.3e} rel-L2 {rel:.3e} bit-identical {same:.4f}")
    assert err <= 1e-2 and rel <= 1e-3 and same >= 0.99
    mat.free()


def test_gemv_single_split(gpu_ctx):
    """M >= 131072 rows: one workgroup per row band over all of K (no split)."""
    M, K = 131072, 256
    rng = np.random.default_rng(7)
    buf = _random_bytes(M, K, rng)
    mat = gpu_ctx.upload_matrix(buf, M, K, fmt="bfp16")
    x = f32_to_bf16(rng.standard_normal((1, K)).astype(np.float32))
    y = mat.linear(x)
    err, rel, same = compare_bf16(y, om.linear(B.dequantize_packed(buf, K, M), x))
    assert err <= 1e-2 and rel <= 1e-3 and same >= 0.99
    mat.free()


def test_linear_dev_matches_host(gpu_ctx):
    """The device-pointer entry point gives the host entry point's bytes."""
    import torch

    M, K, T = 2176, 2560, 3
    blob, _, rng = _packed_case(M, K, 5)
    mat = gpu_ctx.upload_matrix(blob, M, K, fmt="bfp16")
    x = f32_to_bf16(rng.standard_normal((T, K)).astype(np.float32))
    want = mat.linear(x)
    mat.reserve(T)
    xd = torch.from_numpy(x.view(np.int16)).cuda()
    yd = torch.empty((T, M), dtype=torch.int16, device="cuda")
    mat.linear_dev(xd, T, yd)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(yd.cpu().numpy().view(np.uint16), want)
    mat.free()


def test_upload_rejects_bad_shapes(gpu_ctx):
    with pytest.raises(ValueError):
        gpu_ctx.upload_matrix(bytes(100 * 256 * 9 // 8), 100, 256, fmt="bfp16")  # M % 128
    with pytest.raises(ValueError):
        gpu_ctx.upload_matrix(bytes(128 * 200 * 9 // 8), 128, 200, fmt="bfp16")  # K % 256
    with pytest.raises(ValueError):
        gpu_ctx.upload_matrix(bytes(10), 128, 256, fmt="bfp16")  # size
