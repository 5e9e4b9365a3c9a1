"""Pins of oracle.bfp16: the reference's hand-computed cases, the integer-contract sample,
and a second, integer-only encoder."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import bfp16 as B
from oracle.bf16 import bf16_round
from oracle.moe import linear


def _encode_int(x: np.ndarray) -> np.ndarray:
    """conv_even bfp16ebs8 encoder written per block with integer arithmetic only: the
    exact value of x_i is sig_i * 2**(max(f_i, 1) - 150) (f_i the fp32 exponent field),
    so m_i = x_i / 2**(e - 133) is sig_i shifted right by e - max(f_i, 1) + 17 bits,
    rounded half to even; e grows by one while a positive m exceeds 127."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, 8)
    out = np.zeros((x.shape[0], 9), dtype=np.uint8)
    for bi, blk in enumerate(x):
        u = blk.view(np.uint32).astype(np.int64)
        f = (u >> 23) & 0xFF
        sig = (u & 0x7FFFFF) | np.where(f != 0, 1 << 23, 0)
        neg = (u >> 31) == 1
        e = int(f.max())
        while True:
            ms = []
            for i in range(8):
                s = e - max(int(f[i]), 1) + 17
                q, rem = int(sig[i]) >> s, int(sig[i]) & ((1 << s) - 1)
                half = 1 << (s - 1)
                if rem > half or (rem == half and (q & 1)):
                    q += 1
                ms.append(-q if neg[i] else q)
            if max(ms) > 127:
                e += 1
                continue
            break
        out[bi, 0] = e
        out[bi, 1:] = np.clip(ms, -128, 127).astype(np.int8).view(np.uint8)
    return out.reshape(-1)


def test_encode_matches_integer_encoder():
    rng = np.random.default_rng(5)
    cases = [
        rng.standard_normal(8 * 400).astype(np.float32),
        (rng.standard_normal(8 * 400) * np.exp(rng.uniform(-30, 30, 8 * 400))).astype(np.float32),
        # rounding midpoints: m + 0.5 at scale 1 (block max 64 fixes e = 133)
        np.tile(np.array([64.0, 0.5, 1.5, 2.5, -0.5, -1.5, 126.5, -3.5], np.float32), 8),
        # carry: 127.6 rounds to 128 -> e + 1; and values just below the carry point
        np.tile(np.array([127.6, -128.0, 127.5, 1.0, 0.25, 63.75, -127.5, 0.0], np.float32), 8),
        np.array([1e-45, 3e-45, 1e-40, 0.0, -1e-45, 2e-39, 5e-41, 1e-44] * 4, np.float32),  # subnormals
    ]
    for x in cases:
        np.testing.assert_array_equal(B.encode(x).reshape(-1), _encode_int(x))


def test_scale_of_every_exponent():
    """bench/gemv_bfp16/test_bfp16_ref.py:199-212: 2**(max(e,7) - 133) exactly."""
    s = B.kernel_scale(np.arange(256))
    for e in range(256):
        assert float(s[e]) == 2.0 ** (max(e, 7) - 133)


def test_raw_block_exponent_boundaries():
    """bench/gemv_bfp16/test_bfp16_ref.py:214-257: e in {0,1,6,7,127,254,255} x m in {1,-128,127,0}."""
    raw = bytearray(B.GEMV_BLOCK_BYTES)
    exps, mants = [0, 1, 6, 7, 127, 254, 255], [1, -128, 127, 0]
    for r, e in enumerate(exps):
        raw[r] = e
    for c, m in enumerate(mants):
        for r in range(len(exps)):
            raw[16 + c * 16 + r] = m & 0xFF
    out = B.decode_block(bytes(raw))
    for r, e in enumerate(exps):
        for c, m in enumerate(mants):
            with np.errstate(over="ignore"):
                want = np.float32(m * 2.0 ** (max(e, 7) - 133))
            got = out[r, c]
            if np.isinf(want):
                assert np.isinf(got) and np.signbit(got) == np.signbit(want)
            else:
                assert got == want


def test_largest_finite_carries_to_255():
    """:259-272: conv_even of float32 max stores e = 255, mantissa 64 -> +inf."""
    blk = np.zeros((1, 8), np.float32)
    blk[0, 0] = np.finfo(np.float32).max
    enc = B.encode(blk)
    assert enc[0, 0] == 255
    assert enc[0, 1:].view(np.int8).tolist() == [64, 0, 0, 0, 0, 0, 0, 0]
    assert np.isposinf(B.decode(enc)[0, 0])


def test_dot_products_at_scale_one():
    """:274-292 and :408-420: sums at scale 1, and -128 * 0.5 = -64."""
    w = np.zeros((128, 256), np.float32)
    w[0, :8] = [1, 2, 3, 4, -1, -2, -3, -4]
    x = np.zeros(256, np.float32)
    x[:8] = 1.0
    wq = B.parse_gemv(B.pack_gemv(w), 256, 128)
    assert linear(wq, x)[0] == 0.0
    x[:8] = [1, 0, 0, 0, 0, 0, 0, 0]
    assert linear(wq, x)[0] == 1.0
    w2 = np.zeros((128, 256), np.float32)
    w2[0, 0] = -128.0
    x2 = np.zeros(256, np.float32)
    x2[0] = 0.5
    assert linear(B.parse_gemv(B.pack_gemv(w2), 256, 128), x2)[0] == -64.0


def test_saturation_at_127():
    """:423-428."""
    x = np.array([127.4, -128.0, 0.0, 1.0, 2.0, 3.0, 4.0, 5.0], np.float32)
    assert np.isfinite(B.decode(B.encode(x))).all()


def test_integer_contract_sample_bit_exact():
    """:473-486: integer weights and inputs -> exact in fp32 -> equals float64 rounded once."""
    rng = np.random.default_rng(1234)
    w = rng.integers(-4, 5, (128, 256)).astype(np.float32)
    x = rng.integers(-4, 5, 256).astype(np.float32)
    wq = B.parse_gemv(B.pack_gemv(w), 256, 128)
    np.testing.assert_array_equal(wq, w)
    y = bf16_round(linear(wq, x))  # the GEMV's epilogue: fp32 sum, one RTNE to bf16
    want = bf16_round((w.astype(np.float64) @ x.astype(np.float64)).astype(np.float32))
    np.testing.assert_array_equal(y, want)


@pytest.mark.parametrize("shape", [(120, 200), (576, 768), (1088, 2560)])
def test_padding_invariance(shape):
    """:436-467: zero padding does not change the active rows."""
    K0, M0 = shape
    rng = np.random.default_rng(777)
    w = rng.standard_normal((M0, K0)).astype(np.float32)
    x = rng.standard_normal(K0).astype(np.float32)
    wp, (m, k) = B.pad(w)
    assert (m, k) == (M0, K0) and wp.shape[0] % 128 == 0 and wp.shape[1] % 256 == 0
    yp = linear(B.parse_gemv(B.pack_gemv(wp), wp.shape[1], wp.shape[0]), np.pad(x, (0, wp.shape[1] - K0)))
    y = linear(B.quantize(w), x)
    np.testing.assert_array_equal(yp[:M0], y)


def test_flush_rules():
    """:295-385: packed exponents are >= 7; tiny and zero blocks become (e=7, m=0); the public
    codec keeps them."""
    w = np.zeros((128, 256), np.float32)
    w[3, :] = 2.0 ** -125
    w[7, :] = 1e-40
    w[9, :] = np.linspace(-1, 1, 256)
    e, m = B.parse_gemv_raw(B.pack_gemv(w), 256, 128)
    assert (e >= 7).all()
    for r in (0, 3, 7):
        assert (e[r] == 7).all() and (m[r] == 0).all()
    assert (B.quantize(w)[3] != 0).any() and (B.quantize(w)[7] != 0).any()
    e_raw, _ = B.parse_gemv_raw(B.pack_gemv(w, flush_tiny=False), 256, 128)
    assert (e_raw[3] < 7).all()


@pytest.mark.parametrize("shape", [(128, 256), (256, 512), (384, 1280)])
def test_pack_parse_roundtrip(shape):
    M, K = shape
    rng = np.random.default_rng(M + K)
    w = (rng.standard_normal((M, K)) * np.exp(rng.uniform(-8, 8, (M, 1)))).astype(np.float32)
    buf = B.pack_gemv(w)
    assert len(buf) == M * K * 9 // 8
    np.testing.assert_array_equal(B.parse_gemv(buf, K, M), B.quantize(w))
    e, m = B.parse_gemv_raw(buf, K, M)
    enc = B.encode(w).reshape(M, K // 8, 9)
    np.testing.assert_array_equal(e, enc[..., 0])
    np.testing.assert_array_equal(m, enc[..., 1:].view(np.int8).reshape(M, K))
    # the block decoder (kernel scale rule) agrees block by block
    blocks = np.frombuffer(buf, np.uint8).reshape(-1, B.GEMV_BLOCK_BYTES)
    full = B.dequantize_packed(buf, K, M)
    np.testing.assert_array_equal(B.decode_block(blocks[0]), full[:32, :256])
    np.testing.assert_array_equal(B.decode_block(blocks[1]), full[32:64, :256])
    if K > 256:
        np.testing.assert_array_equal(B.decode_block(blocks[4]), full[:32, 256:512])
