"""Oracle pins for the Q4_K -> q4nx mapping (quant/gguf_q4k.py:189-243).

Known answers restated from the reference's own tests (quant/test_gguf_q4k.py:20-72),
a per-element brute force of llama.cpp's block layout, and torch's bf16 rounding as an
independent RNE for the group parameters.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import q4k
from oracle.q4nx import dequantize_simple, pack_gemv, parse_gemv


def _pack_scale_min(scale: np.ndarray, minimum: np.ndarray) -> np.ndarray:
    """Inverse of the 6-bit packing, written from llama.cpp's get_scale_min_k4 layout
    (the same construction as quant/test_gguf_q4k.py:20-26)."""
    out = np.zeros(12, dtype=np.uint8)
    out[:4] = (scale[:4] & 0x3F) | ((scale[4:] >> 4) << 6)
    out[4:8] = (minimum[:4] & 0x3F) | ((minimum[4:] >> 4) << 6)
    out[8:12] = (scale[4:] & 0x0F) | ((minimum[4:] & 0x0F) << 4)
    return out


def test_unpack_known_answer():
    """quant/test_gguf_q4k.py:29-41."""
    scale = np.array([0, 1, 31, 63, 4, 20, 40, 60], dtype=np.uint8)
    minimum = np.array([63, 32, 17, 0, 3, 19, 35, 51], dtype=np.uint8)
    got_s, got_m = q4k.unpack_scale_min(_pack_scale_min(scale, minimum))
    np.testing.assert_array_equal(got_s, scale)
    np.testing.assert_array_equal(got_m, minimum)
    qs = np.arange(128, dtype=np.uint8)
    codes = q4k.unpack_codes(qs)
    for pair in range(4):
        np.testing.assert_array_equal(codes[pair * 2], qs[pair * 32:(pair + 1) * 32] & 15)
        np.testing.assert_array_equal(codes[pair * 2 + 1], qs[pair * 32:(pair + 1) * 32] >> 4)


def _finite_blocks(n: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, size=(n, 144), dtype=np.uint8)
    b[:, 0:2] = (rng.uniform(1e-4, 0.2, n) * rng.choice([-1, 1], n)).astype("<f2").view(np.uint8).reshape(n, 2)
    b[:, 2:4] = rng.uniform(1e-4, 0.2, n).astype("<f2").view(np.uint8).reshape(n, 2)
    return b


def test_to_q4nx_preserves_codes_and_only_rounds_parameters():
    """quant/test_gguf_q4k.py:44-72: codes kept; the change against llama.cpp's
    dequantization is bounded by the two bf16 parameter roundings."""
    rng = np.random.default_rng(20261028)
    blocks = np.zeros((7, 144), dtype=np.uint8)
    blocks[:, 0:2] = np.array([0.001953125, 0.00390625, 0.0078125, 0.015625, 0.03125, 0.0625, 0.125],
                              dtype="<f2").view(np.uint8).reshape(7, 2)
    blocks[:, 2:4] = np.array([0.0029296875, 0.005859375, 0.01171875, 0.0234375, 0.046875, 0.09375, 0.1875],
                              dtype="<f2").view(np.uint8).reshape(7, 2)
    blocks[:, 4:] = rng.integers(0, 256, size=(7, 140), dtype=np.uint8)
    codes, scales, mins = q4k.to_q4nx(blocks)
    reference = q4k.dequantize(blocks)
    converted = dequantize_simple(codes, scales, mins)
    np.testing.assert_array_equal(codes.reshape(7, 8, 32), q4k.unpack_codes(blocks[:, 16:]))
    us, um = q4k.unpack_scale_min(blocks[:, 4:16])
    d = blocks[:, :2].copy().reshape(-1).view("<f2").astype(np.float32)
    dmin = blocks[:, 2:4].copy().reshape(-1).view("<f2").astype(np.float32)
    exact_s = d[:, None] * us
    exact_m = -dmin[:, None] * um
    bound = np.abs(exact_s - scales)[..., None] * codes.reshape(7, 8, 32) + np.abs(exact_m - mins)[..., None] + 2e-6
    assert np.all(np.abs(reference.reshape(7, 8, 32) - converted.reshape(7, 8, 32)) <= bound)


def test_dequantize_matches_bytewise_brute_force():
    blocks = _finite_blocks(24, 77)
    got = q4k.dequantize(blocks)
    for i in range(blocks.shape[0]):
        want = q4k.brute_force_dequantize(blocks[i].tobytes()).astype(np.float32)
        np.testing.assert_array_equal(got[i], want)


def test_parameters_are_torch_bf16_of_exact_products():
    torch = pytest.importorskip("torch")
    blocks = _finite_blocks(64, 78)
    _, scales, mins = q4k.to_q4nx(blocks)
    d, dmin, sc, mn, _ = q4k.fields(blocks)
    ps = torch.from_numpy((d[:, None].astype(np.float64) * sc).astype(np.float32)).to(torch.bfloat16).float().numpy()
    pm = torch.from_numpy((-dmin[:, None].astype(np.float64) * mn).astype(np.float32)).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(scales, ps)
    np.testing.assert_array_equal(mins, pm)


def test_matrix_mapping_survives_gemv_packing():
    """Row-major tensor [M, K]: super-blocks run along each row; the q4nx components go
    through pack_gemv / parse_gemv unchanged (quant/test_gguf_q4k.py:75-85 uses the decode
    packer the same way)."""
    M, K = 128, 512
    raw = _finite_blocks(M * K // 256, 79)
    codes, scales, mins = q4k.matrix_to_q4nx(raw, M, K)
    assert codes.shape == (M, K) and scales.shape == (M, K // 32)
    # row r, columns 256b..256b+255 come from super-block r*(K/256) + b
    c2, s2, m2 = q4k.to_q4nx(raw)
    np.testing.assert_array_equal(codes[3, 256:512], c2[3 * 2 + 1])
    np.testing.assert_array_equal(scales[5, 8:16], s2[5 * 2 + 1])
    back = parse_gemv(pack_gemv(codes, scales, mins), K, M)
    np.testing.assert_array_equal(back[0], codes)
    np.testing.assert_array_equal(back[1], scales)
    np.testing.assert_array_equal(back[2], mins)
    with pytest.raises(ValueError):
        q4k.matrix_to_q4nx(raw, M, 300)
