"""Pins of oracle.bf16 against a library routine (torch's RNE conversion) and brute force."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_ceil, bf16_floor, bf16_next_up, bf16_round, bf16_to_f32, f32_to_bf16


def _torch_bf16_bits(x: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def test_rne_matches_torch_on_random_bit_patterns():
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    np.testing.assert_array_equal(f32_to_bf16(x), _torch_bf16_bits(x))


def test_rne_ties_and_nan_known_answers():
    # quant/test_q4nx.py:521-532
    assert f32_to_bf16(np.array([1.0 + 2**-8], np.float32))[0] == 0x3F80
    assert f32_to_bf16(np.array([1.0 + 2**-7 + 2**-8], np.float32))[0] == 0x3F82
    nan_payloads = np.array([0x7FC00000, 0x7F800001, 0xFFC00001, 0x7FFFFFFF], dtype=np.uint32).view(np.float32)
    assert np.all(f32_to_bf16(nan_payloads) == 0x7FC0)
    assert f32_to_bf16(np.array([np.inf], np.float32))[0] == 0x7F80
    assert f32_to_bf16(np.array([-np.inf], np.float32))[0] == 0xFF80


def test_bf16_to_f32_is_exact_high_half():
    u = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = bf16_to_f32(u)
    assert np.array_equal(f.view(np.uint32) >> 16, u.astype(np.uint32))
    assert np.array_equal(f.view(np.uint32) & 0xFFFF, np.zeros(65536, np.uint32))


def _all_finite_bf16() -> np.ndarray:
    v = bf16_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    v = v[np.isfinite(v)]
    return np.unique(v.astype(np.float64))  # -0 and +0 merge


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_directed_rounding_brute_force(dtype):
    grid = _all_finite_bf16()
    rng = np.random.default_rng(11)
    # Values across the range, ties on the grid, and near-grid values.
    mags = np.exp(rng.uniform(np.log(1e-38), np.log(3e38), 20000)) * rng.choice([-1.0, 1.0], 20000)
    onto = rng.choice(grid, 2000)
    x = np.concatenate([mags, onto, onto * (1 + 2**-20), onto * (1 - 2**-20), [0.0, 1001.1, -1001.1]]).astype(dtype)
    x = x[np.isfinite(x) & (np.abs(x.astype(np.float64)) <= grid[-1])]
    xf = x.astype(np.float64)
    fl = np.asarray(bf16_floor(x), dtype=np.float64)
    ce = np.asarray(bf16_ceil(x), dtype=np.float64)
    i_fl = np.searchsorted(grid, xf, side="right") - 1
    i_ce = np.searchsorted(grid, xf, side="left")
    np.testing.assert_array_equal(fl, grid[i_fl])
    np.testing.assert_array_equal(ce, grid[i_ce])
    assert np.all(bf16_round(fl.astype(np.float32)) == fl.astype(np.float32))


def test_next_up_is_successor_on_the_grid():
    grid = _all_finite_bf16()
    nxt = np.asarray(bf16_next_up(grid[:-1].astype(np.float32)), dtype=np.float64)
    np.testing.assert_array_equal(nxt, grid[1:])
    # -0 is treated as +0 (quant/q4nx.py:116)
    assert bf16_next_up(np.float32(-0.0)) == bf16_to_f32(np.array([1], np.uint16))[0]
