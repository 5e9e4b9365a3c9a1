"""Pins of oracle.q4nx: reference golden hashes, known answers and properties."""

from __future__ import annotations

import hashlib
import json
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from oracle.bf16 import bf16_round
from oracle.q4nx import (
    GROUP,
    dequantize_packed,
    dequantize_simple,
    pack_gemv,
    pad,
    parse_gemv,
    quantize,
)

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


@pytest.mark.parametrize("case", GOLDEN["pack_gemv_sha256"], ids=lambda c: f"{c['M']}x{c['K']}")
def test_pack_gemv_reference_sha256(case):
    rng = np.random.default_rng(case["seed"])
    w = rng.standard_normal((case["M"], case["K"])).astype(np.float32)
    blob = pack_gemv(*quantize(w))
    assert len(blob) == case["bytes"]
    assert hashlib.sha256(blob).hexdigest() == case["sha256"]


def test_pack_parse_round_trip_and_independent_decoder():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((256, 512)) * 0.02).astype(np.float32)
    c, s, m = quantize(w)
    blob = pack_gemv(c, s, m)
    c2, s2, m2 = parse_gemv(blob, K=512, M=256)
    np.testing.assert_array_equal(c2, c)
    np.testing.assert_array_equal(s2, s)
    np.testing.assert_array_equal(m2, m)
    # A second decoder written from the block description (kernels/gemv/reference.py:34-67).
    dec = dequantize_packed(blob, K=512, M=256)
    np.testing.assert_array_equal(dec.astype(np.float32), dequantize_simple(c, s, m))


def test_dequant_hand_calculated():
    h = GOLDEN["dequant_hand_case"]
    M, K = h["M"], h["K"]
    codes = np.full((M, K), h["code"], np.uint8)
    scales = np.full((M, K // GROUP), h["scale"], np.float32)
    mins = np.full((M, K // GROUP), h["min"], np.float32)
    blob = pack_gemv(codes, scales, mins)
    w = dequantize_packed(blob, K=K, M=M)
    assert np.all(w == h["weight"])
    assert np.all(w @ np.ones(K) == h["y_for_ones"])


def test_dequantize_simple_is_single_rounding_of_exact_fma():
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((64, 256)) * rng.uniform(1e-3, 10)).astype(np.float32)
    c, s, m = quantize(w)
    deq = dequantize_simple(c, s, m)
    idx = rng.integers(0, c.size, 400)
    for i in idx:
        r, k = divmod(int(i), c.shape[1])
        exact = Fraction(float(m[r, k // GROUP])) + Fraction(float(s[r, k // GROUP])) * int(c[r, k])
        assert np.float32(float(exact)) == deq[r, k]


def test_quantize_error_bound_and_grid():
    rng = np.random.default_rng(2026)
    w = rng.standard_normal((64, 512)).astype(np.float32) * 2.5
    c, s, m = quantize(w)
    assert c.dtype == np.uint8 and c.max() <= 15
    assert np.all(bf16_round(s) == s) and np.all(bf16_round(m) == m)
    rec = dequantize_simple(c, s, m)
    assert np.all(np.abs(w - rec) <= 0.5 * np.repeat(s, GROUP, axis=-1) + 1e-6)
    # coverage: min + 15*scale >= max per group (quant/q4nx.py:178-184)
    g = w.reshape(64, -1, GROUP)
    assert np.all(m.astype(np.float64) + 15.0 * s.astype(np.float64) >= g.max(-1))


def test_quantize_edge_cases():
    w = np.zeros((32, 128), np.float32)
    w[:, 32:64] = 5.0
    w[:, 64:96] = -12.5
    w[:, 96:] = np.linspace(1.0, 10.0, 32, dtype=np.float32)
    c, s, m = quantize(w)
    assert np.all(s[:, :3] == 0.0) and np.all(s[:, 3] > 0)
    assert np.all(c[:, :96] == 0)
    # inexact constant group (0.1 is not a bf16 value)
    c2, s2, _ = quantize(np.full((32, 32), 0.1, np.float32))
    assert np.all(s2 > 0) and c2.max() <= 15
    for bad in (np.nan, np.inf, -np.inf):
        x = np.ones((32, 64), np.float32)
        x[0, 10] = bad
        with pytest.raises(ValueError, match="non-finite"):
            quantize(x)
    with pytest.raises(ValueError, match="multiple of GROUP"):
        quantize(np.ones((32, 45), np.float32))
    with pytest.raises(ValueError, match="multiple of 128"):
        pack_gemv(np.zeros((100, 256), np.uint8), np.zeros((100, 8), np.float32), np.zeros((100, 8), np.float32))


def test_padding_invariance():
    # bench/gemv/test_gemv_ref.py:306-346: zero x past K_orig contributes nothing.
    rng = np.random.default_rng(9999)
    w = rng.standard_normal((2100, 576)).astype(np.float32)
    x = rng.standard_normal(576).astype(np.float32)
    wp, shape = pad(w, 128, 256)
    assert wp.shape == (2176, 768) and shape == (2100, 576)
    deq = dequantize_simple(*quantize(wp)).astype(np.float64)
    xp = np.pad(x, (0, 192)).astype(np.float64)
    np.testing.assert_allclose((deq @ xp)[:2100], deq[:2100, :576] @ x.astype(np.float64), rtol=1e-12, atol=1e-12)


def test_dequantize_grouped_equals_simple():
    from oracle.q4nx import dequantize_grouped

    rng = np.random.default_rng(77)
    w = (rng.standard_normal((96, 512)) * np.exp2(rng.integers(-20, 20, (96, 1)))).astype(np.float32)
    c, s, m = quantize(w)
    assert np.array_equal(dequantize_grouped(c, s, m), dequantize_simple(c, s, m))
