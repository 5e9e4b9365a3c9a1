"""bfp16ebs8 9-bit weight format (oracle; test infrastructure only).

Restates ``quant/bfp16.py:71-140,216-440`` (codec, GEMV pack / parse) and the kernel's
scale rule of ``kernels/gemv_bfp16/reference.py:25-84`` (``bf16_scale_bits``,
``dequantize_block``).

bfp16ebs8: blocks of 8 consecutive values along the input (K) axis share one exponent
byte ``e``; each value is an int8 mantissa ``m`` and decodes to ``m * 2**(e - 133)``.
Every such value is exact in bf16 (|m| <= 128 has at most 8 significant bits).

GEMV layout (the reference's on-disk / NPU layout, ``pack_bfp16_gemv``): blocks of 32
rows x 256 columns, 9,216 bytes, ordered ``((slice*k_blocks + kb)*4 + r)`` with 128-row
slices.  Inside a block, two halves of 16 rows; per half 32 groups of 144 bytes: 16
exponent bytes (one per row), then 128 mantissa bytes, 8 columns x 16 rows column-major.
With ``flush_tiny`` (the NPU packing rule) every stored exponent is >= 7: a block with
e < 7 is stored as mantissas 0, e = 7.  The kernel decodes with the defensive scale
``2**(max(e, 7) - 133)``.

Pins (tests/test_oracle_bfp16.py):
* the hand-computed cases of ``bench/gemv_bfp16/test_bfp16_ref.py:178-292,408-428``:
  the scale of every exponent 0..255, a raw block with e in {0,1,6,7,127,254,255} and
  m in {1,-128,127,0}, the e = 255 carry of the largest finite float, -128 * 0.5 = -64,
  saturation at +127, dot products at scale 1;
* the integer-contract sample of ``:473-486`` (seed 1234) bit-exact against float64
  rounded once to bf16, padding invariance (``:442-467``), the flush rules (``:295-385``);
* ``bfp16ebs8_encode`` (conv_even) against a second encoder written per block from the
  definition with integer arithmetic only, on random data and on rounding-midpoint and
  carry inputs; ``parse`` against the transpose-free block decoder; pack/parse round trips.
"""

from __future__ import annotations

import numpy as np

BLOCK = 8
BLOCK_BYTES = 9
E_MIN = 7  # NPU packing floor of the stored exponent
M_TILE = 32
K_TILE = 256
GROUPS_PER_TILE = K_TILE // BLOCK  # 32
HALF_ROWS = 16
GROUP_BYTES = HALF_ROWS + HALF_ROWS * BLOCK  # 144
HALF_BYTES = GROUPS_PER_TILE * GROUP_BYTES  # 4608
GEMV_BLOCK_BYTES = 2 * HALF_BYTES  # 9216
_BLOCK_DTYPE = np.dtype([("exponent", np.uint8), ("mantissas", np.int8, (BLOCK,))])


def encode(x, rounding: str = "conv_even") -> np.ndarray:
    """float32 [..., K] -> uint8 [..., K/8*9] (exponent byte, 8 int8 mantissas per block).

    ``quant/bfp16.py:71-125``: e = the largest fp32 exponent field of the block;
    conv_even: m = rint(x / 2**(e-133)) in float64, e += 1 (and requantize) when a
    rounded |m| exceeds 127, then clip to [-128, 127]; floor: the two's-complement of
    the 24-bit significand shifted down by 17 + (e - e_i) bits (-1 / 0 past 31 bits)."""
    if rounding not in ("floor", "conv_even"):
        raise ValueError(f"rounding must be 'floor' or 'conv_even', got {rounding!r}")
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.shape[-1]
    if n % BLOCK:
        raise ValueError(f"last axis {n} is not a multiple of {BLOCK}")
    if not np.isfinite(x).all():
        raise ValueError("inputs must be finite")
    lead = x.shape[:-1]
    bits = x.view(np.uint32).reshape(*lead, n // BLOCK, BLOCK)
    sign = (bits >> 31).astype(bool)
    exp = (bits >> 23) & 0xFF
    emax = exp.max(axis=-1, keepdims=True)
    if rounding == "conv_even":
        blocks = x.reshape(*lead, n // BLOCK, BLOCK).astype(np.float64)
        scale = np.ldexp(1.0, emax.astype(np.int32) - 133)
        v = np.rint(blocks / scale)
        carry = v.max(axis=-1, keepdims=True) > 127
        if carry.any():
            emax = emax + carry.astype(emax.dtype)
            scale = np.where(carry, scale * 2, scale)
            v = np.rint(blocks / scale)
        v = np.clip(v, -128, 127).astype(np.int64)
    else:
        mant = (bits & 0x7FFFFF) | np.where(exp != 0, np.uint32(0x800000), np.uint32(0))
        shift = (emax - exp).astype(np.int64)
        m32 = np.where(sign, (-mant.astype(np.int64)) & 0xFFFFFFFF, mant.astype(np.int64))
        v = ((m32 >> 17) & 0xFF).astype(np.uint8).view(np.int8).astype(np.int64)
        v = v >> np.minimum(shift, 31)
        v = np.where(shift >= 32, np.where(sign, -1, 0), v)
    out = np.empty(lead + (n // BLOCK,), dtype=_BLOCK_DTYPE)
    out["exponent"] = emax[..., 0]
    out["mantissas"] = v
    return out.view(np.uint8).reshape(*lead, n // BLOCK * BLOCK_BYTES)


def decode(b) -> np.ndarray:
    """uint8 [..., n*9] -> float32 [..., n*8]: m * 2**(e-133) in float64, rounded once
    (``quant/bfp16.py:128-140``)."""
    b = np.ascontiguousarray(b, dtype=np.uint8)
    lead = b.shape[:-1]
    blk = b.view(_BLOCK_DTYPE)
    scale = np.ldexp(1.0, blk["exponent"].astype(np.int32) - 133)
    with np.errstate(over="ignore"):
        vals = (blk["mantissas"].astype(np.float64) * scale[..., None]).astype(np.float32)
    return vals.reshape(*lead, b.shape[-1] // BLOCK_BYTES * BLOCK)


def quantize(x, rounding: str = "conv_even") -> np.ndarray:
    """decode(encode(x)) (``quant/bfp16.py:143-180``)."""
    return decode(encode(x, rounding))


def kernel_scale(e) -> np.ndarray:
    """The kernel's scale 2**(max(e, 7) - 133), assembled as bf16 bits (max(e,7) - 6) << 7
    (``kernels/gemv_bfp16/reference.py:25-48``), as float32."""
    e = np.maximum(np.asarray(e, dtype=np.int64), E_MIN)
    return (((e - 6) << 7).astype(np.uint32) << 16).view(np.float32)


def pad(w, m_align: int = 128, k_align: int = 256):
    """Zero-pad [M, K] to multiples of (m_align, k_align); returns (padded, (M, K))
    (``quant/bfp16.py:186-210``)."""
    m, k = w.shape
    pm, pk = (-m) % m_align, (-k) % k_align
    if pm == 0 and pk == 0:
        return w, (m, k)
    out = np.zeros((m + pm, k + pk), dtype=w.dtype)
    out[:m, :k] = w
    return out, (m, k)


def pack_gemv(w_f32, rows: int = 4, rounding: str = "conv_even", flush_tiny: bool = True) -> bytes:
    """float32 [M, K] -> the GEMV byte layout (``quant/bfp16.py:216-329``)."""
    w = np.ascontiguousarray(w_f32, dtype=np.float32)
    M, K = w.shape
    if M % (rows * M_TILE) or K % K_TILE:
        raise ValueError(f"[{M}, {K}] must be multiples of [{rows * M_TILE}, {K_TILE}]")
    blk = encode(w, rounding).view(_BLOCK_DTYPE).reshape(M, K // BLOCK)
    exps = blk["exponent"].copy()
    mants = blk["mantissas"].copy()
    if flush_tiny:
        tiny = exps < E_MIN
        exps[tiny] = E_MIN
        mants[tiny] = 0
    kb_n, slices = K // K_TILE, M // (rows * M_TILE)
    # [slice, kb, r, half, row16, group, col8] -> [slice, kb, r, half, group, (exp16 | col8 x row16)]
    e6 = exps.reshape(slices, rows, 2, HALF_ROWS, kb_n, GROUPS_PER_TILE).transpose(0, 4, 1, 2, 5, 3)
    m7 = mants.reshape(slices, rows, 2, HALF_ROWS, kb_n, GROUPS_PER_TILE, BLOCK).transpose(0, 4, 1, 2, 5, 6, 3)
    out = np.empty((slices, kb_n, rows, 2, GROUPS_PER_TILE, GROUP_BYTES), dtype=np.uint8)
    out[..., :HALF_ROWS] = e6
    out[..., HALF_ROWS:] = m7.reshape(slices, kb_n, rows, 2, GROUPS_PER_TILE, BLOCK * HALF_ROWS).view(np.uint8)
    return out.tobytes()


def parse_gemv_raw(buf, K: int, M: int, rows: int = 4):
    """GEMV bytes -> (exponents uint8 [M, K/8], mantissas int8 [M, K]) (``:332-409``)."""
    b = np.frombuffer(bytes(buf), dtype=np.uint8) if not isinstance(buf, np.ndarray) else buf.astype(np.uint8)
    kb_n, slices = K // K_TILE, M // (rows * M_TILE)
    g = b[: slices * kb_n * rows * GEMV_BLOCK_BYTES].reshape(slices, kb_n, rows, 2, GROUPS_PER_TILE, GROUP_BYTES)
    e = g[..., :HALF_ROWS]  # [s, kb, r, half, group, row16]
    m = g[..., HALF_ROWS:].view(np.int8).reshape(slices, kb_n, rows, 2, GROUPS_PER_TILE, BLOCK, HALF_ROWS)
    exps = e.transpose(0, 2, 3, 5, 1, 4).reshape(M, K // BLOCK)
    mants = m.transpose(0, 2, 3, 6, 1, 4, 5).reshape(M, K)
    return np.ascontiguousarray(exps), np.ascontiguousarray(mants)


def parse_gemv(buf, K: int, M: int, rows: int = 4) -> np.ndarray:
    """GEMV bytes -> float32 [M, K] = m * 2**(e - 133) (``quant/bfp16.py:412-440``)."""
    e, m = parse_gemv_raw(buf, K, M, rows)
    scale = np.repeat(np.ldexp(1.0, e.astype(np.int32) - 133), BLOCK, axis=1)
    with np.errstate(over="ignore"):
        return (m.astype(np.float64) * scale).astype(np.float32)


def decode_block(block) -> np.ndarray:
    """One 9,216-byte block -> float32 [32, 256] with the kernel's scale rule, written from
    the block description (``kernels/gemv_bfp16/reference.py:51-84``)."""
    raw = np.frombuffer(bytes(block)[:GEMV_BLOCK_BYTES], dtype=np.uint8)
    out = np.empty((M_TILE, K_TILE), dtype=np.float32)
    for h in range(2):
        for gi in range(GROUPS_PER_TILE):
            off = h * HALF_BYTES + gi * GROUP_BYTES
            sc = kernel_scale(raw[off : off + HALF_ROWS])
            for c in range(BLOCK):
                col = raw[off + HALF_ROWS + c * HALF_ROWS : off + HALF_ROWS + (c + 1) * HALF_ROWS].view(np.int8)
                with np.errstate(over="ignore"):
                    out[h * HALF_ROWS : (h + 1) * HALF_ROWS, gi * BLOCK + c] = col.astype(np.float32) * sc
    return out


def dequantize_packed(buf, K: int, M: int, rows: int = 4) -> np.ndarray:
    """The kernel's dequantization of GEMV bytes: m * 2**(max(e,7) - 133), float32 [M, K]."""
    e, m = parse_gemv_raw(buf, K, M, rows)
    scale = np.repeat(kernel_scale(e).astype(np.float64), BLOCK, axis=1)
    with np.errstate(over="ignore"):
        return (m.astype(np.float64) * scale).astype(np.float32)
