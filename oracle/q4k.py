"""llama.cpp Q4_K blocks and their q4nx mapping (oracle; test infrastructure only).

Restates ``quant/gguf_q4k.py:189-243`` (``unpack_q4_k_scale_min``,
``unpack_q4_k_codes``, ``_q4_k_fields``, ``q4_k_blocks_to_q4nx``,
``dequantize_q4_k_blocks``).

A Q4_K super-block covers 256 consecutive weights of a row in 144 bytes:
``d`` (fp16), ``dmin`` (fp16), 12 bytes holding eight 6-bit scales and eight 6-bit
mins, then 128 bytes of 4-bit codes.  Sub-block ``j`` (32 weights) dequantizes to
``d*sc[j]*q - dmin*mn[j]`` (llama.cpp ``dequantize_row_q4_K``).  The q4nx mapping
keeps every code and rounds the two group parameters to bf16 (RNE):
``scale = bf16(d*sc[j])``, ``min = bf16(-dmin*mn[j])``; both products are exact in
fp32 (an 11-bit fp16 mantissa times a 6-bit integer), so the bf16 rounding is the only
rounding.

Pins (tests/test_oracle_q4k.py):
* the 6-bit packing: the known answer and the independent inverse packer of
  ``quant/test_gguf_q4k.py:20-36``;
* the code order: the ``arange(128)`` known answer of ``quant/test_gguf_q4k.py:38-41``;
* the mapping: codes preserved and the difference to llama.cpp's dequantization
  bounded by the two parameter roundings, ``quant/test_gguf_q4k.py:44-72``; and, for
  what those leave open, a brute-force per-element restatement of llama.cpp's
  bit layout (read bit by bit from the 144 bytes) that a transposed index or a swapped
  nibble half fails.
"""

from __future__ import annotations

import numpy as np

from .bf16 import bf16_to_f32, f32_to_bf16

QK_K = 256
BLOCK_BYTES = 144


def unpack_scale_min(packed) -> tuple[np.ndarray, np.ndarray]:
    """12-byte K-scale field -> (scale u8[..., 8], min u8[..., 8]); ``quant/gguf_q4k.py:189-200``."""
    p = np.asarray(packed, dtype=np.uint8)
    if p.shape[-1] != 12:
        raise ValueError(f"Q4_K scale field must be 12 bytes, got {p.shape}")
    sc = np.empty(p.shape[:-1] + (8,), dtype=np.uint8)
    mn = np.empty_like(sc)
    sc[..., :4] = p[..., 0:4] & 0x3F
    mn[..., :4] = p[..., 4:8] & 0x3F
    sc[..., 4:] = (p[..., 8:12] & 0x0F) | ((p[..., 0:4] >> 6) << 4)
    mn[..., 4:] = (p[..., 8:12] >> 4) | ((p[..., 4:8] >> 6) << 4)
    return sc, mn


def unpack_codes(qs) -> np.ndarray:
    """128 code bytes -> u8[..., 8, 32] in sub-block order; ``quant/gguf_q4k.py:203-213``.

    Sub-block ``2p`` is the low nibbles of bytes ``32p..32p+31``, sub-block ``2p+1``
    their high nibbles.
    """
    q = np.asarray(qs, dtype=np.uint8)
    if q.shape[-1] != 128:
        raise ValueError(f"Q4_K code field must be 128 bytes, got {q.shape}")
    q = q.reshape(q.shape[:-1] + (4, 32))
    out = np.empty(q.shape[:-2] + (8, 32), dtype=np.uint8)
    out[..., 0::2, :] = q & 0x0F
    out[..., 1::2, :] = q >> 4
    return out


def fields(blocks):
    """``(d f32[N], dmin f32[N], sc u8[N,8], mn u8[N,8], codes u8[N,8,32])``; ``quant/gguf_q4k.py:216-225``."""
    b = np.asarray(blocks, dtype=np.uint8)
    if b.ndim != 2 or b.shape[1] != BLOCK_BYTES:
        raise ValueError(f"Q4_K blocks must have shape [N, 144], got {b.shape}")
    d = b[:, 0:2].copy().reshape(-1).view("<f2").astype(np.float32)
    dmin = b[:, 2:4].copy().reshape(-1).view("<f2").astype(np.float32)
    sc, mn = unpack_scale_min(b[:, 4:16])
    return d, dmin, sc, mn, unpack_codes(b[:, 16:144])


def to_q4nx(blocks) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Q4_K blocks [N, 144] -> q4nx ``(codes u8[N, 256], scales f32[N, 8], mins f32[N, 8])``.

    ``quant/gguf_q4k.py:228-233``: codes kept, ``scale = bf16(d*sc)``, ``min = bf16(-dmin*mn)``.
    """
    d, dmin, sc, mn, codes = fields(blocks)
    scales = bf16_to_f32(f32_to_bf16(d[:, None] * sc.astype(np.float32)))
    mins = bf16_to_f32(f32_to_bf16(-dmin[:, None] * mn.astype(np.float32)))
    return codes.reshape(-1, QK_K), scales, mins


def dequantize(blocks) -> np.ndarray:
    """llama.cpp ``dequantize_row_q4_K`` in fp32: [N, 144] -> [N, 256]; ``quant/gguf_q4k.py:236-243``."""
    d, dmin, sc, mn, codes = fields(blocks)
    v = (d[:, None, None] * sc[..., None].astype(np.float32) * codes.astype(np.float32)
         - dmin[:, None, None] * mn[..., None].astype(np.float32))
    return v.reshape(-1, QK_K).astype(np.float32)


def matrix_to_q4nx(raw, M: int, K: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """A row-major Q4_K tensor [M, K] (K % 256 == 0; super-blocks along each row) ->
    q4nx ``(codes u8[M, K], scales f32[M, K/32], mins f32[M, K/32])``."""
    if K % QK_K:
        raise ValueError(f"Q4_K rows must be a multiple of {QK_K} wide, got K={K}")
    b = np.frombuffer(bytes(raw) if not isinstance(raw, np.ndarray) else raw.tobytes(), dtype=np.uint8)
    nb = M * (K // QK_K)
    if b.size != nb * BLOCK_BYTES:
        raise ValueError(f"Q4_K tensor [{M}, {K}] needs {nb * BLOCK_BYTES} bytes, got {b.size}")
    codes, scales, mins = to_q4nx(b.reshape(nb, BLOCK_BYTES))
    return codes.reshape(M, K), scales.reshape(M, K // 32), mins.reshape(M, K // 32)


def brute_force_dequantize(block: bytes) -> np.ndarray:
    """One super-block, element by element from the bytes: weight ``32j + c`` reads the
    nibble of byte ``16 + 32*(j//2) + c`` (low for even j), the 6-bit scale/min of
    sub-block j (bytes 4..15: j < 4 low six bits of bytes 4+j / 8+j; j >= 4 the nibbles
    of byte 12+(j-4) joined with the top two bits of bytes 4+(j-4) / 8+(j-4)), and
    evaluates ``d*sc*q - dmin*mn`` in float64 (the fp32 products are exact)."""
    raw = bytes(block)
    d = float(np.frombuffer(raw[0:2], dtype="<f2")[0])
    dmin = float(np.frombuffer(raw[2:4], dtype="<f2")[0])
    out = np.empty(QK_K, dtype=np.float64)
    for j in range(8):
        if j < 4:
            sc = raw[4 + j] & 0x3F
            mn = raw[8 + j] & 0x3F
        else:
            sc = (raw[12 + j - 4] & 0x0F) | ((raw[4 + j - 4] >> 6) << 4)
            mn = (raw[12 + j - 4] >> 4) | ((raw[8 + j - 4] >> 6) << 4)
        for c in range(32):
            byte = raw[16 + 32 * (j // 2) + c]
            q = (byte & 0x0F) if j % 2 == 0 else (byte >> 4)
            out[32 * j + c] = d * sc * q - dmin * mn
    return out
