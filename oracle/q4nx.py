"""q4nx 4-bit weight format (oracle; test infrastructure only).

Restates ``quant/q4nx.py:22-29,127-248,335-438`` and the independent layout
decoder ``kernels/gemv/reference.py:34-79``.

q4nx: per 32-wide group of input columns, a bf16 ``scale`` and bf16 ``min``; each
weight is a 4-bit code and dequantizes to ``min + scale*code``.

``pack_gemv`` layout (the reference's on-disk / NPU GEMV layout): 32-row x
256-column blocks of 5,120 bytes; block order ``((slice*k_blocks + kb)*4 + r)``
with 128-row slices; inside a block 256 bf16 scales ``[group][row]``, 256 bf16
mins ``[group][row]``, then 4,096 code bytes in ``(half, group, col, row16)``
order, two adjacent rows per byte (low nibble = even row).

Pins:
* ``quantize`` + ``pack_gemv``: the reference's golden SHA-256 values of
  ``bench/gemv/test_gemv_ref.py:62-116`` (seed 1234, 1024x256 and 2048x512),
  plus the error/edge properties of ``quant/test_q4nx.py:111-259``.
* ``parse_gemv``: inverse of ``pack_gemv`` (round trip) and agreement with
  ``decode_block``/``dequantize_packed``, a second decoder written from the
  block description rather than as the transpose of ``pack_gemv``.
* ``dequantize_simple``: the hand-computed case of
  ``bench/gemv/test_gemv_ref.py:204-229`` (code 3, scale 0.5, min 1 -> 2.5;
  y = 640 for x = 1) and, per element, ``fma(scale, code, min)`` evaluated in
  exact rational arithmetic then rounded once (tests/test_oracle_q4nx.py).
"""

from __future__ import annotations

import numpy as np

from .bf16 import bf16_ceil, bf16_floor, bf16_next_up, bf16_to_f32, f32_to_bf16

M_TILE = 32
K_TILE = 256
GROUP = 32
CHUNK_ROWS = 4 * M_TILE  # 128-row slice of pack_gemv
BLOCK_BYTES = M_TILE * K_TILE * 5 // 8  # 5120
SM_BYTES = 2 * 2 * M_TILE * (K_TILE // GROUP)  # 1024


def quantize(w) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """fp32 ``w[N, K]`` -> ``(codes u8[N,K], scales f32[N,K/32], mins f32[N,K/32])``.

    ``quant/q4nx.py:127-200``.  Per group: ``min_q = bf16_floor(min)``; ``scale_q``
    is the smallest bf16 >= ``(max - min_q)/15`` (float64), bumped to the next bf16
    until ``min_q + 15*scale_q >= max`` in float64; a group with ``max == min_q``
    gets scale 0 and codes 0; codes are ``clip(rint((w - min_q)/scale_q), 0, 15)``
    in float64.
    """
    arr = np.asarray(w)
    if arr.ndim != 2:
        raise ValueError(f"Weight matrix must be 2D, got shape {arr.shape}")
    if not np.all(np.isfinite(arr)):
        raise ValueError("Input weight matrix contains non-finite values (NaN or Inf)")
    w32 = arr.astype(np.float32)
    n, k = w32.shape
    if k % GROUP:
        raise ValueError(f"Columns/in-features ({k}) must be a multiple of GROUP ({GROUP})")
    grouped = w32.reshape(n, k // GROUP, GROUP)
    lo = grouped.min(axis=-1)
    hi64 = grouped.max(axis=-1).astype(np.float64)

    min_q = bf16_floor(lo)
    min64 = min_q.astype(np.float64)
    span = hi64 - min64
    scale_q = bf16_ceil(span / 15.0)
    ok = min64 + 15.0 * scale_q.astype(np.float64) >= hi64
    while not ok.all():
        if not np.isfinite(scale_q).all():
            break
        scale_q = np.where(ok, scale_q, bf16_next_up(scale_q))
        ok = min64 + 15.0 * scale_q.astype(np.float64) >= hi64
    flat = span == 0.0
    scale_q[flat] = 0.0
    if not (np.isfinite(min_q).all() and np.isfinite(scale_q).all()):
        raise ValueError("Quantization parameters (scale_q or min_q) overflowed to non-finite values")

    divisor = np.where(flat, 1.0, scale_q.astype(np.float64))
    q = np.rint((grouped.astype(np.float64) - min64[..., None]) / divisor[..., None])
    codes = np.clip(q, 0, 15).astype(np.uint8)
    codes[np.broadcast_to(flat[..., None], codes.shape)] = 0
    return codes.reshape(n, k), scale_q.astype(np.float32), min_q.astype(np.float32)


def dequantize_simple(codes, scales, mins) -> np.ndarray:
    """``min + scale*code`` in float64, rounded once to float32. ``quant/q4nx.py:203-223``."""
    c = np.asarray(codes)
    g = np.arange(c.shape[1]) // GROUP
    s = np.asarray(scales)[:, g].astype(np.float64)
    m = np.asarray(mins)[:, g].astype(np.float64)
    return (m + s * c.astype(np.float64)).astype(np.float32)


def dequantize_grouped(codes, scales, mins) -> np.ndarray:
    """``dequantize_simple`` by group broadcasting instead of a column gather: the same
    float64 values rounded once to float32 (bit-identical; tests/test_oracle_q4nx.py), a
    few times faster.  Used only to pre-dequantize weights outside timed regions."""
    c = np.asarray(codes)
    n, k = c.shape
    s = np.asarray(scales, np.float64)[:, :, None]
    m = np.asarray(mins, np.float64)[:, :, None]
    return (m + s * c.reshape(n, k // GROUP, GROUP)).astype(np.float32).reshape(n, k)


def pad(w, m_tile: int = 32, k_tile: int = 256):
    """Zero-pad rows to a multiple of ``m_tile`` and columns to ``k_tile``. ``quant/q4nx.py:226-248``."""
    a = np.asarray(w)
    if a.ndim != 2:
        raise ValueError(f"pad requires 2D array, got shape {a.shape}")
    r, c = a.shape
    pr, pc = (-r) % m_tile, (-c) % k_tile
    if pr == 0 and pc == 0:
        return a.copy(), (r, c)
    return np.pad(a, ((0, pr), (0, pc))), (r, c)


def pack_gemv(codes, scales, mins, rows: int = 4) -> bytes:
    """q4nx parameters -> ``pack_gemv`` bytes. ``quant/q4nx.py:335-393``."""
    c = np.asarray(codes, dtype=np.uint8)
    m, k = c.shape
    slice_rows = rows * M_TILE
    if m % slice_rows:
        raise ValueError(f"M ({m}) must be a multiple of {slice_rows} (rows={rows} * M_TILE={M_TILE})")
    if k % K_TILE:
        raise ValueError(f"K ({k}) must be a multiple of K_TILE ({K_TILE})")
    kb, ng, ns = k // K_TILE, K_TILE // GROUP, m // slice_rows

    # Scale/min block: [slice][kb][row-tile][{scale,min}][group][row32].
    def sm_part(vals):
        u = f32_to_bf16(vals).reshape(ns, rows, M_TILE, kb, ng)
        return u.transpose(0, 3, 1, 4, 2)

    sm = np.stack([sm_part(scales), sm_part(mins)], axis=3).reshape(ns * kb * rows, -1)
    sm_bytes = np.ascontiguousarray(sm).view(np.uint8)

    # Code block: element order (half, group, col, row16); pair adjacent rows per byte.
    q = c.reshape(ns, rows, 2, 16, kb, ng, GROUP).transpose(0, 4, 1, 2, 5, 6, 3)
    q = q.reshape(ns * kb * rows, M_TILE * K_TILE)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    return np.concatenate([sm_bytes, packed], axis=1).tobytes()


def parse_gemv(buf, K: int, M: int, rows: int = 4):
    """Inverse of ``pack_gemv``: bytes -> ``(codes, scales, mins)``. ``quant/q4nx.py:396-438``."""
    b = np.frombuffer(buf, dtype=np.uint8) if isinstance(buf, (bytes, bytearray)) else np.asarray(buf, np.uint8).reshape(-1)
    kb, ng, ns = K // K_TILE, K_TILE // GROUP, M // (rows * M_TILE)
    blocks = b[: ns * kb * rows * BLOCK_BYTES].reshape(ns, kb, rows, BLOCK_BYTES)
    sm = bf16_to_f32(blocks[..., :SM_BYTES].copy().view("<u2")).reshape(ns, kb, rows, 2, ng, M_TILE)
    scales = sm[:, :, :, 0].transpose(0, 2, 4, 1, 3).reshape(M, K // GROUP)
    mins = sm[:, :, :, 1].transpose(0, 2, 4, 1, 3).reshape(M, K // GROUP)
    q = blocks[..., SM_BYTES:]
    flat = np.empty(q.shape[:-1] + (2 * q.shape[-1],), dtype=np.uint8)
    flat[..., 0::2] = q & 0x0F
    flat[..., 1::2] = q >> 4
    codes = flat.reshape(ns, kb, rows, 2, ng, GROUP, 16).transpose(0, 2, 3, 6, 1, 4, 5).reshape(M, K)
    return codes, scales.astype(np.float32), mins.astype(np.float32)


def decode_block(block) -> np.ndarray:
    """One 5,120-byte block -> its 32x256 float64 weights. ``kernels/gemv/reference.py:34-46``.

    Written directly from the block description (params ``[2][8][32]`` bf16, then
    nibble stream in ``(half, group, col, row16)`` order), independently of
    ``parse_gemv``'s transposes.
    """
    raw = bytes(block)
    params = bf16_to_f32(np.frombuffer(raw[:SM_BYTES], dtype="<u2")).astype(np.float64)
    scale = params[:256].reshape(8, 32)  # [group][row]
    mn = params[256:].reshape(8, 32)
    nib = np.frombuffer(raw[SM_BYTES:], dtype=np.uint8)
    out = np.empty((M_TILE, K_TILE), dtype=np.float64)
    for e in range(M_TILE * K_TILE):
        byte = nib[e >> 1]
        code = (byte >> 4) if (e & 1) else (byte & 0x0F)
        r16 = e % 16
        col = (e // 16) % 32
        grp = (e // 512) % 8
        half = e // 4096
        row = half * 16 + r16
        out[row, grp * 32 + col] = mn[grp, row] + scale[grp, row] * float(code)
    return out


def dequantize_packed(buf, K: int, M: int, rows: int = 4) -> np.ndarray:
    """Whole ``pack_gemv`` buffer -> float64 ``[M, K]`` via ``decode_block``.

    ``kernels/gemv/reference.py:49-67``: block index ``i`` -> ``(slice, kb, r)`` with
    ``i = (slice*k_blocks + kb)*rows + r``; rows start at ``(slice*rows + r)*32``.
    """
    raw = bytes(buf)
    kb = K // K_TILE
    out = np.empty((M, K), dtype=np.float64)
    for i in range((M // M_TILE) * kb):
        rest, r = divmod(i, rows)
        sl, kk = divmod(rest, kb)
        r0 = (sl * rows + r) * M_TILE
        out[r0 : r0 + M_TILE, kk * K_TILE : (kk + 1) * K_TILE] = decode_block(raw[i * BLOCK_BYTES : (i + 1) * BLOCK_BYTES])
    return out
