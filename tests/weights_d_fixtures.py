"""Synthetic weights-d directories and bundles for the loader and weights-d layer tests.

A manifest entry carries exactly the fields ``_load_manifest_specs`` reads
(npu/backend.py:787-929).  Bundle files are either sparse (``truncate``: only the size
matters to the validator) or filled with valid random GEMV bytes: q4nx blocks of
``quant/q4nx.py:335-393`` (per 5,120-byte block: bf16 scales [8][32], bf16 mins [8][32],
then 4,096 code bytes) and bfp16 groups of ``quant/bfp16.py:216-329`` (per 144-byte
group: 16 exponent bytes, then 128 mantissa bytes).
"""

from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np

from oracle.bf16 import f32_to_bf16


def random_q4nx_bundle(nbytes: int, rng: np.random.Generator, scale=(5e-4, 2e-3)) -> np.ndarray:
    """Arbitrary q4nx GEMV bytes with finite group parameters: scale in ``scale``, min =
    -7.5 * scale * U(0.8, 1.2) so that weights straddle zero."""
    buf = rng.integers(0, 256, nbytes, dtype=np.uint8)
    blk = buf.reshape(-1, 5120)
    n = blk.shape[0]
    s = rng.uniform(scale[0], scale[1], (n, 256)).astype(np.float32)
    m = (-7.5 * s * rng.uniform(0.8, 1.2, (n, 256))).astype(np.float32)
    blk[:, :512] = f32_to_bf16(s).view(np.uint8).reshape(n, 512)
    blk[:, 512:1024] = f32_to_bf16(m).view(np.uint8).reshape(n, 512)
    return buf


def random_bfp16_bundle(nbytes: int, rng: np.random.Generator, e_lo: int = 116, e_hi: int = 120) -> np.ndarray:
    """Arbitrary bfp16 GEMV bytes: uniform int8 mantissas, exponents in [e_lo, e_hi]."""
    buf = rng.integers(0, 256, nbytes, dtype=np.uint8)
    grp = buf.reshape(-1, 144)
    grp[:, :16] = rng.integers(e_lo, e_hi + 1, (grp.shape[0], 16), dtype=np.uint8)
    return buf


def manifest_entry(meta, comps, rel_file: str, sha256: str, size: int | None = None) -> dict:
    """The manifest entry the exporter writes for a canonical bundle."""
    from raon_npu_amd.weights_d import canonical_size

    entry = {
        "bundle": meta.name,
        "file": rel_file,
        "format": meta.fmt,
        "original_shape": list(meta.orig_shape),
        "padded_shape": list(meta.padded_shape),
        "size_bytes": canonical_size(meta)[0] if size is None else size,
        "sha256": sha256,
        "components": [
            {"name": c.hf_name, "row_start": c.row_start, "row_end": c.row_end,
             **({"expert_id": c.extra["expert_id"]} if "expert_id" in c.extra else {})}
            for c in comps.values() if c.bundle == meta.name
        ],
    }
    if meta.expert_count:
        entry["expert_count"] = meta.expert_count
        entry["expert_bytes"] = meta.expert_bytes
    return entry


def sparse_weights_dir(root: Path, names=None) -> tuple[dict, dict, list]:
    """Every canonical bundle (or ``names``) as a sparse file of its canonical size, plus a
    manifest whose sha256 fields are well-formed placeholders.  Returns (comps, bundles,
    entries)."""
    from raon_npu_amd.weights_d import canonical_size, canonical_specs

    comps, bundles = canonical_specs()
    entries = []
    for name, meta in bundles.items():
        if names is not None and name not in names:
            continue
        path = root / meta.rel_file
        path.parent.mkdir(parents=True, exist_ok=True)
        with path.open("wb") as f:
            f.truncate(canonical_size(meta)[0])
        entries.append(manifest_entry(meta, comps, meta.rel_file, "ab" * 32))
    return comps, bundles, entries


def write_manifest(root: Path, entries) -> Path:
    path = root / "manifest.json"
    path.write_text(json.dumps({"bundles": entries}))
    return path


def write_bundle(root: Path, meta, data: np.ndarray) -> str:
    """Write a bundle file and return its sha256."""
    path = root / meta.rel_file
    path.parent.mkdir(parents=True, exist_ok=True)
    buf = np.ascontiguousarray(data, dtype=np.uint8)
    path.write_bytes(buf.tobytes())
    return hashlib.sha256(buf.tobytes()).hexdigest()
