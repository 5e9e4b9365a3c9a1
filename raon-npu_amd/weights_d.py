"""weights-d: the reference's exported bundle directory, validated and loaded onto the GPU.

A ``weights-d`` directory (``export/export_d.py``) holds one ``.bin`` per bundle plus a
``manifest.json`` that names each bundle's format, shapes, size and SHA-256.  This module

* restates the canonical bundle and component map of the released model
  (``build_default_manifest_specs``, npu/backend.py:356-719), a table that has to match
  the exporter's entry for entry;
* checks a manifest against it with the rules of ``_load_manifest_specs``
  (npu/backend.py:729-929), kept here as a table of per-field checks: known bundle
  names, no duplicates, format, padded and original shapes, expert_count /
  expert_bytes of the expert bundles, canonical size_bytes, a 64-digit sha256, file
  paths that stay inside the directory, the file's size on disk, and the component
  list of each bundle;
* loads the MoE hot path's bundles into a ``GpuBackend``: ``moe_b1`` + ``moe_b2`` as a
  weights-d MoE layer, ``shared_gu`` as a dense bfp16 matrix and the shared down
  (``moe_b2`` expert 128, a view of the layer's tiles) served by ``linear``, and, when
  present, layer 0's ``dense_gu`` / ``dense_down`` and the ``lm_head``.  Expert bundles are streamed from disk in slices
  of experts and hashed on the way (``_verify_bundle_file``, npu/backend.py:316-340);
  a digest mismatch discards the layer before it is used.

The attention bundles (rda_in, f_b, mla_in, q_b, k_b, v_b, g, o_proj) are validated but
not loaded: attention is outside the MoE hot path this backend serves.
"""

from __future__ import annotations

import hashlib
import json
import math
import re
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Mapping, Sequence

import numpy as np

RDA_LAYERS = frozenset({0, 1, 2, 4, 5, 6, 8, 9, 10, 12, 13, 14, 16, 17, 18, 20, 21, 22})
MLA_LAYERS = frozenset({3, 7, 11, 15, 19, 23, 24})
NUM_LAYERS = 25
HIDDEN_SIZE = 2560
MOE_INTER = 1088
NUM_ROUTED_EXPERTS = 128
NUM_TOTAL_EXPERTS = 129

# quant/q4nx.py:23-28 and quant/bfp16.py:35-47
Q4NX_M_TILE, Q4NX_K_TILE, Q4NX_BLOCK_BYTES = 32, 256, 5120
BFP16_BLOCK, BFP16_BLOCK_BYTES = 8, 9


@dataclass
class Component:
    """A named weight served by rows of a bundle (``ComponentMeta``, npu/backend.py:88-99)."""

    hf_name: str
    bundle: str
    row_start: int
    row_end: int
    orig_k: int
    padded_k: int
    orig_m: int
    padded_m: int
    fmt: str
    extra: dict[str, Any] = field(default_factory=dict)


@dataclass
class Bundle:
    """One ``.bin`` of the directory (``BundleMeta``, npu/backend.py:102-116)."""

    name: str
    rel_file: str
    fmt: str
    orig_shape: list[int]
    padded_shape: list[int]
    k: int
    m: int
    expert_bytes: int = 0
    expert_count: int = 0
    size_bytes: int = 0
    sha256: str = ""


def canonical_specs() -> tuple[dict[str, Component], dict[str, Bundle]]:
    """Components and bundles of the released model (npu/backend.py:356-719)."""
    comps: dict[str, Component] = {}
    bundles: dict[str, Bundle] = {}

    def bundle(name: str, fmt: str, orig, padded, **kw) -> str:
        bundles[name] = Bundle(name, f"{name}.bin", fmt, list(orig), list(padded), k=padded[-1], m=padded[-2], **kw)
        return name

    def comp(hf: str, b: str, r0: int, r1: int, orig_k: int, padded_k: int, orig_m: int, padded_m: int,
             fmt: str = "bfp16_gemv", **extra) -> None:
        comps[hf] = Component(hf, b, r0, r1, orig_k, padded_k, orig_m, padded_m, fmt, dict(extra))

    # layer 0 dense MLP
    b = bundle("L00/dense_gu", "q4nx_gemv", [24064, 2560], [24064, 2560])
    comp("model.layers.0.mlp.gate_proj.weight", b, 0, 12032, 2560, 2560, 12032, 24064, "q4nx_gemv")
    comp("model.layers.0.mlp.up_proj.weight", b, 12032, 24064, 2560, 2560, 12032, 24064, "q4nx_gemv")
    b = bundle("L00/dense_down", "bfp16_gemv", [2560, 12032], [2560, 12032])
    comp("model.layers.0.mlp.down_proj.weight", b, 0, 2560, 12032, 12032, 2560, 2560)

    for layer in range(NUM_LAYERS):
        p, d = f"model.layers.{layer}", f"L{layer:02d}"
        if layer in RDA_LAYERS:
            b = bundle(f"{d}/rda_in", "bfp16_gemv", [20688, 2560], [20736, 2560])
            rows = [("q_proj", 0, 5120), ("k_proj", 5120, 10240), ("v_proj", 10240, 15360), ("g_proj", 15360, 20480),
                    ("f_a_proj", 20480, 20608), ("b_proj", 20608, 20648), ("rda_w_proj", 20648, 20688)]
            for sub, r0, r1 in rows:
                comp(f"{p}.self_attn.{sub}.weight", b, r0, r1, 2560, 2560, r1 - r0, 20736)
            b = bundle(f"{d}/f_b", "bfp16_gemv", [5120, 128], [5120, 256])
            comp(f"{p}.self_attn.f_b_proj.weight", b, 0, 5120, 128, 256, 5120, 5120)
        else:
            b = bundle(f"{d}/mla_in", "bfp16_gemv", [1152, 2560], [1152, 2560])
            comp(f"{p}.self_attn.q_a_proj.weight", b, 0, 576, 2560, 2560, 576, 1152)
            comp(f"{p}.self_attn.kv_a_proj_with_mqa.weight", b, 576, 1152, 2560, 2560, 576, 1152)
            b = bundle(f"{d}/q_b", "bfp16_gemv", [7680, 576], [7680, 768])
            comp(f"{p}.self_attn.q_b_proj.weight", b, 0, 7680, 576, 768, 7680, 7680)
            kb = bundle(f"{d}/k_b", "bfp16_gemv", [5120, 512], [5120, 512])
            vb = bundle(f"{d}/v_b", "bfp16_gemv", [5120, 512], [5120, 512])
            comp(f"{p}.self_attn.kv_b_proj.weight", f"{d}/kv_b_combined", 0, 10240, 512, 512, 10240, 10240,
                 "mla_kv_b", kb_bundle=kb, vb_bundle=vb)
            b = bundle(f"{d}/g", "bfp16_gemv", [5120, 2560], [5120, 2560])
            comp(f"{p}.self_attn.g_proj.weight", b, 0, 5120, 2560, 2560, 5120, 5120)
        b = bundle(f"{d}/o_proj", "bfp16_gemv", [2560, 5120], [2560, 5120])
        comp(f"{p}.self_attn.o_proj.weight", b, 0, 2560, 5120, 5120, 2560, 2560)
        if layer >= 1:
            gu = 2 * MOE_INTER
            bundle(f"{d}/moe_b1", "q4nx_gemv_bundle", [NUM_ROUTED_EXPERTS, gu, HIDDEN_SIZE],
                   [NUM_ROUTED_EXPERTS, gu, HIDDEN_SIZE], expert_bytes=3481600, expert_count=NUM_ROUTED_EXPERTS)
            b2 = bundle(f"{d}/moe_b2", "bfp16_gemv_bundle", [NUM_TOTAL_EXPERTS, HIDDEN_SIZE, MOE_INTER],
                        [NUM_TOTAL_EXPERTS, HIDDEN_SIZE, 1280], expert_bytes=3686400, expert_count=NUM_TOTAL_EXPERTS)
            b = bundle(f"{d}/shared_gu", "bfp16_gemv", [gu, HIDDEN_SIZE], [gu, HIDDEN_SIZE])
            comp(f"{p}.moe.shared_experts.gate_proj.weight", b, 0, MOE_INTER, 2560, 2560, MOE_INTER, gu)
            comp(f"{p}.moe.shared_experts.up_proj.weight", b, MOE_INTER, gu, 2560, 2560, MOE_INTER, gu)
            comp(f"{p}.moe.shared_experts.down_proj.weight", b2, 0, 2560, MOE_INTER, 1280, 2560, 2560,
                 "shared_down", expert_id=NUM_ROUTED_EXPERTS)

    b = bundle("lm_head", "bfp16_gemv", [259840, 2560], [260096, 2560])
    comp("lm_head.weight", b, 0, 259840, 2560, 2560, 259840, 260096)
    return comps, bundles


# ------------------------------------------------------------- bundle sizes --
# A GEMV format stores a matrix in whole blocks of (rows, cols, bytes): q4nx blocks are
# 32 x 256 weights in 5,120 B (quant/q4nx.py:23-28), bfp16ebs8 blocks are 8 weights of a
# row in 9 B (quant/bfp16.py:35-47).  An expert bundle is expert_count such matrices.
_BLOCK_OF_FAMILY = {"q4nx": (Q4NX_M_TILE, Q4NX_K_TILE, Q4NX_BLOCK_BYTES), "bfp16": (1, BFP16_BLOCK, BFP16_BLOCK_BYTES)}
_FAMILY_OF_FORMAT = {"q4nx_gemv": "q4nx", "q4nx_gemv_bundle": "q4nx", "bfp16_gemv": "bfp16",
                     "bfp16_gemv_bundle": "bfp16"}


def canonical_size(meta: Bundle) -> tuple[int, int]:
    """``(bundle bytes, bytes of one matrix)`` of a canonical bundle, from its padded shape
    and format (the sizes npu/backend.py:729-752 derives)."""
    family = _FAMILY_OF_FORMAT.get(meta.fmt)
    if family is None:
        raise ValueError(f"{meta.name}: no block size is known for format {meta.fmt!r}")
    if len(meta.padded_shape) < 2:
        raise ValueError(f"{meta.name}: padded shape {meta.padded_shape} has no [rows, cols] matrix")
    rows, cols = meta.padded_shape[-2:]
    br, bc, nbytes = _BLOCK_OF_FAMILY[family]
    if rows % br or cols % bc:
        raise ValueError(f"{meta.name}: [{rows}, {cols}] is not a whole number of {br}x{bc} {family} blocks")
    one = (rows // br) * (cols // bc) * nbytes
    return one * max(meta.expert_count, 1), one


def component_names(comps: Mapping[str, Component], meta: Bundle) -> tuple[set[str], set[str]]:
    """``(required, allowed)`` component names of a bundle's manifest entry: the canonical
    components served from it, plus the names the exporter writes for padding rows and
    for the routed experts' rows (the contract of npu/backend.py:755-784)."""
    required = {c.hf_name for c in comps.values() if c.bundle == meta.name}
    extra = {"padding"}
    m = re.fullmatch(r"L(\d+)/(moe_b1|moe_b2|k_b|v_b)", meta.name)
    if m:
        layer, leaf = int(m.group(1)), m.group(2)
        pfx = f"model.layers.{layer}"
        if leaf == "moe_b1" and meta.expert_count:
            extra.add(f"{pfx}.moe.experts.0..{meta.expert_count - 1}.(gate|up)_proj.weight")
        elif leaf == "moe_b2" and meta.expert_count:
            # the last expert of moe_b2 is the shared one: routed experts 0..count-2
            extra.add(f"{pfx}.moe.experts.0..{meta.expert_count - 2}.down_proj.weight")
        elif leaf in ("k_b", "v_b"):
            extra.add(f"{pfx}.self_attn.kv_b_proj.weight ({'key' if leaf == 'k_b' else 'val'}_part)")
    return required, required | extra


def bundle_path(weights_dir: Path, rel_file: str, name: str) -> Path:
    """Where a manifest's relative file name points, refusing any path that is absolute,
    climbs with ``..`` or resolves (symlinks included) outside ``weights_dir`` -- the
    rule of npu/backend.py:278-291."""
    rel = Path(rel_file)
    if rel.is_absolute() or any(part == ".." for part in rel.parts):
        raise ValueError(f"Unsafe file path for {name}: {rel_file!r} (absolute, or climbs with '..')")
    root = Path(weights_dir).resolve()
    target = (root / rel).resolve(strict=False)
    if target != root and root not in target.parents:
        raise ValueError(f"Unsafe file path for {name}: {rel_file!r} resolves outside {root}")
    return target


def loads_strict(data: bytes | str) -> Any:
    """Parse JSON, refusing NaN, +-Infinity and numbers that overflow to them, and turning
    pathological nesting into a ValueError (the decoding rules of host/strict_json.py)."""
    text = data.decode("utf-8") if isinstance(data, (bytes, bytearray)) else data

    def no_constant(tok: str):
        raise ValueError(f"JSON number {tok} is non-finite")

    def finite(tok: str) -> float:
        v = float(tok)
        if math.isinf(v) or math.isnan(v):
            raise ValueError(f"JSON number {tok} is non-finite")
        return v

    try:
        return json.loads(text, parse_constant=no_constant, parse_float=finite)
    except RecursionError as exc:
        raise ValueError("JSON nesting too deep") from exc


# ------------------------------------------------------- manifest validation --
def _is_int(v) -> bool:
    return isinstance(v, int) and not isinstance(v, bool)


# Each check returns None or the whole message.  Messages that the reference's own tests
# match keep its words: "Manifest {key} mismatch for" (npu/test_backend_small.py:475,485),
# "canonical size_bytes mismatch" (:588) and the field name of expert_count/expert_bytes
# (:620-625).
def _expect_equal(key: str):
    def check(value, meta: Bundle, want):
        return None if value == want else f"Manifest {key} mismatch for {meta.name}: {value!r} != {want!r}"
    return check


def _check_shape(key: str):
    def check(value, meta: Bundle, want):
        ok = isinstance(value, list) and list(value) == list(want)
        return None if ok else f"Manifest {key} mismatch for {meta.name}: {value!r} != {list(want)!r}"
    return check


def _check_count(key: str):
    def check(value, meta: Bundle, want):
        ok = _is_int(value) and value == want
        return None if ok else f"Manifest {key} mismatch for {meta.name}: {value!r} != {want}"
    return check


def _check_file(value, meta: Bundle, want):
    return None if isinstance(value, str) and value else f"Manifest file missing for {meta.name}"


def _check_size(value, meta: Bundle, want):
    if not _is_int(value) or value < 0:
        return f"Manifest size_bytes for {meta.name} is not a byte count: {value!r}"
    return None if value == want else f"Manifest entry {meta.name}: canonical size_bytes mismatch: {value} != {want}"


def _check_sha(value, meta: Bundle, want):
    ok = isinstance(value, str) and re.fullmatch(r"[0-9a-fA-F]{64}", value) is not None
    return None if ok else f"Manifest sha256 for {meta.name} is not 64 hex digits: {value!r}"


# (manifest key, check, the canonical value it is compared with, applies to the bundle?)
# in the order they are checked; the first failing rule names the entry and the field.
_ENTRY_RULES = (
    ("format", _expect_equal("format"), lambda m: m.fmt, lambda m: True),
    ("padded_shape", _check_shape("padded_shape"), lambda m: m.padded_shape, lambda m: True),
    ("original_shape", _check_shape("original_shape"), lambda m: m.orig_shape, lambda m: True),
    ("expert_count", _check_count("expert_count"), lambda m: m.expert_count, lambda m: m.expert_count > 0),
    ("expert_bytes", _check_count("expert_bytes"), lambda m: m.expert_bytes, lambda m: m.expert_count > 0),
    ("file", _check_file, lambda m: None, lambda m: True),
    ("size_bytes", _check_size, lambda m: canonical_size(m)[0], lambda m: True),
    ("sha256", _check_sha, lambda m: None, lambda m: True),
)


def _check_components(item: dict, meta: Bundle, comps: Mapping[str, Component], require_complete: bool) -> None:
    listed = item.get("components")
    if not isinstance(listed, list):
        raise ValueError(f"Manifest entry {meta.name}: components must be a list, got {listed!r}")
    required, allowed = component_names(comps, meta)
    named = set()
    for c in listed:
        if not isinstance(c, dict) or not isinstance(c.get("name"), str):
            raise ValueError(f"Manifest entry {meta.name}: component {c!r} has no name")
        cname = c["name"]
        if cname not in allowed:
            raise ValueError(f"Unknown component for {meta.name}: {cname!r}")
        named.add(cname)
        canon = comps.get(cname)
        if canon is None:
            continue
        rows = (c.get("row_start"), c.get("row_end"))
        if ("row_start" in c or "row_end" in c) and rows != (canon.row_start, canon.row_end):
            raise ValueError(f"Manifest entry {meta.name}: component {cname} rows {rows} differ from "
                             f"({canon.row_start}, {canon.row_end})")
        if "expert_id" in c and "expert_id" in canon.extra and c["expert_id"] != canon.extra["expert_id"]:
            raise ValueError(f"Manifest entry {meta.name}: component {cname} expert_id {c['expert_id']!r} differs "
                             f"from {canon.extra['expert_id']}")
    missing = required - named
    if require_complete and missing:
        raise ValueError(f"Manifest entry {meta.name}: missing canonical components " + ", ".join(sorted(missing)))


def load_manifest(path: str | Path, comps: Mapping[str, Component], bundles: Mapping[str, Bundle], *,
                  weights_dir: str | Path | None = None, require_complete: bool = True) -> None:
    """Check ``manifest.json`` against the canonical bundle map and record each bundle's
    file, size and digest in ``bundles``.

    The rules are those of npu/backend.py:787-929: the payload is a list of bundle
    entries (or ``{"bundles": [...]}``); ``host_safetensors`` entries are skipped; every
    other entry names a canonical bundle exactly once and carries its format, padded and
    original shapes, the expert count and size of an expert bundle, a file that stays
    inside the directory, the canonical size in bytes, a 64-digit sha256, and the
    bundle's component list; with ``weights_dir`` the file must exist with that size;
    with ``require_complete`` every canonical bundle and component must be listed.
    Violations raise ``ValueError`` (``FileNotFoundError`` for a missing file)."""
    path = Path(path)
    payload = loads_strict(path.read_bytes())
    if isinstance(payload, list):
        entries = payload
    elif isinstance(payload, dict) and isinstance(payload.get("bundles"), list):
        entries = payload["bundles"]
    elif isinstance(payload, dict):
        raise ValueError(f"{path}: manifest object has no 'bundles' list")
    else:
        raise ValueError(f"{path}: manifest top-level value must be a list or an object")

    listed: set[str] = set()
    for item in entries:
        if not isinstance(item, dict):
            raise ValueError(f"{path}: manifest bundle entry {item!r} is not an object")
        if item.get("format") == "host_safetensors":
            continue
        name = item.get("bundle")
        meta = bundles.get(name) if isinstance(name, str) else None
        if meta is None:
            raise ValueError(f"Unknown NPU bundle in manifest: {name!r} ({path})")
        if name in listed:
            raise ValueError(f"Duplicate NPU bundle in manifest: {name} ({path})")
        listed.add(name)
        if meta.expert_count and canonical_size(meta)[1] != meta.expert_bytes:
            raise ValueError(f"canonical map: {name} expert_bytes {meta.expert_bytes} != one matrix "
                             f"{canonical_size(meta)[1]}")
        for key, check, want, applies in _ENTRY_RULES:
            if applies(meta):
                msg = check(item.get(key), meta, want(meta))
                if msg:
                    raise ValueError(msg)
        if weights_dir is not None:
            target = bundle_path(Path(weights_dir), item["file"], name)
            try:
                on_disk = target.stat().st_size
            except FileNotFoundError as exc:
                raise FileNotFoundError(f"Missing D bundle binary: {target}") from exc
            if on_disk != item["size_bytes"]:
                raise ValueError(f"Manifest entry {name}: file has {on_disk} bytes, size_bytes says {item['size_bytes']}")
        meta.rel_file, meta.size_bytes, meta.sha256 = item["file"], item["size_bytes"], item["sha256"].lower()
        _check_components(item, meta, comps, require_complete)

    if require_complete:
        absent = set(bundles) - listed
        if absent:
            raise ValueError(f"{path}: manifest is missing NPU bundles " + ", ".join(sorted(absent)))


class _Reader:
    """Reads one bundle file in slices, hashing as it goes when a digest is expected."""

    def __init__(self, weights_dir: Path, meta: Bundle):
        self.meta = meta
        self.path = bundle_path(weights_dir, meta.rel_file, meta.name)
        try:
            st = self.path.stat()
        except FileNotFoundError as exc:
            raise FileNotFoundError(f"Missing D bundle binary: {self.path}") from exc
        want = meta.size_bytes or canonical_size(meta)[0]
        if st.st_size != want:
            raise ValueError(f"Manifest size_bytes mismatch for {meta.name}: file has {st.st_size}, manifest has {want}")
        self.hasher = hashlib.sha256() if meta.sha256 else None
        self._f = self.path.open("rb")

    def read(self, n: int) -> bytes:
        data = self._f.read(n)
        if len(data) != n:
            raise ValueError(f"Short read in {self.path}: got {len(data)} bytes, expected {n}")
        if self.hasher is not None:
            self.hasher.update(data)
        return data

    def finish(self) -> None:
        """Check the digest of everything read (the whole file) against the manifest."""
        rest = self._f.read()
        self._f.close()
        if rest:
            raise ValueError(f"{self.path} is longer than the {self.meta.name} bundle")
        if self.hasher is not None and self.hasher.hexdigest() != self.meta.sha256:
            raise ValueError(f"Manifest sha256 mismatch for {self.meta.name}: {self.hasher.hexdigest()} != {self.meta.sha256}")

    def close(self) -> None:
        if not self._f.closed:
            self._f.close()


def _read_whole(weights_dir: Path, meta: Bundle) -> bytes:
    r = _Reader(weights_dir, meta)
    try:
        data = r.read(r.meta.size_bytes or canonical_size(meta)[0])
        r.finish()
    finally:
        r.close()
    return data


def load_weights_d(backend, weights_dir: str | Path, manifest_path: str | Path | None = None, *,
                   layers: Sequence[int] | None = None, top_k: int = 6, require_complete: bool = True,
                   load_dense: bool = True, load_lm_head: bool = True, experts_per_read: int = 16,
                   routers: Mapping[int, tuple[np.ndarray, np.ndarray | None]] | None = None,
                   renormalize: bool = True, routed_scaling_factor: float = 1.0) -> dict[str, list]:
    """Load a weights-d directory's MoE-path bundles into ``backend`` (a ``GpuBackend``).

    ``layers`` selects the MoE layers (default: every layer 1..24 whose bundles exist);
    ``routers`` optionally maps a layer to its ``(gate.weight bf16 [128, 2560],
    e_score_correction_bias f32 [128] or None)`` for the device router (sigmoid scores,
    as RaonModel._route_token, host/raon.py:1224-1247).  Without ``manifest.json`` the
    canonical file names are used and nothing is hashed, as ``DWeights`` does.  Returns
    the names of the loaded and of the validated-but-skipped bundles.
    """
    from .geometry import MoeGeometry

    wdir = Path(weights_dir)
    mpath = Path(manifest_path) if manifest_path else wdir / "manifest.json"
    comps, bundles = canonical_specs()
    if mpath.is_file():
        load_manifest(mpath, comps, bundles, weights_dir=wdir, require_complete=require_complete)
    present = {n for n, m in bundles.items() if bundle_path(wdir, m.rel_file, n).is_file()}
    if layers is None:
        layers = [l for l in range(1, NUM_LAYERS) if f"L{l:02d}/moe_b1" in present]
    loaded: list[str] = []

    def register_dense(name: str, fmt: str, data: bytes | None = None) -> None:
        meta = bundles[name]
        backend.register_bundle(name, data if data is not None else _read_whole(wdir, meta), meta.m, meta.k, fmt=fmt)
        for c in comps.values():
            if c.bundle == name:
                backend.register_component(c.hf_name, name, c.row_start, c.row_end, orig_k=c.orig_k)
        loaded.append(name)

    geom = MoeGeometry(hidden=HIDDEN_SIZE, inter=MOE_INTER, n_routed=NUM_ROUTED_EXPERTS, n_shared=1, top_k=top_k)
    for layer in layers:
        d = f"L{int(layer):02d}"
        if not 1 <= int(layer) < NUM_LAYERS:
            raise ValueError(f"layer {layer} is not a MoE layer (1..{NUM_LAYERS - 1})")
        for leaf in ("moe_b1", "moe_b2", "shared_gu"):
            if f"{d}/{leaf}" not in present:
                raise FileNotFoundError(f"Missing D bundle binary: {bundle_path(wdir, bundles[f'{d}/{leaf}'].rel_file, leaf)}")
        lyr = backend.ctx.create_layer_d(int(layer), geom)
        try:
            for bundle_id, leaf in ((1, "moe_b1"), (2, "moe_b2")):
                meta = bundles[f"{d}/{leaf}"]
                reader = _Reader(wdir, meta)
                try:
                    for e0 in range(0, meta.expert_count, experts_per_read):
                        n = min(experts_per_read, meta.expert_count - e0)
                        chunk = reader.read(n * meta.expert_bytes)
                        lyr.upload_d(bundle_id, e0, chunk)
                    reader.finish()
                finally:
                    reader.close()
        except BaseException:
            lyr.free()
            raise
        if routers and int(layer) in routers:
            w, bias = routers[int(layer)]
            lyr.set_router(w, bias, "sigmoid", renormalize, routed_scaling_factor)
        backend._layers[int(layer)] = lyr
        loaded += [f"{d}/moe_b1", f"{d}/moe_b2"]
        register_dense(f"{d}/shared_gu", "bfp16_gemv")
        # The shared expert's down projection (component fmt "shared_down") is moe_b2's
        # expert 128, served by linear in place as a bfp16 [2560, 1280] matrix whose input
        # is zero-padded from 1088 columns.
        sd = comps[f"model.layers.{int(layer)}.moe.shared_experts.down_proj.weight"]
        backend.register_view(f"{d}/shared_down", lyr.expert_matrix(sd.extra["expert_id"], "down"))
        backend.register_component(sd.hf_name, f"{d}/shared_down", sd.row_start, sd.row_end, orig_k=sd.orig_k)

    if load_dense and {"L00/dense_gu", "L00/dense_down"} <= present:
        register_dense("L00/dense_gu", "q4nx_gemv")
        register_dense("L00/dense_down", "bfp16_gemv")
    if load_lm_head and "lm_head" in present:
        register_dense("lm_head", "bfp16_gemv")
    skipped = sorted(present - set(loaded))
    return {"loaded": loaded, "skipped": skipped}
