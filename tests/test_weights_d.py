"""weights-d manifest validation and canonical map (CPU; npu/backend.py:278-340, 356-929).

The canonical sizes are pinned to the constants the reference writes by hand
(``expert_bytes`` 3,481,600 and 3,686,400, npu/backend.py:635,650) and to the q4nx /
bfp16 bit rates (5 and 9 bits per weight); every validation rule is exercised by a
manifest that breaks exactly that rule, on sparse bundle files of the canonical sizes.
"""

from __future__ import annotations

import copy
import json

import numpy as np
import pytest

from raon_npu_amd import weights_d as W

from weights_d_fixtures import sparse_weights_dir, write_bundle, write_manifest


def test_canonical_map_shape():
    comps, bundles = W.canonical_specs()
    # 2 dense + 18 RDA layers x 3 + 7 MLA layers x 6 + 24 MoE layers x 3 + lm_head
    assert len(bundles) == 2 + 18 * 3 + 7 * 6 + 24 * 3 + 1
    assert W.RDA_LAYERS | W.MLA_LAYERS == set(range(25)) and not (W.RDA_LAYERS & W.MLA_LAYERS)
    b1, b2 = bundles["L07/moe_b1"], bundles["L07/moe_b2"]
    assert W.canonical_size(b1) == (128 * 3481600, 3481600) and b1.expert_bytes == 3481600
    assert W.canonical_size(b2) == (129 * 3686400, 3686400) and b2.expert_bytes == 3686400
    # 5 and 9 bits per weight
    assert 3481600 * 8 == 2176 * 2560 * 5 and 3686400 * 8 == 2560 * 1280 * 9
    assert W.canonical_size(bundles["lm_head"])[0] == 260096 * 2560 * 9 // 8
    sd = comps["model.layers.7.moe.shared_experts.down_proj.weight"]
    assert (sd.bundle, sd.fmt, sd.extra["expert_id"], sd.orig_k, sd.padded_k) == ("L07/moe_b2", "shared_down", 128, 1088, 1280)
    kv = comps["model.layers.3.self_attn.kv_b_proj.weight"]
    assert kv.bundle == "L03/kv_b_combined" and kv.extra == {"kb_bundle": "L03/k_b", "vb_bundle": "L03/v_b"}
    # every component's rows fit its bundle and each bundle's rows are covered without overlap
    for c in comps.values():
        if c.bundle in bundles:
            assert 0 <= c.row_start < c.row_end <= bundles[c.bundle].m
    with pytest.raises(ValueError):
        W.canonical_size(W.Bundle("x", "x.bin", "q4nx_gemv", [100, 256], [100, 256], 256, 100))
    with pytest.raises(ValueError):
        W.canonical_size(W.Bundle("x", "x.bin", "fp8", [128, 256], [128, 256], 256, 128))


def test_component_names():
    comps, bundles = W.canonical_specs()
    req, allowed = W.component_names(comps, bundles["L05/moe_b1"])
    assert req == set() and "model.layers.5.moe.experts.0..127.(gate|up)_proj.weight" in allowed
    req, allowed = W.component_names(comps, bundles["L05/moe_b2"])
    assert req == {"model.layers.5.moe.shared_experts.down_proj.weight"}
    assert "model.layers.5.moe.experts.0..127.down_proj.weight" in allowed and "padding" in allowed
    req, allowed = W.component_names(comps, bundles["L03/k_b"])
    assert req == set() and "model.layers.3.self_attn.kv_b_proj.weight (key_part)" in allowed


@pytest.fixture(scope="module")
def full_dir(tmp_path_factory):
    root = tmp_path_factory.mktemp("weights_d")
    comps, bundles, entries = sparse_weights_dir(root)
    return root, entries


def _validate(root, entries, **kw):
    comps, bundles = W.canonical_specs()
    path = write_manifest(root, entries)
    W.load_manifest(path, comps, bundles, weights_dir=root, **kw)
    return bundles


def test_full_manifest_validates(full_dir):
    root, entries = full_dir
    bundles = _validate(root, entries)
    assert bundles["L01/moe_b1"].sha256 == "ab" * 32 and bundles["L01/moe_b1"].size_bytes == 128 * 3481600
    # host_safetensors entries are skipped; a dict or a bare list both parse
    _validate(root, entries + [{"format": "host_safetensors", "file": "host.safetensors"}])
    comps, b2 = W.canonical_specs()
    (root / "manifest.json").write_text(json.dumps(entries))
    W.load_manifest(root / "manifest.json", comps, b2, weights_dir=root)


def _broken(entries, name, **changes):
    out = copy.deepcopy(entries)
    for e in out:
        if e.get("bundle") == name:
            for k, v in changes.items():
                if v is _DROP:
                    e.pop(k, None)
                else:
                    e[k] = v
    return out


_DROP = object()


# The patterns are the phrases the reference's manifest tests match
# (npu/test_backend_small.py:475,485,588,608,613,620-625,635,671,676).
@pytest.mark.parametrize("name,changes,pattern", [
    ("L01/moe_b1", {"format": "q4nx_gemv"}, "Manifest format mismatch"),
    ("L01/moe_b2", {"padded_shape": [129, 2560, 1088]}, "Manifest padded_shape mismatch"),
    ("L01/moe_b2", {"original_shape": _DROP}, "Manifest original_shape mismatch"),
    ("L02/moe_b1", {"expert_count": 129}, "expert_count"),
    ("L02/moe_b1", {"expert_bytes": 3481601}, "expert_bytes"),
    ("L02/shared_gu", {"size_bytes": True}, "is not a byte count"),
    ("L02/shared_gu", {"size_bytes": 6266881}, "canonical size_bytes mismatch"),
    ("lm_head", {"sha256": "xyz"}, "is not 64 hex digits"),
    ("lm_head", {"sha256": "ab" * 31}, "is not 64 hex digits"),
    ("L00/f_b", {"file": "../f_b.bin"}, "Unsafe file path"),
    ("L00/f_b", {"file": "/etc/passwd"}, "Unsafe file path"),
    ("L00/f_b", {"file": ""}, "Manifest file missing"),
    ("L00/f_b", {"components": "none"}, "components must be a list"),
    ("L00/f_b", {"components": [{"name": "model.layers.0.mlp.gate_proj.weight"}]}, "Unknown component"),
    ("L01/shared_gu", {"components": [{"name": "model.layers.1.moe.shared_experts.gate_proj.weight", "row_start": 0,
                                       "row_end": 1000}]}, "rows .* differ"),
    ("L01/moe_b2", {"components": [{"name": "model.layers.1.moe.shared_experts.down_proj.weight", "expert_id": 127}]},
     "expert_id .* differs"),
    ("L01/moe_b2", {"components": []}, "missing canonical components"),
    ("L04/o_proj", {"bundle": "L04/o_proj_v2"}, "Unknown NPU bundle"),
])
def test_manifest_rules(full_dir, name, changes, pattern):
    root, entries = full_dir
    with pytest.raises(ValueError, match=pattern):
        _validate(root, _broken(entries, name, **changes))


def test_manifest_rules_structure(full_dir, tmp_path):
    root, entries = full_dir
    with pytest.raises(ValueError, match="Duplicate NPU bundle"):
        _validate(root, entries + [entries[3]])
    with pytest.raises(ValueError, match="missing NPU bundles"):
        _validate(root, entries[:-1])
    _validate(root, entries[:-1], require_complete=False)
    with pytest.raises(ValueError, match="is not an object"):
        _validate(root, entries + [7])
    comps, bundles = W.canonical_specs()
    for text, pattern in (('{"bundles": [], "x": NaN}', "non-finite"), ('{"b": 1e999}', "non-finite"),
                          ('{"nobundles": []}', "no 'bundles' list"), ('"x"', "top-level")):
        (tmp_path / "m.json").write_text(text)
        with pytest.raises(ValueError, match=pattern):
            W.load_manifest(tmp_path / "m.json", comps, bundles)
    # padding and the expert pattern names are allowed component names
    ok = _broken(entries, "L01/moe_b1", components=[{"name": "padding"},
                                                    {"name": "model.layers.1.moe.experts.0..127.(gate|up)_proj.weight"}])
    _validate(root, ok)


def test_manifest_file_checks(full_dir, tmp_path):
    root, entries = full_dir
    (root / "L00" / "f_b.bin").rename(root / "L00" / "f_b.moved")
    try:
        with pytest.raises(FileNotFoundError, match="Missing D bundle binary"):
            _validate(root, entries)
        with (root / "L00" / "f_b.bin").open("wb") as f:
            f.truncate(1474560 - 1)
        with pytest.raises(ValueError, match="file has 1474559"):
            _validate(root, entries)
    finally:
        (root / "L00" / "f_b.moved").replace(root / "L00" / "f_b.bin")
    # a symlink out of the directory is caught after resolution
    (root / "escape").symlink_to(tmp_path)
    try:
        with pytest.raises(ValueError, match="Unsafe file path"):
            _validate(root, _broken(entries, "L00/f_b", file="escape/f_b.bin"))
    finally:
        (root / "escape").unlink()


def test_reader_hashes_and_rejects_mismatch(tmp_path):
    meta = W.Bundle("L09/tiny", "L09/tiny.bin", "bfp16_gemv", [128, 256], [128, 256], 256, 128)
    data = np.random.default_rng(3).integers(0, 256, W.canonical_size(meta)[0], dtype=np.uint8)
    sha = write_bundle(tmp_path, meta, data)
    meta.sha256, meta.size_bytes = sha, data.size
    assert W._read_whole(tmp_path, meta) == data.tobytes()
    meta.sha256 = "0" * 64
    with pytest.raises(ValueError, match="sha256 mismatch"):
        W._read_whole(tmp_path, meta)
    meta.sha256 = ""
    r = W._Reader(tmp_path, meta)
    with pytest.raises(ValueError, match="Short read"):
        r.read(data.size + 1)
    r.close()


class _FakeLayer:
    def __init__(self, log, layer, geom):
        self.log, self.layer, self.geom = log, layer, geom
        self.gu_expert_bytes = geom.gu_bytes
        self.dn_expert_bytes = geom.hidden * geom.inter_pad * 9 // 8
        self.uploads = []

    def upload_d(self, bundle, expert0, data):
        self.uploads.append((bundle, expert0, bytes(data)))

    def expert_matrix(self, expert, part):
        return ("view", self.layer, expert, part)

    def set_router(self, *a):
        self.log.append(("router", self.layer) + a)

    def free(self):
        self.log.append(("free", self.layer))


class _FakeCtx:
    def __init__(self, log):
        self.log, self.layers = log, []

    def create_layer_d(self, layer, geom):
        lyr = _FakeLayer(self.log, layer, geom)
        self.layers.append(lyr)
        return lyr


class _FakeBackend:
    """Records what the loader registers (the host logic of GpuBackend.load_weights_d)."""

    def __init__(self):
        self.log = []
        self.ctx = _FakeCtx(self.log)
        self._layers, self.bundles, self.components = {}, {}, {}

    def register_bundle(self, name, data, M, K, fmt):
        self.bundles[name] = (bytes(data), M, K, fmt)

    def register_component(self, name, bundle, r0, r1, orig_k=None):
        self.components[name] = (bundle, r0, r1, orig_k)

    def register_view(self, name, matrix):
        self.bundles[name] = matrix


@pytest.fixture(scope="module")
def real_dir(tmp_path_factory):
    """L02's MoE bundles and L00's dense pair as real files (random bytes: the loader only
    moves them) with a manifest that leaves the other bundles out."""
    from weights_d_fixtures import manifest_entry

    root = tmp_path_factory.mktemp("weights_d_real")
    comps, bundles = W.canonical_specs()
    rng = np.random.default_rng(9)
    data, entries = {}, []
    for name in ("L02/moe_b1", "L02/moe_b2", "L02/shared_gu", "L00/dense_gu", "L00/dense_down"):
        buf = rng.integers(0, 256, W.canonical_size(bundles[name])[0], dtype=np.uint8)
        sha = write_bundle(root, bundles[name], buf)
        data[name] = buf
        entries.append(manifest_entry(bundles[name], comps, bundles[name].rel_file, sha))
    write_manifest(root, entries)
    return root, data


def test_loader_host_logic(real_dir):
    tmp_path, data = real_dir
    be = _FakeBackend()
    w = np.zeros((128, 2560), np.uint16)
    info = W.load_weights_d(be, tmp_path, require_complete=False, experts_per_read=40,
                            routers={2: (w, None)}, routed_scaling_factor=2.5)
    assert sorted(info["loaded"]) == sorted(["L02/moe_b1", "L02/moe_b2", "L02/shared_gu", "L00/dense_gu",
                                            "L00/dense_down"])
    lyr = be._layers[2]
    # moe_b1 then moe_b2, streamed in slices of 40 experts, reassembling the files exactly
    b1 = b"".join(d for b, _, d in lyr.uploads if b == 1)
    b2 = b"".join(d for b, _, d in lyr.uploads if b == 2)
    assert b1 == data["L02/moe_b1"].tobytes() and b2 == data["L02/moe_b2"].tobytes()
    assert [e0 for b, e0, _ in lyr.uploads if b == 2] == [0, 40, 80, 120]
    # the shared down is moe_b2's expert 128 in place (a view of the layer), served with K_in = 1088
    assert be.bundles["L02/shared_down"] == ("view", 2, 128, "down")
    assert be.components["model.layers.2.moe.shared_experts.down_proj.weight"] == ("L02/shared_down", 0, 2560, 1088)
    assert be.components["model.layers.2.moe.shared_experts.up_proj.weight"] == ("L02/shared_gu", 1088, 2176, 2560)
    assert be.bundles["L00/dense_gu"][1:] == (24064, 2560, "q4nx_gemv")
    assert be.components["model.layers.0.mlp.down_proj.weight"] == ("L00/dense_down", 0, 2560, 12032)
    assert ("router", 2, w, None, "sigmoid", True, 2.5) in be.log


def test_loader_rejects_corrupt_expert_bundle(real_dir):
    tmp_path, data = real_dir
    path = tmp_path / "L02" / "moe_b2.bin"
    bad = data["L02/moe_b2"].copy()
    bad[7] ^= 1
    path.write_bytes(bad.tobytes())
    try:
        be = _FakeBackend()
        with pytest.raises(ValueError, match="sha256 mismatch for L02/moe_b2"):
            W.load_weights_d(be, tmp_path, require_complete=False)
        assert 2 not in be._layers and ("free", 2) in be.log
    finally:
        path.write_bytes(data["L02/moe_b2"].tobytes())
    with pytest.raises(ValueError, match="not a MoE layer"):
        W.load_weights_d(_FakeBackend(), tmp_path, require_complete=False, layers=[0])
