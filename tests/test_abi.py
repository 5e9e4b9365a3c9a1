"""CPU checks of the C ABI: the library loads and exports every declared entry point."""

from __future__ import annotations

import re
from pathlib import Path

import pytest

import raon_npu_amd
from raon_npu_amd import _lib
from raon_npu_amd.geometry import BASELINE, RAON_1_MINI, MoeGeometry

HEADER = Path(__file__).resolve().parents[1] / "include" / "raon_moe.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rmoe_[a-z_0-9]+)\s*\(", text)))


def test_header_declares_the_bound_functions():
    assert set(declared_functions()) == set(_lib.SIGNATURES)


def test_library_loads_and_exports_every_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.rmoe_version().decode().endswith("gfx950")


def test_error_mapping_without_a_device():
    lib = _lib.load()
    # A null context is rejected before any HIP call.
    with pytest.raises(ValueError):
        _lib.check(lib.rmoe_synchronize(None))
    with pytest.raises(ValueError):
        _lib.check(lib.rmoe_layer_free(None, 0))


def test_geometry_matches_reference_constants():
    # kernels/moe/pack.py:53-75 (reference model) and SURVEY/BASELINE byte counts.
    assert RAON_1_MINI.gu_bytes == 3_481_600
    assert RAON_1_MINI.dn_bytes == 2_048_000
    assert RAON_1_MINI.inter_pad == 1280
    assert BASELINE.gu_bytes == 1_966_080 and BASELINE.dn_bytes == 983_040
    assert BASELINE.expert_bytes == 2_949_120
    assert BASELINE.decode_bytes() == 27_066_368
    assert BASELINE.flops_per_assignment == 9_437_184
    with pytest.raises(ValueError):
        MoeGeometry(hidden=2000, inter=768)


def test_package_exports():
    assert raon_npu_amd.BASELINE.top_k == 8


def test_stream_argument_mapping():
    """The wrappers' stream argument: None selects the context's stream (the library's
    NULL); a torch stream passes its handle, and torch's default stream (handle 0, HIP's
    null stream) is passed as hipStreamLegacy (1), since a 0 handle would select the
    context's own stream, which is not ordered with torch's work."""
    from raon_npu_amd.device import _stream_ptr

    class FakeStream:
        def __init__(self, handle):
            self.cuda_stream = handle

    assert _stream_ptr(None) is None
    assert _stream_ptr(FakeStream(0)) == 1
    assert _stream_ptr(FakeStream(0x7F00AB00)) == 0x7F00AB00
    assert _stream_ptr(0x1234) == 0x1234
