"""CPU: a property of the grouped GEMM's gfx950 code that the compiler, not the source,
decides.

The GEMM loads the correction coefficients with inline-assembly loads that the compiler
does not count (``gload16`` in ``csrc/moe_prefill.hip``): it treats their destination
registers as written at issue, while the data arrives only by the kernel's own
``s_waitcnt vmcnt`` (also inline assembly).  Any instruction the compiler places between
the two that reads, copies or spills those registers sees whatever they held before.
Such a copy once sat before the wait, inside each branch of a switch over the wait
count, and corrupted one expert's rows in a few percent of calls.  This test compiles
the file to assembly and checks every such load.

It also checks the LDS copies (``global_load_lds_dwordx4``): on gfx9 one takes M0 as its
LDS address and needs one wait state after an SALU write of M0.  The compiler pads the
copies it emits itself; the grouped GEMM's copies are inline assembly that set M0 and
must pad it themselves.
"""

from __future__ import annotations

import re
import shutil
import subprocess

import pytest

from __graft_entry__ import _load_build_module

_VREG_RANGE = re.compile(r"v\[(\d+):(\d+)\]")
_VREG = re.compile(r"(?<![\w\[])v(\d+)\b")
_LOAD = re.compile(r"^\s*global_load_dwordx4 (v\[\d+:\d+\]), v\[\d+:\d+\], off\s*$")


def _vregs(text: str) -> set[int]:
    out = set()
    for m in _VREG_RANGE.finditer(text):
        out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    out.update(int(m.group(1)) for m in _VREG.finditer(text))
    return out


def _instructions(lines):
    """(index, text, in_inline_asm) for each instruction line."""
    in_asm = False
    for i, line in enumerate(lines):
        t = line.strip()
        if t.startswith(";;#ASMSTART"):
            in_asm = True
        elif t.startswith(";;#ASMEND"):
            in_asm = False
        elif t and not t.startswith((";", ".")) and not t.endswith(":"):
            yield i, t.split(";")[0].strip(), in_asm


def uncounted_load_hazards(asm_text: str, kernel_substr: str):
    """For each inline-assembly ``global_load_dwordx4`` in the kernels whose symbol
    contains ``kernel_substr``: the instructions between it and the next inline-assembly
    ``s_waitcnt vmcnt`` (in code order) that name one of its destination registers.
    Returns (number of loads, list of hazards)."""
    lines = asm_text.split("\n")
    insts = list(_instructions(lines))
    # function of each line: the last label "_Z...:" before it
    fn_at = {}
    cur = None
    for i, line in enumerate(lines):
        if re.match(r"^_Z\S*:", line):
            cur = line.split(":")[0]
        fn_at[i] = cur
    loads, hazards = 0, []
    for n, (i, t, in_asm) in enumerate(insts):
        m = _LOAD.match(t)
        if not (m and in_asm and kernel_substr in (fn_at[i] or "")):
            continue
        loads += 1
        dest = _vregs(m.group(1))
        for j, u, u_asm in insts[n + 1:]:
            if u_asm and u.startswith("s_waitcnt") and "vmcnt(" in u:
                break
            if fn_at[j] != fn_at[i]:
                hazards.append((i + 1, t, "no wait before the end of the function"))
                break
            if _LOAD.match(u) and u_asm:
                # a later uncounted load: only its address may not be one of ours
                if _vregs(u.split(",", 1)[1]) & dest:
                    hazards.append((i + 1, t, f"line {j + 1}: {u}"))
                continue
            if _vregs(u) & dest:
                hazards.append((i + 1, t, f"line {j + 1}: {u}"))
    return loads, hazards


def test_scanner_flags_a_copy_before_the_wait():
    """The checker itself, on a hand-written fragment: a copy of a loaded register before
    the wait is a hazard; the same copy after the wait is not."""
    head = "_ZN4rmoe19grouped_gemm_kernelE:\n\t;;#ASMSTART\n\tglobal_load_dwordx4 v[2:5], v[2:3], off\n\t;;#ASMEND\n"
    wait = "\t;;#ASMSTART\n\ts_waitcnt vmcnt(3) lgkmcnt(0)\n\ts_barrier\n\t;;#ASMEND\n"
    copy = "\tv_mov_b64_e32 v[20:21], v[4:5]\n"
    other = "\tv_mov_b64_e32 v[20:21], v[6:7]\n"
    assert uncounted_load_hazards(head + copy + wait, "grouped_gemm")[1]
    assert uncounted_load_hazards(head + other + wait + copy, "grouped_gemm") == (1, [])


def m0_lds_dma_hazards(asm_text: str):
    """LDS copies whose preceding instruction (in code order) writes M0."""
    hazards, prev = [], None
    for i, t, _ in _instructions(asm_text.split("\n")):
        if re.match(r"^(global|buffer)_load_lds", t) and prev and re.match(r"^s_\w+\s+m0\b", prev[1]):
            hazards.append((i + 1, prev[1], t))
        prev = (i, t)
    return hazards


def test_scanner_flags_an_lds_copy_right_after_m0():
    asm = "\ts_mov_b32 m0, s6\n\tglobal_load_lds_dwordx4 v[4:5], off\n"
    padded = "\ts_mov_b32 m0, s6\n\ts_nop 0\n\tglobal_load_lds_dwordx4 v[4:5], off\n"
    assert m0_lds_dma_hazards(asm) and not m0_lds_dma_hazards(padded)


def _device_asm(tmp_path, name: str) -> str:
    b = _load_build_module()
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not shutil.which(hipcc):
        pytest.skip("hipcc not available")
    src = b.PKG / "csrc" / name
    out = tmp_path / (src.stem + ".s")
    cmd = [hipcc, *b.COMMON, "-I", str(b.PKG.parent / "include"), "--cuda-device-only", "-S", str(src), "-o",
           str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    return out.read_text()


@pytest.fixture(scope="module")
def prefill_asm(tmp_path_factory):
    return _device_asm(tmp_path_factory.mktemp("asm"), "moe_prefill.hip")


def test_grouped_gemm_coefficient_registers_untouched_before_wait(prefill_asm):
    loads, hazards = uncounted_load_hazards(prefill_asm, "grouped_gemm_kernel")
    # eight coefficient loads ahead of the K loop and four per later block, per tile class
    assert loads >= 36, loads
    assert not hazards, hazards[:10]


@pytest.mark.parametrize("name", ["moe_prefill.hip", "moe_decode_stack.hip"])
def test_lds_copies_wait_after_m0(prefill_asm, tmp_path, name):
    text = prefill_asm if name == "moe_prefill.hip" else _device_asm(tmp_path, name)
    assert text.count("global_load_lds_dwordx4") > 0
    hazards = m0_lds_dma_hazards(text)
    assert not hazards, hazards[:10]
