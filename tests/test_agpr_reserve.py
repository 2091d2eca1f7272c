"""Register-level invariants of the 64-rows-per-wave attention kernels, checked
on their gfx950 assembly (CPU only: hipcc cross-compiles).

Those kernels keep the O accumulators in AGPRs a128..a255 that only inline asm
touches (csrc/agpr_tiles.h), and accumulate into them with asm MFMAs that the
compiler's hazard recognizer does not see. The tests compile attn_kernels.hip
with the library's flags and check, for every such kernel:

* no compiler-emitted instruction (outside the inline-asm blocks) reads or
  writes a128..a255, so the compiler keeps nothing of its own there;
* no asm MFMA reads a VGPR that one of the two instructions before it wrote
  (a VALU write needs 2 wait states before an MFMA reads it);
* every asm block that reads, scales or zeroes the accumulators is preceded
  by at least 24 wait states of padding after the last MFMA before it.
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "delta-attention_amd")

pytestmark = pytest.mark.skipif(not os.path.exists("/opt/rocm/bin/hipcc") and not shutil.which("hipcc"),
                                reason="hipcc is not installed")


@pytest.fixture(scope="module")
def kernels(tmp_path_factory):
    import sys
    sys.path.insert(0, PKG)
    import build_lib
    out = str(tmp_path_factory.mktemp("isa") / "attn.s")
    flags = [f for f in build_lib.HIPCC_FLAGS if f not in ("-shared", "-fPIC")]
    cmd = [build_lib.hipcc(), *flags, "--cuda-device-only", "-S",
           f"-I{build_lib.INCLUDE}", f"-I{build_lib.CSRC}",
           os.path.join(build_lib.CSRC, "attn_kernels.hip"), "-o", out]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    s = open(out).read()
    ks = {}
    for m in re.finditer(r"^(_ZN2da15attn_fwd_kernel\S+):(.*?)^\.Lfunc_end", s, re.S | re.M):
        # template arguments <T, D, MODE, RG>: the 64-rows-per-wave kernels end in Li2EEEv
        if m.group(1).endswith("Li2EEEvNS_8AttnArgsE"):
            ks[m.group(1)] = m.group(2).splitlines()
    assert len(ks) >= 4, "bf16 and fp16 kernels (1) and fused at 64 rows per wave"
    return ks


def _regs(spec):
    m = re.fullmatch(r"([av])\[(\d+):(\d+)\]", spec)
    if m:
        return {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.fullmatch(r"([av])(\d+)", spec)
    return {(m.group(1), int(m.group(2)))} if m else set()


def _instrs(lines):
    """(text, in_asm) for each instruction line."""
    in_asm = False
    for line in lines:
        t = line.strip()
        if t.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if t.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if not t or t.startswith(";") or t.startswith(".") or t.endswith(":"):
            continue
        yield t.split(";")[0].strip(), in_asm


def _operands(text):
    return re.findall(r"\b[av]\[\d+:\d+\]|\b[av]\d+\b", text)


def test_compiler_never_touches_reserved_agprs(kernels):
    for name, lines in kernels.items():
        bad = [t for t, in_asm in _instrs(lines)
               if not in_asm and any(r[0] == "a" and r[1] >= 128
                                     for o in _operands(t) for r in _regs(o))]
        assert not bad, f"{name}: {bad[:3]}"


def test_asm_mfma_sources_two_wait_states_after_valu(kernels):
    for name, lines in kernels.items():
        ins = list(_instrs(lines))
        n_checked = 0
        for i, (t, in_asm) in enumerate(ins):
            if not (in_asm and t.startswith("v_mfma") and " a[" in t.split(",")[0]):
                continue
            n_checked += 1
            srcs = set()
            for o in _operands(t)[1:]:
                srcs |= {r for r in _regs(o) if r[0] == "v"}
            for p, _ in ins[max(0, i - 2):i]:
                if p.startswith("v_") and not p.startswith("v_mfma"):
                    ops = _operands(p)
                    dst = _regs(ops[0]) if ops else set()
                    assert not (dst & srcs), f"{name}: '{p}' then '{t}'"
        assert n_checked >= 32, name


def test_accumulator_access_padded_after_mfma(kernels):
    for name, lines in kernels.items():
        ins = list(_instrs(lines))
        since = None   # wait states since the last asm MFMA on the reserved tiles
        for t, in_asm in ins:
            if in_asm and t.startswith("v_mfma") and " a[" in t.split(",")[0]:
                since = 0
                continue
            if since is None:
                continue
            m = re.match(r"s_nop (\d+)", t)
            if m:
                since += int(m.group(1)) + 1
                continue
            if in_asm and t.startswith("v_accvgpr") and any(
                    r[0] == "a" and r[1] >= 128 for o in _operands(t) for r in _regs(o)):
                assert since >= 24, f"{name}: '{t}' {since} wait states after an MFMA"
                since = None
                continue
            since += 1


def test_checks_catch_planted_violations():
    """The three checks, run on short synthetic listings that break each rule."""
    touch = [";;#ASMSTART", "v_mfma_f32_32x32x16_bf16 a[128:143], v[0:3], v[4:7], a[128:143]",
             ";;#ASMEND", "v_accvgpr_read_b32 v9, a130"]
    with pytest.raises(AssertionError):
        test_compiler_never_touches_reserved_agprs({"planted": touch})
    early = ["v_cvt_pk_bf16_f32 v5, v1, v2", ";;#ASMSTART",
             "v_mfma_f32_32x32x16_bf16 a[128:143], v[0:3], v[4:7], a[128:143]", ";;#ASMEND"]
    with pytest.raises(AssertionError):
        test_asm_mfma_sources_two_wait_states_after_valu({"planted": early * 40})
    unpadded = [";;#ASMSTART", "v_mfma_f32_32x32x16_bf16 a[128:143], v[0:3], v[4:7], a[128:143]",
                ";;#ASMEND", "s_nop 7", ";;#ASMSTART", "v_accvgpr_read_b32 v9, a130", ";;#ASMEND"]
    with pytest.raises(AssertionError):
        test_accumulator_access_padded_after_mfma({"planted": unpadded})
    padded = [";;#ASMSTART", "v_mfma_f32_32x32x16_bf16 a[128:143], v[0:3], v[4:7], a[128:143]",
              ";;#ASMEND", ";;#ASMSTART", "s_nop 15", "s_nop 7", ";;#ASMEND",
              ";;#ASMSTART", "v_accvgpr_read_b32 v9, a130", ";;#ASMEND"]
    test_accumulator_access_padded_after_mfma({"planted": padded})
