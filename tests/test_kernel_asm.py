"""Checks on the gfx950 assembly of the bf16/f16 direct-to-LDS GEMM (no GPU
needed: hipcc compiles it here).

The NN and TN kernels issue their global-to-LDS loads as inline asm
(rt_dev::dma16_asm) so that the compiler does not order each stage's
fragment reads behind the next stage's loads.  That relies on two facts
about the code the compiler emits, which a compiler change could break
silently; these tests pin them:

* M0 (the LDS destination of the load) is written only by the asm statement
  itself, right before each load, and read by nothing else;
* inside the main loop no `s_waitcnt vmcnt` comes before the stage barrier
  (the wait the asm form exists to remove).
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "rgpu_amd", "csrc")

# gemm_half_dma_kernel<256, 256, 2, 4, A_KC, B_KC, IS_BF16, 64, 2>: the NN and
# TN instantiations (B M/N-contiguous) of the 256x256 tile, bf16 and f16.
ASM_KERNELS = {
    "NN bf16": "ILi256ELi256ELi2ELi4ELb1ELb0ELb1ELi64ELi2E",
    "NN f16": "ILi256ELi256ELi2ELi4ELb1ELb0ELb0ELi64ELi2E",
    "TN bf16": "ILi256ELi256ELi2ELi4ELb0ELb0ELb1ELi64ELi2E",
    "TN f16": "ILi256ELi256ELi2ELi4ELb0ELb0ELb0ELi64ELi2E",
}


def _hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    return None


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not available")
    out = str(tmp_path_factory.mktemp("asm") / "gemm_half.s")
    cmd = [hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-I", os.path.join(ROOT, "include"), "-I", CSRC, "-S", "--cuda-device-only",
           os.path.join(CSRC, "gemm_half.hip"), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return open(out).read()


def _body(asm_text, key):
    names = [n for n in re.findall(r"^(_Z\w*gemm_half_dma_kernel\w*):", asm_text, re.M) if key in n]
    assert len(names) == 1, (key, names)
    body = asm_text[asm_text.index(names[0] + ":"):]
    body = body[:body.index(".Lfunc_end")]
    return [l.strip() for l in body.split("\n")]


def _code(lines):
    """Instruction lines (no labels, directives or comments)."""
    return [l for l in lines if l and not l.startswith((".", ";")) and not l.endswith(":")]


@pytest.mark.parametrize("kind", sorted(ASM_KERNELS))
def test_m0_is_set_by_each_lds_load_and_used_by_nothing_else(asm, kind):
    code = _code(_body(asm, ASM_KERNELS[kind]))
    loads = [i for i, l in enumerate(code) if l.startswith("buffer_load_dwordx4") and l.endswith(" lds")]
    assert loads, "the kernel issues no direct-to-LDS loads"
    for i in loads:
        assert re.fullmatch(r"s_mov_b32 m0, s\d+", code[i - 1]), (kind, code[i - 1], code[i])
    others = [l for i, l in enumerate(code) if "m0" in l and not (i + 1 in loads and l.startswith("s_mov_b32 m0"))]
    assert not others, (kind, others[:5])


@pytest.mark.parametrize("kind", sorted(ASM_KERNELS))
def test_main_loop_waits_for_loads_only_at_the_stage_barrier(asm, kind):
    lines = _body(asm, ASM_KERNELS[kind])
    head = next(i for i, l in enumerate(lines) if "Inner Loop Header" in l)
    code = _code(lines[head:])
    bar = next(i for i, l in enumerate(code) if l.startswith("s_barrier"))
    vm = [i for i, l in enumerate(code[:bar]) if l.startswith("s_waitcnt") and "vmcnt" in l]
    # exactly one load wait before the first barrier: the one right before it
    assert vm == [bar - 1], (kind, [code[i] for i in vm], bar)
    mfma_before = sum(1 for l in code[:bar] if l.startswith("v_mfma"))
    assert mfma_before > 0
