"""The hand-scheduled key-step loop of flexrel_w64.hip (CPU only).

* The generator's checks (csrc/gen_w64_step.py over csrc/gen_asm.py) pass
  on the loop it writes, and they catch planted mistakes: a removed wait
  state, a missing LDS wait, a missing copy wait, a missing wait at the exit.
* The special steps' per-path blocks: the softmax shares its block with the
  phase's products, and no copy's offset register is overwritten before
  the copy reads it.
* Operand placement in the compiled kernel: the loop's text names fixed
  registers (v0-v148, v152-v231, s64-s95);
  every register the compiler substituted for a named operand must lie
  outside them.  (An operand bound to a fixed register whose value is
  undefined at the loop entry lets the compiler place other inputs inside
  it -- a mistake this test catches.)
"""

from __future__ import annotations

import importlib.util
import re
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
CSRC = REPO / "sidon-triton_amd" / "csrc"


def _gen(name="gen_w64_step"):
    sys.path.insert(0, str(CSRC))
    try:
        spec = importlib.util.spec_from_file_location(name, CSRC / f"{name}.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
    finally:
        sys.path.pop(0)
    return mod


def test_hazard_check_catches_a_removed_wait_state():
    gen = _gen()
    _, step, _ = gen.build()
    seq = gen.FENCE + step
    # plant: drop the wait states between a probability conversion and the
    # row-sum product reading it by moving the product right after it
    i = next(k for k, ins in enumerate(seq) if ins.text.startswith("v_mfma_f32_16x16x32_f16"))
    cvt = next(k for k, ins in enumerate(seq) if ins.text.startswith("v_cvt_pk_f16_f32"))
    reader = next(k for k in range(cvt + 1, len(seq)) if seq[k].kind == "mfma" and seq[k].reads & seq[cvt].writes)
    planted = seq[:cvt + 1] + [seq[reader]] + seq[cvt + 1:reader] + seq[reader + 1:]
    with pytest.raises(AssertionError, match="hazard"):
        gen.check_hazards(planted)
    gen.check_hazards(seq)
    del i


def test_wait_check_catches_a_missing_lds_wait():
    gen = _gen()
    _, step, _ = gen.build()
    # plant: drop the lgkmcnt wait between the K operand reads of the K slot
    # and the copy that refills that slot
    waits = [k for k, ins in enumerate(step) if ins.text == "s_waitcnt lgkmcnt(0)"]
    assert waits
    planted = step[:waits[0]] + step[waits[0] + 1:]
    with pytest.raises(AssertionError):
        gen.check_waits(planted + planted, [])
    gen.check_waits(step + step, [])


def test_w64_generator_checks_pass():
    gen = _gen("gen_w64_step")
    loop, step, cycles = gen.build()
    assert len(step) > 100 and 500 < cycles < 1000
    kinds = [i.kind for i in step]
    # two blocks per step: 16 score, 16 PV and 4 row-sum products, 32 exp2
    assert kinds.count("mfma") == 20 and kinds.count("trans") == 32
    assert "a[" not in " ".join(i.text for i in loop)   # VGPRs only (two wavefronts per SIMD)


def test_w64_wait_check_catches_a_missing_copy_wait():
    gen = _gen("gen_w64_step")
    _, step, _ = gen.build()
    # plant: drop the vmcnt wait before the K operand reads of the K slot
    waits = [k for k, ins in enumerate(step) if ins.text == "s_waitcnt vmcnt(4)"]
    assert waits
    planted = step[:waits[0]] + step[waits[0] + 1:]
    with pytest.raises(AssertionError):
        gen.check_waits(planted + planted, [])
    gen.check_waits(step + step, [])


def test_loop_returns_with_no_lds_read_in_flight():
    """The loop statement's register outputs must be final when it ends: its
    last V^T and K operand reads are LDS reads, and the compiled code after
    it may move register-only work (the last PV products) above any wait of
    its own.  The tail after the L_end label retires every LDS read and every
    copy; dropping that wait must trip the check."""
    gen = _gen()
    loop, step, _ = gen.build()    # checks every exit path
    end = max(k for k, ins in enumerate(loop) if ins.text == "L_end_%=:")
    tail = loop[end + 1:]
    assert any(ins.text == "s_waitcnt lgkmcnt(0)" for ins in tail)
    copies = True
    read = next(ins for ins in step if ins.kind == "lds")    # an operand read left in flight
    gen.assert_quiet([read] + tail, copies=copies)
    planted = [ins for ins in tail if ins.text != "s_waitcnt lgkmcnt(0)"]
    with pytest.raises(AssertionError, match="in flight at the end"):
        gen.assert_quiet([read] + planted, copies=copies)


def _compiled_loop(src="flexrel_w64.hip"):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    sys.path.insert(0, str(REPO / "sidon-triton_amd"))
    try:
        import build as sidon_build
    finally:
        sys.path.pop(0)
    sidon_build.generate()
    flags = [f for f in sidon_build.HIP_FLAGS if f not in ("-fPIC", "-shared")]
    out = subprocess.run([hipcc, *flags, "--cuda-device-only", "-S", "-o", "-", f"-I{REPO / 'include'}",
                          str(CSRC / src)], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stderr[-2000:]
    asm = out.stdout
    blocks = re.findall(r";;#ASMSTART\n(.*?);;#ASMEND", asm, re.S)
    loop = [b for b in blocks if "L_sp_top_" in b]
    assert len(loop) == 1
    return [ln.strip() for ln in loop[0].splitlines() if ln.strip()]


def _template(inc="flexrel_w64_step.inc", macro="SIDON_W64_LOOP"):
    text = (CSRC / inc).read_text()
    body = text.split(f"#define {macro} \\\n", 1)[1]
    return [m.group(1).strip() for m in re.finditer(r'"(.*?)\\n\\t"', body)]


def _reg_set(tok):
    m = re.fullmatch(r"([vsa])(\d+)", tok) or re.fullmatch(r"([vsa])\[(\d+):(\d+)\]", tok)
    assert m, tok
    lo = int(m.group(2))
    hi = int(m.group(3)) if m.lastindex == 3 else lo
    return {(m.group(1), r) for r in range(lo, hi + 1)}


KERNELS = {
    "w64": ("flexrel_w64.hip", "flexrel_w64_step.inc", "SIDON_W64_LOOP",
            {("v", r) for r in list(range(0, 149)) + list(range(152, 232))},
            ("qbase", "laned", "g8", "ka0", "ka3", "tv00", "ko0", "kl0", "m0", "m1", "nslow", "w", "q0", "lk")),
}


@pytest.mark.parametrize("kernel", sorted(KERNELS))
def test_compiled_operands_avoid_the_loop_registers(kernel):
    src, inc, macro, fixed, inputs = KERNELS[kernel]
    compiled = _compiled_loop(src)
    template = [ln for ln in _template(inc, macro)]
    assert len(compiled) == len(template)
    bound = {}
    for tpl, got in zip(template, compiled):
        if "%[" not in tpl:
            continue
        # split both lines into tokens and pair the placeholders
        tt = re.split(r"[\s,]+", tpl.replace("%=", "0"))
        gt = re.split(r"[\s,]+", got)
        assert len(tt) == len(gt), (tpl, got)
        for a, b in zip(tt, gt):
            if a.startswith("%["):
                name = a[2:a.index("]")]
                bound.setdefault(name, set()).add(b)
    reserved = fixed | {("s", r) for r in range(64, 96)}
    seen = {}
    for name, regs in bound.items():
        assert len(regs) == 1, (name, regs)   # one register per operand throughout the loop
        reg = next(iter(regs))
        rs = _reg_set(reg)
        assert not (rs & reserved), (name, reg)
        for other, ors in seen.items():
            assert not (rs & ors), (name, reg, other)
        seen[name] = rs
    # every input the loop reads is bound
    for name in inputs:
        assert name in bound, name


def _special_blocks(gen):
    """{(slot parity, phase, path): scheduled block} of the special steps."""
    pre = gen.special_preamble()
    out = {}
    for sl in (0, 1):
        _, phases = gen.special_step(sl, gen.FENCE + pre)
        for J, variants in enumerate(phases):
            for pth, seq in variants.items():
                start = max(k for k, ins in enumerate(seq) if ins.kind == "label" and f"L_v{sl}{J}{pth}_" in ins.text)
                out[(sl, J, pth)] = seq[start + 1:]
    return out


def test_special_step_paths_interleave_their_softmax_with_the_products():
    """Each phase of a special step has one scheduled block per path of its
    item; the softmax (after the gathered biases' wait) shares its block with
    the phase's products rather than following all of them, and the six
    paths cover the general code's cases."""
    gen = _gen()
    assert set(gen.PATHS) == {"P", "G", "GM", "F0", "FG", "FGM"}
    for (sl, J, pth), block in _special_blocks(gen).items():
        kinds = [ins.kind for ins in block]
        assert kinds.count("mfma") == 10, (sl, J, pth)
        wait = next(k for k, ins in enumerate(block) if ins.tag == f"W.{J}")   # the gathered biases
        softmax = next(k for k in range(wait + 1, len(block)) if block[k].kind in ("valu", "trans"))
        last_mfma = max(k for k, kind in enumerate(kinds) if kind == "mfma")
        assert softmax < last_mfma, (sl, J, pth)
        exps = sum(1 for ins in block if ins.text.startswith("v_exp_f32"))
        assert exps == 16 + (1 if pth.startswith("F") else 0), (sl, J, pth)


def test_special_step_copies_read_their_offsets_before_the_softmax_reuses_them():
    """The K copies of a special step take their lane offsets from v145-v148,
    which the softmax also uses as temporaries: in every scheduled block no
    instruction writes a copy's offset register before that copy, and the
    check this test applies catches a planted write."""
    gen = _gen()

    def check(block):
        for k, ins in enumerate(block):
            if ins.kind != "dma":
                continue
            for prev in block[:k]:
                assert not (prev.writes & ins.reads - {"m0"}), (prev.text, ins.text)

    blocks = _special_blocks(gen)
    for block in blocks.values():
        check(block)
    block = next(b for (sl, J, pth), b in blocks.items() if J == 0 and pth == "FG")
    dmas = [k for k, ins in enumerate(block) if ins.kind == "dma" and ins.reads & {"v145", "v146", "v147", "v148"}]
    assert len(dmas) == 4
    dma = dmas[0]
    writer = next(ins for ins in block[dma:] if ins.writes & block[dmas[-1]].reads - {"m0"})  # e.g. the max's temporaries
    planted = block[:dma] + [writer] + block[dma:]
    with pytest.raises(AssertionError):
        check(planted)
