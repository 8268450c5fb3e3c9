"""Shared pieces of the hand-scheduled gfx950 loop generator (gen_w64_step.py):
the instruction record, the issue model and list scheduler, and the
wait-state checks.

* ``Ins`` records one instruction with the registers it reads and writes
  (``srcc``: an MFMA's accumulator input), its kind and, for LDS reads and
  copies, the ring slot it touches.
* ``schedule`` interleaves a phase's MFMAs (in order, with the memory
  operations attached before or after each) with its vector instructions
  (any order their dependencies and wait states allow): an MFMA goes out
  when the matrix core is free, a ready vector instruction otherwise.  Its
  issue model is one wavefront per SIMD on MI355X: a vector instruction
  every ~5.44 cycles (v_exp_f32 9.14), a 32x32x16 MFMA holding the matrix
  core 32 cycles and a 16x16x32 one 16.
* ``required_states`` / ``check_hazards`` / ``pad`` apply the wait states
  the hardware does not interlock on gfx950 (MFMA result -> VALU, LDS or
  VMEM access; VALU write -> MFMA operand; transcendental -> VALU;
  VALU -> v_permlane32_swap; M0 -> LDS DMA; accumulator read -> overwrite);
  ``assert_quiet`` checks that every LDS read and copy has retired at the
  end of a sequence.
"""

from __future__ import annotations


def vregs(lo, n):
    return {f"v{lo + i}" for i in range(n)}


def aregs(lo, n):
    return {f"a{lo + i}" for i in range(n)}


class Ins:
    """One instruction: text, kind and the registers it reads / writes."""

    def __init__(self, text, kind, reads=(), writes=(), srcc=(), passes=0, tag="", lds_slot=None):
        self.text = text
        self.kind = kind          # mfma, valu, trans, permlane, salu, m0, dma, lds, waitcnt, nop, branch, label
        self.reads = set(reads)
        self.writes = set(writes)
        self.srcc = set(srcc)     # MFMA accumulator input
        self.passes = passes
        self.tag = tag
        self.lds_slot = lds_slot  # LDS ring slot read (lds) or written (dma)
        self.deps = []            # tags that must be issued earlier (ordering only)

    def states(self):
        """Wait states this instruction provides (s_nop N: N + 1; labels and
        branches: counted as none)."""
        if self.kind == "nop":
            return int(self.text.split()[1]) + 1
        if self.kind in ("label", "branch"):
            return 0
        return 1


def valu(text, reads=(), writes=(), tag="", kind="valu"):
    return Ins(text, kind, reads=reads, writes=writes, tag=tag)


def salu(text):
    return Ins(text, "salu")


def nop(n):
    return Ins(f"s_nop {n}", "nop")


def label(name):
    return Ins(f"{name}:", "label")


def branch(text):
    return Ins(text, "branch")


# ---- issue model (cycles of one wavefront; measured on MI355X with one
# wavefront per SIMD: VALU 5.44, v_exp_f32 9.14, MFMA 32x32x16 32.1 and
# 16x16x32 16.6 on the matrix core) ----
COSTS = {"valu": 5.44, "trans": 9.14, "permlane": 5.44, "mfma": 4.0, "salu": 4.0, "m0": 4.0, "dma": 4.0,
         "lds": 4.0, "gload": 4.0, "waitcnt": 4.0, "nop": 4.0, "branch": 4.0, "label": 0.0}
PIPE = {8: 32.0, 4: 16.0}


def _regs(op):
    kind, lo = op
    return vregs(lo, 4) if kind == "v" else aregs(lo, 4)


def mfma32(dst, a, b, c, tag):
    srcc = set() if c is None else vregs(c, 16)
    c_txt = "0" if c is None else f"v[{c}:{c + 15}]"
    return Ins(f"v_mfma_f32_32x32x16_f16 v[{dst}:{dst + 15}], {a[0]}[{a[1]}:{a[1] + 3}], "
               f"{b[0]}[{b[1]}:{b[1] + 3}], {c_txt}",
               "mfma", reads=_regs(a) | _regs(b), writes=vregs(dst, 16), srcc=srcc, passes=8, tag=tag)


def mfma16(dst, a, b, tag):
    return Ins(f"v_mfma_f32_16x16x32_f16 v[{dst}:{dst + 3}], {a[0]}[{a[1]}:{a[1] + 3}], "
               f"{b[0]}[{b[1]}:{b[1] + 3}], v[{dst}:{dst + 3}]",
               "mfma", reads=_regs(a) | _regs(b), writes=vregs(dst, 4), srcc=vregs(dst, 4), passes=4, tag=tag)


def pad(seq):
    """Inserts s_nop where a block's own instructions need wait states."""
    i = 0
    while i < len(seq):
        c = seq[i]
        states, need = 0, 0
        for p in reversed(seq[max(0, i - 40):i]):
            need = max(need, required_states(p, c) - states)
            states += p.states()
        if need > 0:
            seq.insert(i, nop(need - 1))
            i += 1
        i += 1


# ---- hazards: wait states required between a producer and a consumer ----
def required_states(p, c):
    """Wait states that must separate producer p from a later consumer c
    (0 if none)."""
    need = 0
    if p.kind == "mfma":
        touched = c.reads | c.writes | c.srcc
        if c.kind == "mfma":
            if p.writes & c.srcc:
                if not (c.srcc == p.writes and c.writes == p.writes):
                    raise AssertionError(f"partial accumulator overlap: {p.text} -> {c.text}")
            if p.writes & c.reads:
                raise AssertionError(f"MFMA result as a multiplicand: {p.text} -> {c.text}")
            if p.writes & c.writes and not (c.srcc == p.writes):
                need = max(need, p.passes + 4)
        elif p.writes & touched:
            need = max(need, p.passes + 4)          # XDL write -> VALU/LDS/VMEM access
        if c.kind in ("valu", "trans", "permlane", "lds", "gload") and p.srcc & c.writes:
            need = max(need, 2 * p.passes)          # accumulator read late -> overwrite
    if p.kind in ("valu", "trans", "permlane") and c.kind == "mfma" and p.writes & (c.reads | c.srcc):
        need = max(need, 2)                         # VALU write -> MFMA read
    if p.kind == "trans" and c.kind in ("valu", "trans", "permlane") and p.writes & c.reads:
        need = max(need, 1)                         # transcendental result forwarding
    if p.kind in ("valu", "trans") and c.kind == "permlane" and p.writes & c.reads:
        need = max(need, 2)                         # VALU write -> v_permlane32_swap
    if p.kind == "m0" and c.kind == "dma":
        need = max(need, 1)                         # M0 -> LDS DMA
    return need


def check_hazards(seq):
    """Raises on a wait-state violation anywhere in seq (a list of Ins)."""
    for ci, c in enumerate(seq):
        states = 0
        for pi in range(ci - 1, max(-1, ci - 40), -1):
            p = seq[pi]
            need = required_states(p, c)
            if need > states:
                raise AssertionError(f"hazard: {p.text!r} -> {c.text!r}: {states} wait states, {need} needed")
            states += p.states()


def assert_quiet(seq, copies=True):
    """Raises unless every LDS read (and, with copies, every copy) issued in
    seq has retired by its end (whatever was in flight before it, too)."""
    lds, vm = 99, 99   # (anything in flight before seq counts)
    for c in seq:
        if c.kind == "waitcnt":
            kind, n = c.text.split()[1].split("(")
            n = int(n.rstrip(")"))
            if kind == "lgkmcnt":
                lds = min(lds, n)
            else:
                vm = min(vm, n)
            continue
        lds += c.kind == "lds"
        vm += c.kind in ("dma", "gload")
    if lds or (copies and vm):
        raise AssertionError(f"{lds} LDS reads / {vm} copies in flight at the end")


# ---- list scheduler ----
def schedule(mf, pre, post, valu_list, history):
    """Interleaves the MFMAs (in order, with their memory operations) with
    the vector list (any order its dependencies and wait states allow):
    an MFMA goes out when the matrix core is free, a ready vector
    instruction otherwise.  Returns (instructions, modelled cycles)."""
    out = []
    t_now = 0.0
    pipe_free = 0.0
    issued = set()

    def hazard_need(c):
        states = 0
        need_extra = 0
        seq = history + out
        for pi in range(len(seq) - 1, max(-1, len(seq) - 41), -1):
            p = seq[pi]
            need = required_states(p, c)
            if need > states:
                need_extra = max(need_extra, need - states)
            states += p.states()
        return need_extra

    def emit(ins):
        nonlocal t_now, pipe_free
        if ins.kind == "mfma":
            t_now = max(t_now, pipe_free)
            pipe_free = t_now + PIPE[ins.passes]
        t_now += COSTS[ins.kind]
        out.append(ins)
        issued.add(ins.tag)

    pending = list(valu_list)
    mi = 0
    while mi < len(mf) or pending:
        m = mf[mi] if mi < len(mf) else None
        ready_v = None
        for v in pending:
            if all(d in issued for d in v.deps) and hazard_need(v) == 0:
                ready_v = v
                break
        if m is not None and (pipe_free <= t_now + 2.0 or ready_v is None):
            for op in pre[m.tag]:
                extra = hazard_need(op)
                if extra:
                    emit(nop(extra - 1))
                emit(op)
            extra = hazard_need(m)
            if extra:
                emit(nop(extra - 1))
            emit(m)
            for op in post[m.tag]:
                extra = hazard_need(op)
                if extra:
                    emit(nop(extra - 1))
                emit(op)
            mi += 1
            continue
        if ready_v is not None:
            emit(ready_v)
            pending.remove(ready_v)
            continue
        # nothing ready: the oldest pending vector instruction waits out its hazard
        v = next(v for v in pending if all(d in issued for d in v.deps))
        emit(nop(hazard_need(v) - 1))
    return out, t_now


FENCE = [nop(7), nop(7), nop(7)]
