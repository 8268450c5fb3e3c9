"""Generates flexrel_wide_step.inc: the key-step loop of flexrel_wide.hip as
hand-scheduled gfx950 assembly (one inline-assembly text).

Run by build.py before every compile (``python gen_wide_step.py`` writes the
file next to this script).  The loop runs a wavefront's key steps in the
kernel's processing order: the special steps first (band steps, where a
block needs the per-score q.rel gather; the step straddling LK; the first
step, which sets the running max exactly), then the plain steps (every block
entirely left or entirely right of the window).  Every item computes exactly
what the general code of flexrel_wide.hip computes for it -- the same MFMAs
on the same operands, the same fma / exp2 / fp16 rounding per score, the same
row-sum accumulation -- so the kernel's C++ rerun (taken when a probability
leaves the fp16 range) reproduces every query that did not overflow bit for
bit.

The plain step is ordered for a single wavefront per SIMD, which issues one
vector instruction every ~5.4 cycles (v_exp_f32: ~9.1) while a 32x32x16 MFMA
holds the matrix core for 32 cycles: a phase's 40 vector instructions and
its ten MFMAs (288 matrix-core cycles) take about the same time, so a list
scheduler over that issue model (COSTS) interleaves them.  The special steps
(a few per wavefront) run the same MFMA skeleton with the bias gather beside
it and a straight-line, uniformly branched softmax after it.

Registers (fixed; the C++ side binds every value to them with physical
register constraints):

  v[0:127]    O^T accumulators: block J, dims half db at v[32 J + 16 db]
  v[128:143]  scores buffer 0, v[144:159] buffer 1 (plain steps: softmaxed in place)
  v[160:175]  fp16 probabilities [buffer][16-key half], 4 VGPRs each
  v[176:191]  running row sums, block J at v[176 + 4 J]
  v[192:195]  the 0/1 selector operand of the row-sum MFMA
  v[196:220]  scratch (special steps: biases / scores t0-t15, copy offsets,
              five temporaries; plain steps: exponent offsets in v[196:203])
  a[0:63]     Q^T operands: block J, k-step s at a[16 J + 4 s]
  a[64:79]    K operands of the current step (k-step s at a[64 + 4 s])
  a[80:95]    V^T operands [hh][db] at a[80 + 8 hh + 4 db]
  s64 step index j, s65 nu, s66 jump, s67 ring LDS address, s68 scale,
  s[70:73] copy bases (K, V), s[74:77] copy advances, s69 and s[78:95] scratch

Phase J of step j (item i = 4 j + J, buffer bf = J & 1) issues the row sums
of item i - 1 (two 16x16x32 MFMAs accumulating into its block's running
sums), S^T of item i + 1 (four 32x32x16 MFMAs), O^T += V^T P^T of item i - 2
(four) and the softmax of item i.  Memory: K(j + 2) copy in phase 0, V(j)
transpose reads at the end of phase 1, V(j + 2) copy and K(j + 1) operand
reads in phase 2 -- the copy order and wait counts of the C++ step.

Checks (raise on failure): the wait-state rules the compiler applies to
gfx950 code (required_states) over every order the loop can run -- every
branch path of the special softmax, every step alternation, the entry and
exit -- and the outstanding-load accounting of every LDS read and ring slot
(check_waits).
"""

from __future__ import annotations

import itertools
import sys
from pathlib import Path

OUT = Path(__file__).resolve().parent / "flexrel_wide_step.inc"

# ---- register map ----
SACC = (128, 144)
PK = 160          # pk[bf][hh] at PK + 8 bf + 4 hh
RSACC = 176       # block J at RSACC + 4 J
SEL = 192
T0 = 196          # t0..t15
O0 = 212          # o0..o3: copy offsets of a special step
X0 = 216          # x0..x4
NB, NBR = 196, 200  # plain steps: exponent offsets (left / current), right
QOP = 0           # a[16 J + 4 s]
KOP = 64
VOP = 80
S_J, S_NU, S_JUMP, S_RING, S_SCALE, S_T = 64, 65, 66, 67, 68, 69
S_GK, S_GV, S_DSTEP, S_DJUMP, S_D = 70, 72, 74, 76, 78   # pairs
S_GEN, S_MSK, S_NEEDY, S_DU, S_LIM, S_72 = 80, 81, 82, 83, 87, 88   # S_DU: four
S_TMP = 89        # s89..s95
QR_BLOCK = 32 * 76 * 4   # bytes between the q.rel rows of query blocks J and J + 1
VGPR_CLOBBERS = [f"v{r}" for r in range(T0, X0 + 5)]
SGPR_CLOBBERS = ["s69", "s78", "s79"] + [f"s{r}" for r in range(80, 96)]


def oacc(J, db):
    return 32 * J + 16 * db


def pk(bf, hh):
    return PK + 8 * bf + 4 * hh


def t(i):
    return f"v{T0 + i}"


def x(i):
    return f"v{X0 + i}"


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


def skeleton(J, sl, special):
    """The MFMAs of phase J with the memory operations attached before (pre)
    or after (post) them, for a step whose K/V ring slot is sl."""
    bf = J & 1
    jm2, jm1, jp1 = (J + 2) & 3, (J + 3) & 3, (J + 1) & 3
    sn = SACC[bf ^ 1]
    rs = RSACC + 4 * jm1
    mf = [mfma16(rs, ("v", SEL), ("v", pk(bf ^ 1, 0)), f"R1.{J}"),
          mfma16(rs, ("v", SEL), ("v", pk(bf ^ 1, 1)), f"R2.{J}")]
    for k in range(4):
        mf.append(mfma32(sn, ("a", KOP + 4 * k), ("a", QOP + 16 * jp1 + 4 * k), None if k == 0 else sn, f"Q{k}.{J}"))
    for hh in range(2):
        for db in range(2):
            o = oacc(jm2, db)
            mf.append(mfma32(o, ("a", VOP + 8 * hh + 4 * db), ("v", pk(bf, hh)), o, f"P{hh}{db}.{J}"))
    pre = {m.tag: [] for m in mf}
    post = {m.tag: [] for m in mf}

    def dma(which, slot):
        lds = (0 if which == "k" else 8192) + 4096 * slot[1]
        base = S_GK if which == "k" else S_GV
        ops = [Ins(f"s_add_u32 m0, s{S_RING}, {lds}", "m0", writes={"m0"}), nop(0)]
        for i in range(4):
            off = f" offset:{1024 * i}" if i else ""
            voff = f"v{O0 + i}" if special else f"%[ko{i}]"
            ops.append(Ins(f"global_load_lds_dwordx4 {voff}, s[{base}:{base + 1}]{off}", "dma",
                           reads={"m0"} | ({voff} if special else set()), lds_slot=slot))
        return ops

    if J == 0:  # K(j + 2) into the K slot of step j (its operand reads ended in phase 3)
        post[f"Q0.{J}"] += dma("k", ("K", sl))
    if J == 1:  # V(j) has landed: its transpose reads, after the last PV reading the old operands
        post[f"P11.{J}"].append(Ins("s_waitcnt vmcnt(12)", "waitcnt"))
        for hh in range(2):
            for db in range(2):
                v = VOP + 8 * hh + 4 * db
                off = 8192 + 4096 * sl + 2048 * hh
                for hf in range(2):
                    post[f"P11.{J}"].append(Ins(f"ds_read_b64_tr_b16 a[{v + 2 * hf}:{v + 2 * hf + 1}], %[tv{hf}{db}] "
                                                f"offset:{off}", "lds", writes=aregs(v + 2 * hf, 2),
                                                lds_slot=("V", sl)))
    if J == 2:
        # the V(j) operand reads are done (and the PV below needs them):
        # refill the V slot with V(j + 2); K(j + 1) has landed: its operand
        # reads, after the last score product reading K(j)
        pre[f"P00.{J}"].append(Ins("s_waitcnt lgkmcnt(0)", "waitcnt"))
        pre[f"P00.{J}"] += dma("v", ("V", sl))
        pre[f"P00.{J}"].append(Ins("s_waitcnt vmcnt(12)", "waitcnt"))
        for k in range(4):
            pre[f"P00.{J}"].append(Ins(f"ds_read_b128 a[{KOP + 4 * k}:{KOP + 4 * k + 3}], %[ka{k}] "
                                       f"offset:{4096 * (sl ^ 1)}", "lds", writes=aregs(KOP + 4 * k, 4),
                                       lds_slot=("K", sl ^ 1)))
    if J == 3:  # the K(j + 1) operands
        pre[f"Q0.{J}"].append(Ins("s_waitcnt lgkmcnt(0)", "waitcnt"))
    return mf, pre, post


def plain_valu(J):
    """Softmax of a plain item in place: p = exp2(s * scale + nb) -> fp16."""
    bf = J & 1
    s = SACC[bf]
    out = []
    for g in range(4):
        for i in range(4 * g, 4 * g + 4):
            out.append(valu(f"v_fma_f32 v{s + i}, v{s + i}, s{S_SCALE}, v{NB + J}", {f"v{s + i}", f"v{NB + J}"},
                            {f"v{s + i}"}, f"F{i}.{J}"))
        for i in range(4 * g, 4 * g + 4):
            e = valu(f"v_exp_f32 v{s + i}, v{s + i}", {f"v{s + i}"}, {f"v{s + i}"}, f"E{i}.{J}", "trans")
            e.deps = [f"F{i}.{J}"]
            out.append(e)
        for k in (2 * g, 2 * g + 1):
            hh, r = k >> 2, k & 3
            c = valu(f"v_cvt_pk_f16_f32 v{pk(bf, hh) + r}, v{s + 2 * k}, v{s + 2 * k + 1}",
                     {f"v{s + 2 * k}", f"v{s + 2 * k + 1}"}, {f"v{pk(bf, hh) + r}"}, f"C{k}.{J}")
            # the PV products of this phase read the old probabilities
            c.deps = [f"E{2 * k}.{J}", f"E{2 * k + 1}.{J}", f"P{hh}0.{J}", f"P{hh}1.{J}"]
            out.append(c)
    return out


def key_col(i):
    """Key of score element i within the lane's 32-key step, less 8 g."""
    return 16 * (i >> 3) + (i & 7)


def gather_valu(J):
    """Special step, beside the MFMAs: the q.rel bias of every score of item
    (j, J), t_i = qr[query][clamp(key - query + 64, 0, 72)], read from the
    LDS table (rows of block J at qbase + QR_BLOCK J)."""
    out = [valu(f"v_add_u32_e32 {x(0)}, s{S_DU + J}, %[laned]", (), {x(0)}, f"D.{J}")]
    for i in range(16):
        a = valu(f"v_add_u32_e32 {t(i)}, {key_col(i)}, {x(0)}", {x(0)}, {t(i)}, f"A{i}.{J}")
        a.deps = [f"D.{J}"]
        m = valu(f"v_med3_i32 {t(i)}, {t(i)}, 0, s{S_72}", {t(i)}, {t(i)}, f"M{i}.{J}")
        m.deps = [a.tag]
        sh = valu(f"v_lshl_add_u32 {t(i)}, {t(i)}, 2, %[qbase]", {t(i)}, {t(i)}, f"S{i}.{J}")
        sh.deps = [m.tag]
        rd = Ins(f"ds_read_b32 {t(i)}, {t(i)} offset:{QR_BLOCK * J}", "lds", reads={t(i)}, writes={t(i)},
                 tag=f"G{i}.{J}")
        rd.deps = [sh.tag]
        out += [a, m, sh, rd]
    return out


def special_softmax(J, sl):
    """Softmax of item (j, J) of a special step, after its bias gather, as
    the general code forms it: y = s * scale + bias (masked keys -inf); at
    the first step the running max from y (and the running sums scaled by
    exp2(m_old - m_new)); then p = exp2(y - m) for band or masked items,
    exp2(s * scale + (bias - m)) for plain ones.  Returns (text, path) where
    path(needy, msk, first, gen) is the instruction sequence that runs."""
    bf = J & 1
    s = SACC[bf]
    m = f"%[m{J}]"
    lab = {n: f"L_{n}{sl}{J}_%=" for n in ("noy", "nomask", "plain", "cvt")}
    head = [Ins("s_waitcnt lgkmcnt(0)", "waitcnt"),
            valu(f"v_mov_b32_e32 {x(1)}, {t(0)}", {t(0)}, {x(1)}),   # the bias of a plain item (all equal)
            salu(f"s_bitcmp1_b32 s{S_NEEDY}, {J}"), branch(f"s_cbranch_scc0 {lab['noy']}")]
    ys = [valu(f"v_fma_f32 {t(i)}, v{s + i}, s{S_SCALE}, {t(i)}", {f"v{s + i}", t(i)}, {t(i)}) for i in range(16)]
    chk_m = [salu(f"s_bitcmp1_b32 s{S_MSK}, {J}"), branch(f"s_cbranch_scc0 {lab['nomask']}")]
    # (-inf from a register: v_cndmask_b32 reads VCC over the constant bus)
    mask = [valu(f"v_sub_u32_e32 {x(0)}, s{S_LIM}, %[g8]", (), {x(0)}),
            valu(f"v_mov_b32_e32 {x(3)}, 0xff800000", (), {x(3)})]
    for i in range(16):
        mask.append(valu(f"v_cmp_lt_i32_e32 vcc, {key_col(i)}, {x(0)}", {x(0)}, {"vcc"}))
        mask.append(valu(f"v_cndmask_b32_e32 {t(i)}, {x(3)}, {t(i)}, vcc", {t(i), x(3), "vcc"}, {t(i)}))
    chk_f = [salu(f"s_cmp_lg_u32 s{S_J}, 0"), branch(f"s_cbranch_scc1 {lab['noy']}")]
    first = [valu(f"v_max3_f32 {x(0)}, {t(0)}, {t(1)}, {t(2)}", {t(0), t(1), t(2)}, {x(0)})]
    for i in range(3, 15, 2):
        first.append(valu(f"v_max3_f32 {x(0)}, {x(0)}, {t(i)}, {t(i + 1)}", {x(0), t(i), t(i + 1)}, {x(0)}))
    first.append(valu(f"v_max_f32_e32 {x(0)}, {x(0)}, {t(15)}", {x(0), t(15)}, {x(0)}))
    first += [valu(f"v_mov_b32_e32 {x(3)}, {x(0)}", {x(0)}, {x(3)}),
              valu(f"v_mov_b32_e32 {x(4)}, {x(0)}", {x(0)}, {x(4)}),
              Ins(f"v_permlane32_swap_b32_e32 {x(3)}, {x(4)}", "permlane", reads={x(3), x(4)},
                  writes={x(3), x(4)}),
              valu(f"v_max3_f32 {x(0)}, {m}, {x(3)}, {x(4)}", {x(3), x(4)}, {x(0)}),      # m_new
              valu(f"v_sub_f32_e32 {x(2)}, {m}, {x(0)}", {x(0)}, {x(2)}),
              valu(f"v_exp_f32_e32 {x(2)}, {x(2)}", {x(2)}, {x(2)}, kind="trans")]           # alpha
    rsum = RSACC + 4 * J
    first += [valu(f"v_mul_f32_e32 v{rsum + k}, v{rsum + k}, {x(2)}", {f"v{rsum + k}", x(2)}, {f"v{rsum + k}"})
              for k in range(4)]
    first.append(valu(f"v_mov_b32_e32 {m}, {x(0)}", {x(0)}, ()))
    chk_g = [salu(f"s_bitcmp1_b32 s{S_GEN}, {J}"), branch(f"s_cbranch_scc0 {lab['plain']}")]
    gen = []
    for i in range(0, 16, 2):
        gen += [valu(f"v_sub_f32_e32 {t(i)}, {t(i)}, {m}", {t(i)}, {t(i)}),
                valu(f"v_sub_f32_e32 {t(i + 1)}, {t(i + 1)}, {m}", {t(i + 1)}, {t(i + 1)}),
                valu(f"v_exp_f32_e32 {t(i)}, {t(i)}", {t(i)}, {t(i)}, kind="trans"),
                valu(f"v_exp_f32_e32 {t(i + 1)}, {t(i + 1)}", {t(i + 1)}, {t(i + 1)}, kind="trans")]
    gen.append(branch(f"s_branch {lab['cvt']}"))
    plain = [valu(f"v_sub_f32_e32 {x(2)}, {x(1)}, {m}", {x(1)}, {x(2)})]
    for i in range(0, 16, 2):
        plain += [valu(f"v_fma_f32 {t(i)}, v{s + i}, s{S_SCALE}, {x(2)}", {f"v{s + i}", x(2)}, {t(i)}),
                  valu(f"v_fma_f32 {t(i + 1)}, v{s + i + 1}, s{S_SCALE}, {x(2)}", {f"v{s + i + 1}", x(2)},
                       {t(i + 1)}),
                  valu(f"v_exp_f32_e32 {t(i)}, {t(i)}", {t(i)}, {t(i)}, kind="trans"),
                  valu(f"v_exp_f32_e32 {t(i + 1)}, {t(i + 1)}", {t(i + 1)}, {t(i + 1)}, kind="trans")]
    cvt = [nop(0)]
    for k in range(8):
        hh, r = k >> 2, k & 3
        cvt.append(valu(f"v_cvt_pk_f16_f32 v{pk(bf, hh) + r}, {t(2 * k)}, {t(2 * k + 1)}", {t(2 * k), t(2 * k + 1)},
                        {f"v{pk(bf, hh) + r}"}))
    cvt.append(nop(1))   # the next phase's MFMAs read these probabilities
    for seq in (first, gen, plain, mask):   # keep the hazard rules satisfied inside each block
        _pad(seq)
    text = (head + ys + chk_m + mask + [label(lab["nomask"])] + chk_f + first + [label(lab["noy"])] + chk_g + gen
            + [label(lab["plain"])] + plain + [label(lab["cvt"])] + cvt)

    def path(needy, msk, first_step, general):
        seq = list(head)
        if needy:
            seq += ys + chk_m + (mask if msk else []) + [label(lab["nomask"])] + chk_f + (first if first_step else [])
        seq += [label(lab["noy"])] + chk_g
        seq += (gen if general else [label(lab["plain"])] + plain) + [label(lab["cvt"])] + cvt
        return seq
    return text, path


def special_paths():
    """(needy, masked, first, general) of every item kind: needy = general or
    first; masked implies general."""
    out = []
    for needy, msk, first, gen in itertools.product((0, 1), repeat=4):
        if needy != (gen or first) or (msk and not gen):
            continue
        out.append((needy, msk, first, gen))
    return out


def _pad(seq):
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


def check_waits(seq, vm_outstanding):
    """Outstanding-operation check: an LDS read result is used only after an
    lgkmcnt wait retired it, a ring slot is read only after the vmcnt wait
    that retires its copy, and a slot is refilled only after the reads of its
    previous contents retired.  vm_outstanding: slots of the copies in flight
    at the start (oldest first, 4 instructions each)."""
    lgkm = []   # (regs, slot) of LDS reads in flight
    vm = []     # slot per copy instruction in flight
    for slot in vm_outstanding:
        vm += [slot] * 4
    for c in seq:
        if c.kind == "waitcnt":
            kind, n = c.text.split()[1].split("(")
            n = int(n.rstrip(")"))
            if kind == "lgkmcnt":
                lgkm = lgkm[len(lgkm) - n:] if n else []
            else:
                vm = vm[len(vm) - n:] if n else []
            continue
        for regs, _ in lgkm:
            if regs & (c.reads | c.srcc | c.writes):
                raise AssertionError(f"register of an LDS load in flight touched: {c.text}")
        if c.kind == "lds":
            if c.lds_slot is not None and c.lds_slot in vm:
                raise AssertionError(f"LDS read of a slot whose copy is in flight: {c.text}")
            lgkm.append((c.writes, c.lds_slot))
        if c.kind == "dma":
            if any(slot == c.lds_slot for _, slot in lgkm):
                raise AssertionError(f"slot refilled while reads of it are in flight: {c.text}")
            vm.append(c.lds_slot)
    return vm


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


def plain_step(sl, history):
    seq, total = [], 0.0
    for J in range(4):
        mf, pre, post = skeleton(J, sl, special=False)
        ph, cyc = schedule(mf, pre, post, plain_valu(J), history + seq)
        seq += ph
        total += cyc
    return seq, total


def special_step(sl, history):
    """(text, phases): phases[J] = (part A instructions, path function)."""
    text, phases = [], []
    for J in range(4):
        mf, pre, post = skeleton(J, sl, special=True)
        # worst case before part A: a softmax path of the previous phase
        part_a, _ = schedule(mf, pre, post, gather_valu(J), history)
        sm_text, sm_path = special_softmax(J, sl)
        text += part_a + sm_text
        phases.append((part_a, sm_path))
        history = part_a + sm_path(1, 1, 1, 1)
    return text, phases


def u_of(xreg, dst):
    """SALU: local step of processing index xreg into dst (s89, s90 scratch)."""
    a, b = f"s{S_TMP}", f"s{S_TMP + 1}"
    return [salu(f"s_sub_i32 {a}, {xreg}, %[ns]"),
            salu(f"s_cmp_ge_i32 {a}, %[cl]"),
            salu(f"s_cselect_b32 {b}, %[nband], 0"),
            salu(f"s_add_i32 {a}, {a}, {b}"),                 # plain steps
            salu(f"s_cmp_lt_i32 {xreg}, %[ns]"),
            salu(f"s_cselect_b32 {a}, %[ue], {a}"),            # the straddling step
            salu(f"s_add_i32 {b}, %[cl], {xreg}"),
            salu(f"s_cmp_lt_i32 {xreg}, %[nband]"),
            salu(f"s_cselect_b32 {dst}, {b}, {a}")]            # band steps


def copy_bases(special):
    """SALU: copy bases of step min(j + 2, nu - 1) into s[70:73]; special
    steps also select the tile offsets (the last, ragged step re-reads row
    LK - 1 for its rows past LK)."""
    xr, u, tmp = f"s{S_TMP + 2}", f"s{S_TMP + 3}", f"s{S_TMP + 4}"
    out = [salu(f"s_add_i32 {xr}, s{S_J}, 2"), salu(f"s_sub_i32 {tmp}, s{S_NU}, 1"), salu(f"s_min_i32 {xr}, {xr}, {tmp}")]
    out += u_of(xr, u)
    out.append(salu(f"s_lshl2_add_u32 {u}, {u}, %[w]"))      # global step t = w + 4 u
    if special:
        out += [salu(f"s_cmp_eq_u32 {u}, %[tlast]"), salu(f"s_cselect_b64 s[{S_D}:{S_D + 1}], -1, 0")]
    a, b = f"s{S_TMP}", f"s{S_TMP + 1}"
    out += [salu(f"s_mul_i32 {a}, {u}, %[rowb]"), salu(f"s_mul_hi_u32 {b}, {u}, %[rowb]"),
            salu(f"s_add_u32 s{S_GK}, %[kblo], {a}"), salu(f"s_addc_u32 s{S_GK + 1}, %[kbhi], {b}"),
            salu(f"s_add_u32 s{S_GV}, %[vblo], {a}"), salu(f"s_addc_u32 s{S_GV + 1}, %[vbhi], {b}")]
    if special:
        out += [valu(f"v_cndmask_b32_e64 v{O0 + i}, %[ko{i}], %[kl{i}], s[{S_D}:{S_D + 1}]", (), {f"v{O0 + i}"})
                for i in range(4)]
    return out


def special_preamble():
    """SALU per special step: item kinds of the four blocks and the bias /
    mask offsets, then the copy bases."""
    u, k0, a, b = f"s{S_TMP + 3}", f"s{S_TMP + 4}", f"s{S_TMP + 5}", f"s{S_TMP + 6}"
    out = u_of(f"s{S_J}", u)
    out += [salu(f"s_lshl2_add_u32 {k0}, {u}, %[w]"), salu(f"s_lshl_b32 {k0}, {k0}, 5"),   # first key k0
            salu(f"s_add_i32 {a}, {k0}, 32"), salu(f"s_cmp_gt_i32 {a}, %[lk]"),
            salu(f"s_cselect_b32 s{S_MSK}, 15, 0"),                                            # straddles LK
            salu(f"s_mov_b32 s{S_GEN}, s{S_MSK}")]
    for J in range(4):
        # band: neither entirely left (k0 + 31 - qlo <= -64) nor entirely
        # right (k0 - (qlo + 31) >= 8) of the window, qlo = q0 + 32 J
        out += [salu(f"s_add_i32 {a}, {k0}, {95 - 32 * J}"), salu(f"s_cmp_gt_i32 {a}, %[q0]"),
                salu(f"s_cselect_b32 {a}, {1 << J}, 0"),
                salu(f"s_add_i32 {b}, {k0}, {-39 - 32 * J}"), salu(f"s_cmp_lt_i32 {b}, %[q0]"),
                salu(f"s_cselect_b32 {b}, {1 << J}, 0"),
                salu(f"s_and_b32 {a}, {a}, {b}"), salu(f"s_or_b32 s{S_GEN}, s{S_GEN}, {a}")]
    out += [salu(f"s_cmp_eq_u32 s{S_J}, 0"), salu(f"s_cselect_b32 s{S_NEEDY}, 15, 0"),
            salu(f"s_or_b32 s{S_NEEDY}, s{S_NEEDY}, s{S_GEN}"),
            # bias index offset of block J: k0 - (q0 + 32 J) + 64 (+ 8 g - n per lane)
            salu(f"s_sub_i32 s{S_DU}, {k0}, %[q0]"), salu(f"s_add_i32 s{S_DU}, s{S_DU}, 64")]
    out += [salu(f"s_sub_i32 s{S_DU + J}, s{S_DU}, {32 * J}") for J in range(1, 4)]
    out.append(salu(f"s_sub_i32 s{S_LIM}, %[lk], {k0}"))                                       # LK - k0
    return out + copy_bases(special=True)


def advance():
    """After a plain step of index j: j += 1; the copy bases move to step
    j + 2 (by 4 key steps, across the band at index jump, not past nu - 1)."""
    return [salu(f"s_add_u32 s{S_J}, s{S_J}, 1"),
            salu(f"s_add_u32 s{S_T}, s{S_J}, 2"),
            salu(f"s_cmp_eq_u32 s{S_T}, s{S_JUMP}"),
            salu(f"s_cselect_b64 s[{S_D}:{S_D + 1}], s[{S_DJUMP}:{S_DJUMP + 1}], s[{S_DSTEP}:{S_DSTEP + 1}]"),
            salu(f"s_cmp_lt_i32 s{S_T}, s{S_NU}"),
            salu(f"s_cselect_b64 s[{S_D}:{S_D + 1}], s[{S_D}:{S_D + 1}], 0"),
            salu(f"s_add_u32 s{S_GK}, s{S_GK}, s{S_D}"),
            salu(f"s_addc_u32 s{S_GK + 1}, s{S_GK + 1}, s{S_D + 1}"),
            salu(f"s_add_u32 s{S_GV}, s{S_GV}, s{S_D}"),
            salu(f"s_addc_u32 s{S_GV + 1}, s{S_GV + 1}, s{S_D + 1}"),
            salu(f"s_cmp_eq_u32 s{S_J}, s{S_JUMP}")]


def switch(tag):
    """From index jump on the plain steps lie right of the window: their
    exponent offsets (taken when the preceding compare held)."""
    return ([branch(f"s_cbranch_scc0 L_left{tag}_%=")]
            + [valu(f"v_mov_b32_e32 v{NB + J}, v{NBR + J}", {f"v{NBR + J}"}, {f"v{NB + J}"}) for J in range(4)]
            + [label(f"L_left{tag}_%=")])


def plain_entry():
    """Before the first plain step: copy bases, and the exponent offsets
    qr_l - m, qr_r - m of the four blocks (as the general code forms them)."""
    out = [salu(f"s_cmp_ge_i32 s{S_J}, s{S_NU}"), branch("s_cbranch_scc1 L_end_%=")]
    out += copy_bases(special=False)
    for J in range(4):
        out += [Ins(f"ds_read_b32 v{NB + J}, %[qbase] offset:{QR_BLOCK * J}", "lds", writes={f"v{NB + J}"}),
                Ins(f"ds_read_b32 v{NBR + J}, %[qbase] offset:{QR_BLOCK * J + 72 * 4}", "lds",
                    writes={f"v{NBR + J}"})]
    out.append(Ins("s_waitcnt lgkmcnt(0)", "waitcnt"))
    for J in range(4):
        out += [valu(f"v_sub_f32_e32 v{NB + J}, v{NB + J}, %[m{J}]", {f"v{NB + J}"}, {f"v{NB + J}"}),
                valu(f"v_sub_f32_e32 v{NBR + J}, v{NBR + J}, %[m{J}]", {f"v{NBR + J}"}, {f"v{NBR + J}"})]
    out += [salu(f"s_cmp_lt_i32 s{S_J}, s{S_JUMP}"), branch("s_cbranch_scc1 L_isleft_%=")]
    out += [valu(f"v_mov_b32_e32 v{NB + J}, v{NBR + J}", {f"v{NBR + J}"}, {f"v{NB + J}"}) for J in range(4)]
    out.append(label("L_isleft_%="))
    return out


FENCE = [nop(7), nop(7), nop(7)]


def build():
    # plain steps alternate slots 0, 1, 0, ...: schedule each against the
    # other's tail until both are stable
    s0, _ = plain_step(0, FENCE)
    s1, _ = plain_step(1, s0)
    for _ in range(4):
        n0, c0 = plain_step(0, s1)
        n1, c1 = plain_step(1, n0)
        stable = [i.text for i in n0] == [i.text for i in s0] and [i.text for i in n1] == [i.text for i in s1]
        s0, s1 = n0, n1
        if stable:
            break
    pre = special_preamble()
    sp_hist = FENCE + pre
    sp_text, sp_phases = {}, {}
    for sl in (0, 1):
        sp_text[sl], sp_phases[sl] = special_step(sl, sp_hist)
    # the last block's row sums; then every LDS read has retired: the
    # statement's register outputs (the V^T and K operands among them) are
    # final when it ends (the compiler may move register-only work after it,
    # such as the last PV products, above a wait in the compiled code)
    tail = [mfma16(RSACC + 12, ("v", SEL), ("v", pk(1, 0)), "R1.end"),
            mfma16(RSACC + 12, ("v", SEL), ("v", pk(1, 1)), "R2.end"), Ins("s_waitcnt lgkmcnt(0)", "waitcnt")]
    entry = FENCE + [salu(f"s_movk_i32 s{S_72}, 0x48"), label("L_sp_top_%="),
                     salu(f"s_cmp_ge_i32 s{S_J}, %[nslow]"), branch("s_cbranch_scc1 L_plain_entry_%=")]
    sp_loop = (pre + [salu(f"s_bitcmp1_b32 s{S_J}, 0"), branch("s_cbranch_scc1 L_sp_odd_%=")] + sp_text[0]
               + [salu(f"s_add_u32 s{S_J}, s{S_J}, 1"), branch("s_branch L_sp_top_%="), label("L_sp_odd_%=")]
               + sp_text[1] + [salu(f"s_add_u32 s{S_J}, s{S_J}, 1"), branch("s_branch L_sp_top_%=")])
    p_entry = [label("L_plain_entry_%=")] + plain_entry() + [salu(f"s_bitcmp1_b32 s{S_J}, 0"),
                                                             branch("s_cbranch_scc1 L_odd_%="), label("L_even_%=")]
    even = s0 + advance() + switch(0) + [salu(f"s_cmp_ge_i32 s{S_J}, s{S_NU}"),
                                         branch("s_cbranch_scc1 L_end_%="), label("L_odd_%=")]
    odd = s1 + advance() + switch(1) + [salu(f"s_cmp_lt_i32 s{S_J}, s{S_NU}"),
                                        branch("s_cbranch_scc1 L_even_%="), label("L_end_%=")]
    loop = entry + sp_loop + p_entry + even + odd + tail + FENCE

    # -- hazard checks over every order the loop can run --
    e0, e1 = s0 + advance(), s1 + advance()
    pe = plain_entry()
    for seq in (FENCE + e0 + e1 + e0 + tail + FENCE, FENCE + e1 + e0 + e1 + tail + FENCE,
                FENCE + e0 + tail + FENCE, FENCE + e1 + tail + FENCE, FENCE + pe + e0 + tail, FENCE + pe + e1 + tail):
        check_hazards(seq)
    paths = special_paths()
    for sl in (0, 1):
        phases = sp_phases[sl]
        # each phase after every softmax path of the phase before (or the
        # preamble), followed by every path and the start of the next phase
        for J in range(4):
            a_j, path_j = phases[J]
            befores = [FENCE + pre] if J == 0 else [phases[J - 1][0] + phases[J - 1][1](*p) for p in paths]
            if J == 0:   # also after the previous special step's last phase
                a3, path3 = sp_phases[sl ^ 1][3]
                befores += [a3 + path3(*p) + [salu("s_add_u32"), branch("s_branch")] + pre for p in paths]
            afters = ([phases[J + 1][0][:40]] if J < 3 else
                      [pre + sp_phases[sl ^ 1][0][0][:40], pe + s0[:40], pe + s1[:40], tail + FENCE])
            for before in befores:
                for p in paths:
                    for after in afters:
                        check_hazards(before[-40:] + a_j + path_j(*p) + after)
    # -- outstanding loads: special steps, then plain ones, in both parities --
    for first in (0, 1):
        seq = []
        for sl in (first, first ^ 1):
            for J in range(4):
                a_j, path_j = sp_phases[sl][J]
                seq += a_j + path_j(1, 1, 1, 1)
        seq += pe + (s0 + s1 if first == 0 else s1 + s0)
        vm = check_waits(seq, [("K", first), ("V", first), ("K", first ^ 1), ("V", first ^ 1)])
        assert len(vm) <= 12, vm
    # every exit leaves no LDS read in flight (the copies still in flight
    # write only LDS, which the compiled code awaits before reusing it)
    for seq in (pe + tail, pe + e0 + tail, pe + e1 + tail, pe + e0 + e1 + tail):
        assert_quiet(seq, copies=False)
    return loop, s0, c0


def render(seq):
    return " \\\n".join(f'  "{i.text}\\n\\t"' for i in seq)


def main():
    loop, s0, c0 = build()
    counts = {}
    for i in s0:
        counts[i.kind] = counts.get(i.kind, 0) + 1
    text = [
        "// flexrel_wide_step.inc -- generated by gen_wide_step.py (run by build.py); do not edit.",
        "// The key-step loop of flexrel_wide.hip.  One plain step: " + ", ".join(
            f"{v} {k}" for k, v in sorted(counts.items())) + f" instructions; modelled issue time {c0:.0f} cycles.",
        "#pragma once",
        "",
        "#define SIDON_WIDE_VGPR_CLOBBERS " + ", ".join(f'"{r}"' for r in VGPR_CLOBBERS),
        "#define SIDON_WIDE_SGPR_CLOBBERS " + ", ".join(f'"{r}"' for r in SGPR_CLOBBERS),
        "",
        "#define SIDON_WIDE_LOOP \\",
        render(loop),
        "",
    ]
    OUT.write_text("\n".join(text))
    print(f"wrote {OUT} ({len(loop)} instructions; one plain step {len(s0)}, modelled {c0:.0f} cycles)",
          file=sys.stderr)


if __name__ == "__main__":
    main()
