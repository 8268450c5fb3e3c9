"""Generates flexrel_w64_step.inc: the key-step loop of flexrel_w64.hip (64
query rows per workgroup, two 32-row blocks per wavefront, two workgroups
per compute unit) as hand-scheduled gfx950 assembly.

Run by build.py before every compile (the instruction record, issue model,
list scheduler and wait-state rules are gen_asm.py's).  The loop runs a
wavefront's key steps in the kernel's processing order: the special steps
first (band steps, where a block needs the per-score q.rel gather; the step
straddling LK; the first step, which sets the running max exactly), then the
plain steps (every block entirely left or entirely right of the window).
Every item computes exactly what the general code of flexrel_w64.hip
computes for it -- the same MFMAs on the same operands, the same fma / exp2 /
fp16 rounding per score, the same row-sum accumulation -- so the C++ rerun
(taken when a probability leaves the fp16 range) reproduces every query that
did not overflow bit for bit.

* two phases per key step (blocks 0 and 1); phase J of step j runs the PV
  of item (j - 1, J), the softmax of item (j, J), the row sums of the
  previous item and the score product of the next one;
* a phase of a special step branches on the step's flags to one of six
  scheduled blocks, one per path of its item (PATHS), each interleaving the
  path's bias gather and softmax with the phase's products;
* K tiles pass through one LDS slot per wavefront into two register
  buffers: in phase 0 of step j, after the score product of item (j, 1)
  read K(j), K(j + 2) is read from the slot into that buffer, and then
  K(j + 3) is copied into the slot; V tiles use a two-slot ring (V(j + 1) is
  copied in phase 0 of step j, V(j) read transposed in phase 1), so three
  4 KB tiles per wavefront and two workgroups fit on a compute unit;
* registers (per wavefront, at most 256 with two wavefronts per SIMD; all
  of them VGPRs: a kernel that names AGPRs gets at most half of its 256 as
  VGPRs):

  v[0:63]     O^T accumulators: block J, dims half db at v[32 J + 16 db]
  v[64:79]    scores buffer 0, v[80:95] buffer 1
  v[96:111]   fp16 probabilities [buffer][16-key half], 4 VGPRs each
  v[112:119]  running row sums, block J at v[112 + 4 J]
  v[120:123]  the 0/1 selector operand of the row-sum MFMA
  v[124:149]  scratch (special steps: biases / scores t0-t15, V copy
              offsets, temporaries, the K load offset; plain steps:
              exponent offsets in v[124:127])
  v[152:183]  Q^T operands: block J, k-step s at v[152 + 16 J + 4 s]
  v[184:215]  K operands, buffer b, k-step s at v[184 + 16 b + 4 s]
  v[216:231]  V^T operands [hh][db] at v[216 + 8 hh + 4 db]
  s64 step index j, s65 nu, s66 jump, s67 V ring LDS address, s68 scale,
  s[70:71] K load base (step j + 2), s[72:73] V copy base (step j + 1),
  s[74:77] advances, s69 and s[78:95] scratch
"""

from __future__ import annotations

import itertools
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parent))
import gen_asm as G  # noqa: E402
from gen_asm import (Ins, assert_quiet, branch, check_hazards, label, mfma16, mfma32, nop,  # noqa: E402
                           salu, schedule, valu)

OUT = Path(__file__).resolve().parent / "flexrel_w64_step.inc"

NBLK = 2
SACC = (64, 80)
SEL = 120
T0, O0, X0 = 124, 140, 144
V_SLOT, K_SLOT = 16384, 32768   # LDS offsets of V slot 1 and of the K slot from the ring base
NB, NBR = 124, 126
S_J, S_NU, S_JUMP, S_RING, S_SCALE, S_T = 64, 65, 66, 67, 68, 69
S_GK, S_GV, S_DSTEP, S_DJUMP, S_D = 70, 72, 74, 76, 78
S_GEN, S_MSK, S_NEEDY, S_DU, S_LIM = 80, 81, 82, 83, 85   # S_DU: two
S_TMP = 87        # s87..s95
QR_ROW = 92 * 4      # bytes per q.rel row: 8 floats of padding (position 0), 73 positions, padding (72)
QR_BLOCK = 32 * QR_ROW
VGPR_CLOBBERS = [f"v{r}" for r in range(T0, X0 + 5)]
SGPR_CLOBBERS = ["s69", "s78", "s79"] + [f"s{r}" for r in range(80, 96)]


def oacc(J, db):
    return 32 * J + 16 * db


def pk(bf, hh):
    return 96 + 8 * bf + 4 * hh


def rs(J):
    return 112 + 4 * J


def qop(J, s):
    return 152 + 16 * J + 4 * s


def kop(b, s):
    return 184 + 16 * b + 4 * s


def vop(hh, db):
    return 216 + 8 * hh + 4 * db


def t(i):
    return f"v{T0 + i}"


def x(i):
    return f"v{X0 + i}"


def skeleton(J, sl, special):
    """MFMAs of phase J (step with ring / K buffer parity sl) with their
    memory operations."""
    bf = J
    jm1 = J ^ 1
    sn = SACC[bf ^ 1]
    kb = sl if J == 0 else sl ^ 1          # phase 0: K(j) (item (j, 1)); phase 1: K(j + 1) (item (j + 1, 0))
    rsum = [mfma16(rs(jm1), ("v", SEL), ("v", pk(bf ^ 1, 0)), f"R1.{J}"),
            mfma16(rs(jm1), ("v", SEL), ("v", pk(bf ^ 1, 1)), f"R2.{J}")]
    score = [mfma32(sn, ("v", kop(kb, k)), ("v", qop(jm1, k)), None if k == 0 else sn, f"Q{k}.{J}")
             for k in range(4)]
    # phase 0 issues its score product first: the K register buffer it
    # frees is refilled from LDS while the row-sum products run
    mf = score + rsum if J == 0 else rsum + score
    for hh in range(2):
        for db in range(2):
            o = oacc(J, db)
            mf.append(mfma32(o, ("v", vop(hh, db)), ("v", pk(bf, hh)), o, f"P{hh}{db}.{J}"))
    pre = {m.tag: [] for m in mf}
    post = {m.tag: [] for m in mf}
    if J == 0:
        # K(j) was last read by the score product above: K(j + 2), copied
        # into the wavefront's K slot one step ago, into its register buffer
        # (in flight, oldest first: K(j + 2), V(j))
        post["Q3.0"].append(Ins("s_waitcnt vmcnt(4)", "waitcnt"))
        for k in range(4):
            post["Q3.0"].append(Ins(f"ds_read_b128 v[{kop(sl, k)}:{kop(sl, k) + 3}], %[ka{k}] offset:{K_SLOT}",
                                    "lds", writes=G.vregs(kop(sl, k), 4), lds_slot=("K", 0)))
        # those reads and the V(j - 1) operand reads are done (the PV below
        # needs V(j - 1)): copy K(j + 3) into the K slot and V(j + 1) into
        # the slot V(j - 1) held
        pre["P00.0"].append(Ins("s_waitcnt lgkmcnt(0)", "waitcnt"))
        for name, base, slot, lds in (("K", S_GK, ("K", 0), K_SLOT), ("V", S_GV, ("V", sl ^ 1), V_SLOT * (sl ^ 1))):
            pre["P00.0"] += [Ins(f"s_add_u32 m0, s{S_RING}, {lds}", "m0", writes={"m0"}), nop(0)]
            for i in range(4):
                off = f" offset:{1024 * i}" if i else ""
                voff = (f"v{X0 + 1 + i}" if name == "K" else f"v{O0 + i}") if special else f"%[ko{i}]"
                pre["P00.0"].append(Ins(f"global_load_lds_dwordx4 {voff}, s[{base}:{base + 1}]{off}", "dma",
                                        reads={"m0"} | ({voff} if special else set()), lds_slot=slot))
    if J == 1:
        # in flight, oldest first: V(j), K(j + 3), V(j + 1)
        post["P11.1"].append(Ins("s_waitcnt vmcnt(8)", "waitcnt"))   # V(j) landed
        for hh in range(2):  # V(j) operands, after the last PV reading V(j - 1)
            for db in range(2):
                v = vop(hh, db)
                for hf in range(2):
                    post["P11.1"].append(Ins(f"ds_read_b64_tr_b16 v[{v + 2 * hf}:{v + 2 * hf + 1}], %[tv{hf}{db}] "
                                             f"offset:{V_SLOT * sl + 2048 * hh}", "lds",
                                             writes=G.vregs(v + 2 * hf, 2), lds_slot=("V", sl)))
    return mf, pre, post


def plain_valu(J):
    bf = J
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
            c.deps = [f"E{2 * k}.{J}", f"E{2 * k + 1}.{J}", f"P{hh}0.{J}", f"P{hh}1.{J}"]
            out.append(c)
    return out


def key_col(i):
    return 16 * (i >> 3) + (i & 7)


def gather_valu(J):
    """LDS reads of the 16 biases of a band item.  The lane's keys are the
    runs d0 + [0, 8) and d0 + 16 + [0, 8) of positions (d0 = k0 + 8 g -
    (q0 + 32 J + n) + 64), each clamped to [0, 72]; the q.rel row repeats
    position 0 in the 8 floats before it and position 72 in the 8 after it,
    so each run is 8 consecutive floats of the row from its clamped start
    s' = clamp(s, -8, 72) -- formed as clamp(s - 8, -16, 64) (both bounds
    inline constants) -- read by four ds_read2_b32.  Addresses in t7 and t15
    (each the last destination of its run's reads) and x0."""
    d = valu(f"v_add_u32_e32 {x(0)}, s{S_DU + J}, %[laned]", (), {x(0)}, f"D.{J}")
    out = [d]
    adr = []
    for h in range(2):
        r = t(8 * h + 7)
        a = valu(f"v_add_u32_e32 {r}, {16 * h - 8}, {x(0)}", {x(0)}, {r}, f"A{h}.{J}")
        a.deps = [d.tag]
        m = valu(f"v_med3_i32 {r}, {r}, -16, 64", {r}, {r}, f"M{h}.{J}")
        m.deps = [a.tag]
        out += [a, m]
        adr.append(r)
    # the row's position 0 (block J) + 4 x 8: the byte address of s' is base + 4 (s - 8)
    base = valu(f"v_add_u32_e32 {x(0)}, {QR_BLOCK * J + 32}, %[qbase]", (), {x(0)}, f"Q.{J}")
    base.deps = ["A0." + str(J), "A1." + str(J)]
    out.append(base)
    for h in range(2):
        r = adr[h]
        sh = valu(f"v_lshl_add_u32 {r}, {r}, 2, {x(0)}", {r, x(0)}, {r}, f"L{h}.{J}")
        sh.deps = [f"M{h}.{J}", base.tag]
        out.append(sh)
        for k in range(4):
            i = 8 * h + 2 * k
            rd = Ins(f"ds_read2_b32 v[{T0 + i}:{T0 + i + 1}], {r} offset0:{2 * k} offset1:{2 * k + 1}", "lds",
                     reads={r}, writes={t(i), t(i + 1)}, tag=f"G{i}.{J}")
            rd.deps = [sh.tag] + ([f"G{i - 2}.{J}"] if k else [])
            out.append(rd)
    return out


# Special items by path: (needy, masked, first, general).  needy: y = s *
# scale + bias is formed (the first step, band and masked items); masked: keys
# >= LK get y = -inf; first: the running max is set from y (and the running
# sums scaled by exp2(m_old - m_new)); general: p = exp2(y - m), else the plain
# form exp2(s * scale + (bias - m)).  Masked items are general, and an item
# is needy exactly when it is general or in the first step.
PATHS = {"P": (0, 0, 0, 0), "G": (1, 0, 0, 1), "GM": (1, 1, 0, 1),
         "F0": (1, 0, 1, 0), "FG": (1, 0, 1, 1), "FGM": (1, 1, 1, 1)}


def auto_deps(seq):
    """Orders a straight-line list for the list scheduler: each instruction
    depends on every earlier one that writes a register it reads or writes,
    or reads a register it writes."""
    for i, c in enumerate(seq):
        for p in seq[:i]:
            if (p.writes & (c.reads | c.writes)) or (p.reads & c.writes):
                if p.tag not in c.deps:
                    c.deps.append(p.tag)
    return seq


def special_valu(J, path):
    """Vector list of item (j, J) of a special step on one path: the bias
    gather, then the softmax as the general code forms it (see PATHS),
    straight-line, for the list scheduler to interleave with the phase's
    products.  %[m J] (the running max) is tracked as the pseudo-register
    mJ."""
    needy, msk, first_step, general = PATHS[path]
    bf = J
    s = SACC[bf]
    m = f"%[m{J}]"
    mr = f"m{J}"
    tags = iter(range(1000))

    def v(text, reads=(), writes=(), kind="valu"):
        return valu(text, set(reads), set(writes), f"S{next(tags)}.{J}", kind)

    gather = gather_valu(J)
    ts = {t(i) for i in range(16)}
    wait = Ins("s_waitcnt lgkmcnt(0)", "waitcnt", writes=ts, tag=f"W.{J}")   # the gathered biases have landed
    seq = [wait] + ([] if general else [v(f"v_mov_b32_e32 {x(1)}, {t(0)}", {t(0)}, {x(1)})])
    if needy:
        seq += [v(f"v_fma_f32 {t(i)}, v{s + i}, s{S_SCALE}, {t(i)}", {f"v{s + i}", t(i)}, {t(i)}) for i in range(16)]
    if msk:
        seq += [v(f"v_sub_u32_e32 {x(0)}, s{S_LIM}, %[g8]", (), {x(0)}),
                v(f"v_mov_b32_e32 {x(3)}, 0xff800000", (), {x(3)})]
        for i in range(16):
            seq.append(v(f"v_cmp_lt_i32_e32 vcc, {key_col(i)}, {x(0)}", {x(0)}, {"vcc"}))
            seq.append(v(f"v_cndmask_b32_e32 {t(i)}, {x(3)}, {t(i)}, vcc", {t(i), x(3), "vcc"}, {t(i)}))
    if first_step:
        seq.append(v(f"v_max3_f32 {x(0)}, {t(0)}, {t(1)}, {t(2)}", {t(0), t(1), t(2)}, {x(0)}))
        for i in range(3, 15, 2):
            seq.append(v(f"v_max3_f32 {x(0)}, {x(0)}, {t(i)}, {t(i + 1)}", {x(0), t(i), t(i + 1)}, {x(0)}))
        seq += [v(f"v_max_f32_e32 {x(0)}, {x(0)}, {t(15)}", {x(0), t(15)}, {x(0)}),
                v(f"v_mov_b32_e32 {x(3)}, {x(0)}", {x(0)}, {x(3)}),
                v(f"v_mov_b32_e32 {x(4)}, {x(0)}", {x(0)}, {x(4)}),
                v(f"v_permlane32_swap_b32_e32 {x(3)}, {x(4)}", {x(3), x(4)}, {x(3), x(4)}, "permlane"),
                v(f"v_max3_f32 {x(0)}, {m}, {x(3)}, {x(4)}", {x(3), x(4), mr}, {x(0)}),
                v(f"v_sub_f32_e32 {x(2)}, {m}, {x(0)}", {x(0), mr}, {x(2)}),
                v(f"v_exp_f32_e32 {x(2)}, {x(2)}", {x(2)}, {x(2)}, "trans")]
        seq += [v(f"v_mul_f32_e32 v{rs(J) + k}, v{rs(J) + k}, {x(2)}", {f"v{rs(J) + k}", x(2)}, {f"v{rs(J) + k}"})
                for k in range(4)]
        seq.append(v(f"v_mov_b32_e32 {m}, {x(0)}", {x(0)}, {mr}))
    if general:
        for i in range(16):
            seq.append(v(f"v_sub_f32_e32 {t(i)}, {t(i)}, {m}", {t(i), mr}, {t(i)}))
            seq.append(v(f"v_exp_f32_e32 {t(i)}, {t(i)}", {t(i)}, {t(i)}, "trans"))
    else:
        seq.append(v(f"v_sub_f32_e32 {x(2)}, {x(1)}, {m}", {x(1), mr}, {x(2)}))
        for i in range(16):
            seq.append(v(f"v_fma_f32 {t(i)}, v{s + i}, s{S_SCALE}, {x(2)}", {f"v{s + i}", x(2), t(i)}, {t(i)}))
            seq.append(v(f"v_exp_f32_e32 {t(i)}, {t(i)}", {t(i)}, {t(i)}, "trans"))
    for k in range(8):
        hh, r = k >> 2, k & 3
        c = v(f"v_cvt_pk_f16_f32 v{pk(bf, hh) + r}, {t(2 * k)}, {t(2 * k + 1)}", {t(2 * k), t(2 * k + 1)},
              {f"v{pk(bf, hh) + r}"})
        c.deps += [f"P{hh}0.{J}", f"P{hh}1.{J}"]   # after the PV products that read the previous contents
        seq.append(c)
    out = gather + seq
    auto_deps(out)
    return out


def dispatch(sl, J):
    """SALU branches from the step's flags to the scheduled variant of the
    item's path (wave-uniform), as (text, {path: executed prefix})."""
    lab = {pth: f"L_v{sl}{J}{pth}_%=" for pth in PATHS}
    lf = f"L_vf{sl}{J}_%="
    c_needy = [salu(f"s_bitcmp1_b32 s{S_NEEDY}, {J}"), branch(f"s_cbranch_scc0 {lab['P']}")]
    c_first = [salu(f"s_cmp_eq_u32 s{S_J}, 0"), branch(f"s_cbranch_scc1 {lf}")]
    c_msk = [salu(f"s_bitcmp1_b32 s{S_MSK}, {J}"), branch(f"s_cbranch_scc1 {lab['GM']}"),
             branch(f"s_branch {lab['G']}")]
    c_gen = [label(lf), salu(f"s_bitcmp1_b32 s{S_GEN}, {J}"), branch(f"s_cbranch_scc0 {lab['F0']}")]
    c_fmsk = [salu(f"s_bitcmp1_b32 s{S_MSK}, {J}"), branch(f"s_cbranch_scc1 {lab['FGM']}"),
              branch(f"s_branch {lab['FG']}")]
    text = c_needy + c_first + c_msk + c_gen + c_fmsk
    executed = {"P": c_needy, "G": c_needy + c_first + c_msk, "GM": c_needy + c_first + c_msk[:2],
                "F0": c_needy + c_first + c_gen, "FG": c_needy + c_first + c_gen + c_fmsk,
                "FGM": c_needy + c_first + c_gen + c_fmsk[:2]}
    return text, {pth: seq + [label(lab[pth])] for pth, seq in executed.items()}, lab


def plain_step(sl, history):
    seq, total = [], 0.0
    for J in range(NBLK):
        mf, pre, post = skeleton(J, sl, special=False)
        ph, cyc = schedule(mf, pre, post, plain_valu(J), history + seq)
        seq += ph
        total += cyc
    return seq, total


def special_step(sl, history):
    """Both phases of a special step: for each, the dispatch to one scheduled
    block per path (the phase's products interleaved with the gather and the
    path's softmax), each ending at the phase's join.  Returns (text, phases)
    with phases[J] = {path: executed sequence of phase J on that path}."""
    text, phases = [], []
    for J in range(NBLK):
        d_text, d_exec, lab = dispatch(sl, J)
        join = f"L_vj{sl}{J}_%="
        text += d_text
        variants = {}
        for pth in PATHS:
            mf, pre, post = skeleton(J, sl, special=True)
            # the phase's memory operations keep their place before any
            # vector instruction that touches their registers (the K copy
            # offsets in v145-v148 are softmax temporaries)
            ops = [o for mm in mf for o in pre[mm.tag] + post[mm.tag]]
            for i, o in enumerate(ops):
                o.tag = o.tag or f"X{i}.{J}"
            vl = special_valu(J, pth)
            for c in vl:
                for o in ops:
                    if (c.writes & (o.reads | o.writes)) or (c.reads & o.writes):
                        c.deps.append(o.tag)
            block, _ = schedule(mf, pre, post, vl, history)
            block.append(nop(1))   # its last vector writes -> the next phase's first products
            text += [label(lab[pth])] + block + [branch(f"s_branch {join}")]
            variants[pth] = d_exec[pth] + block + [branch(f"s_branch {join}"), label(join)]
        text.append(label(join))
        phases.append(variants)
        history = variants["FGM"]
    return text, phases


def u_of(xreg, dst):
    a, b = f"s{S_TMP}", f"s{S_TMP + 1}"
    return [salu(f"s_sub_i32 {a}, {xreg}, %[ns]"),
            salu(f"s_cmp_ge_i32 {a}, %[cl]"),
            salu(f"s_cselect_b32 {b}, %[nband], 0"),
            salu(f"s_add_i32 {a}, {a}, {b}"),
            salu(f"s_cmp_lt_i32 {xreg}, %[ns]"),
            salu(f"s_cselect_b32 {a}, %[ue], {a}"),
            salu(f"s_add_i32 {b}, %[cl], {xreg}"),
            salu(f"s_cmp_lt_i32 {xreg}, %[nband]"),
            salu(f"s_cselect_b32 {dst}, {b}, {a}")]


def base_of(ahead, dst, special):
    """SALU: copy base of the K (ahead = 3, into s[70:71]) or V (ahead = 1,
    into s[72:73]) tile of step min(j + ahead, nu - 1); special steps also
    select the tile offsets of the last, ragged step (which re-reads row
    LK - 1 for its rows past LK) into v145-148 (K) or v140-143 (V)."""
    xr, u, tmp = f"s{S_TMP + 2}", f"s{S_TMP + 3}", f"s{S_TMP + 4}"
    out = [salu(f"s_add_i32 {xr}, s{S_J}, {ahead}"), salu(f"s_sub_i32 {tmp}, s{S_NU}, 1"),
           salu(f"s_min_i32 {xr}, {xr}, {tmp}")]
    out += u_of(xr, u)
    out.append(salu(f"s_lshl2_add_u32 {u}, {u}, %[w]"))
    if special:
        out += [salu(f"s_cmp_eq_u32 {u}, %[tlast]"), salu(f"s_cselect_b64 s[{S_D}:{S_D + 1}], -1, 0")]
    a, b = f"s{S_TMP}", f"s{S_TMP + 1}"
    which = "k" if ahead == 3 else "v"
    out += [salu(f"s_mul_i32 {a}, {u}, %[rowb]"), salu(f"s_mul_hi_u32 {b}, {u}, %[rowb]"),
            salu(f"s_add_u32 s{dst}, %[{which}blo], {a}"), salu(f"s_addc_u32 s{dst + 1}, %[{which}bhi], {b}")]
    if special:
        first = X0 + 1 if ahead == 3 else O0
        out += [valu(f"v_cndmask_b32_e64 v{first + i}, %[ko{i}], %[kl{i}], s[{S_D}:{S_D + 1}]", (), {f"v{first + i}"})
                for i in range(4)]
    return out


def special_preamble():
    u, k0, a, b = f"s{S_TMP + 3}", f"s{S_TMP + 4}", f"s{S_TMP + 5}", f"s{S_TMP + 6}"
    out = u_of(f"s{S_J}", u)
    out += [salu(f"s_lshl2_add_u32 {k0}, {u}, %[w]"), salu(f"s_lshl_b32 {k0}, {k0}, 5"),
            salu(f"s_add_i32 {a}, {k0}, 32"), salu(f"s_cmp_gt_i32 {a}, %[lk]"),
            salu(f"s_cselect_b32 s{S_MSK}, 3, 0"),
            salu(f"s_mov_b32 s{S_GEN}, s{S_MSK}")]
    for J in range(NBLK):
        out += [salu(f"s_add_i32 {a}, {k0}, {95 - 32 * J}"), salu(f"s_cmp_gt_i32 {a}, %[q0]"),
                salu(f"s_cselect_b32 {a}, {1 << J}, 0"),
                salu(f"s_add_i32 {b}, {k0}, {-39 - 32 * J}"), salu(f"s_cmp_lt_i32 {b}, %[q0]"),
                salu(f"s_cselect_b32 {b}, {1 << J}, 0"),
                salu(f"s_and_b32 {a}, {a}, {b}"), salu(f"s_or_b32 s{S_GEN}, s{S_GEN}, {a}")]
    out += [salu(f"s_cmp_eq_u32 s{S_J}, 0"), salu(f"s_cselect_b32 s{S_NEEDY}, 3, 0"),
            salu(f"s_or_b32 s{S_NEEDY}, s{S_NEEDY}, s{S_GEN}"),
            salu(f"s_sub_i32 s{S_DU}, {k0}, %[q0]"), salu(f"s_add_i32 s{S_DU}, s{S_DU}, 64"),
            salu(f"s_sub_i32 s{S_DU + 1}, s{S_DU}, 32"),
            salu(f"s_sub_i32 s{S_LIM}, %[lk], {k0}")]
    return out + base_of(1, S_GV, True) + base_of(3, S_GK, True)


def advance():
    """After a plain step: j += 1; the V copy base moves to step j + 1 and
    the K copy base to step j + 3 (by 4 key steps, across the band at index
    jump, not past nu - 1)."""
    out = [salu(f"s_add_u32 s{S_J}, s{S_J}, 1")]
    for ahead, base in ((1, S_GV), (3, S_GK)):
        out += [salu(f"s_add_u32 s{S_T}, s{S_J}, {ahead}"),
                salu(f"s_cmp_eq_u32 s{S_T}, s{S_JUMP}"),
                salu(f"s_cselect_b64 s[{S_D}:{S_D + 1}], s[{S_DJUMP}:{S_DJUMP + 1}], s[{S_DSTEP}:{S_DSTEP + 1}]"),
                salu(f"s_cmp_lt_i32 s{S_T}, s{S_NU}"),
                salu(f"s_cselect_b64 s[{S_D}:{S_D + 1}], s[{S_D}:{S_D + 1}], 0"),
                salu(f"s_add_u32 s{base}, s{base}, s{S_D}"),
                salu(f"s_addc_u32 s{base + 1}, s{base + 1}, s{S_D + 1}")]
    out.append(salu(f"s_cmp_eq_u32 s{S_J}, s{S_JUMP}"))
    return out


def switch(tag):
    return ([branch(f"s_cbranch_scc0 L_left{tag}_%=")]
            + [valu(f"v_mov_b32_e32 v{NB + J}, v{NBR + J}", {f"v{NBR + J}"}, {f"v{NB + J}"}) for J in range(NBLK)]
            + [label(f"L_left{tag}_%=")])


def plain_entry():
    out = [salu(f"s_cmp_ge_i32 s{S_J}, s{S_NU}"), branch("s_cbranch_scc1 L_end_%=")]
    out += base_of(1, S_GV, False) + base_of(3, S_GK, False)
    for J in range(NBLK):
        out += [Ins(f"ds_read_b32 v{NB + J}, %[qbase] offset:{QR_BLOCK * J}", "lds", writes={f"v{NB + J}"}),
                Ins(f"ds_read_b32 v{NBR + J}, %[qbase] offset:{QR_BLOCK * J + 72 * 4}", "lds",
                    writes={f"v{NBR + J}"})]
    out.append(Ins("s_waitcnt lgkmcnt(0)", "waitcnt"))
    for J in range(NBLK):
        out += [valu(f"v_sub_f32_e32 v{NB + J}, v{NB + J}, %[m{J}]", {f"v{NB + J}"}, {f"v{NB + J}"}),
                valu(f"v_sub_f32_e32 v{NBR + J}, v{NBR + J}, %[m{J}]", {f"v{NBR + J}"}, {f"v{NBR + J}"})]
    out += [salu(f"s_cmp_lt_i32 s{S_J}, s{S_JUMP}"), branch("s_cbranch_scc1 L_isleft_%=")]
    out += [valu(f"v_mov_b32_e32 v{NB + J}, v{NBR + J}", {f"v{NBR + J}"}, {f"v{NB + J}"}) for J in range(NBLK)]
    out.append(label("L_isleft_%="))
    return out


FENCE = G.FENCE


def check_waits(seq, vm_outstanding):
    """Outstanding-operation check: an LDS read result is used only after an
    lgkmcnt wait retired it, a ring slot is read only after the vmcnt wait
    that retires its copy, a slot is refilled only after the reads of its
    previous contents retired, and the registers of a load from global
    memory (kind gload) are read only after a vmcnt wait retired it.
    vm_outstanding: (slot, registers) of the loads in flight at the start,
    oldest first."""
    lgkm = []
    vm = []     # (slot, regs) per instruction in flight
    for slot, regs in vm_outstanding:
        vm.append((slot, regs))
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
        for _, regs in vm:
            if regs & (c.reads | c.srcc | c.writes):
                raise AssertionError(f"register of a global load in flight touched: {c.text}")
        if c.kind == "lds":
            if c.lds_slot is not None and any(s == c.lds_slot for s, _ in vm):
                raise AssertionError(f"LDS read of a slot whose copy is in flight: {c.text}")
            lgkm.append((c.writes, c.lds_slot))
        if c.kind == "dma":
            if any(slot == c.lds_slot for _, slot in lgkm):
                raise AssertionError(f"slot refilled while reads of it are in flight: {c.text}")
            vm.append((c.lds_slot, set()))
        if c.kind == "gload":
            vm.append((None, c.writes))
    return vm


def build():
    s0, _ = plain_step(0, FENCE)
    s1, _ = plain_step(1, s0)
    c0 = 0.0
    for _ in range(4):
        n0, c0 = plain_step(0, s1)
        n1, _ = plain_step(1, n0)
        stable = [i.text for i in n0] == [i.text for i in s0] and [i.text for i in n1] == [i.text for i in s1]
        s0, s1 = n0, n1
        if stable:
            break
    pre = special_preamble()
    sp_text, sp_phases = {}, {}
    for sl in (0, 1):
        sp_text[sl], sp_phases[sl] = special_step(sl, FENCE + pre)
    # the last block's row sums; then every copy and every LDS read has
    # retired: the statement's register outputs (the V^T and K operands among
    # them) are final when it ends.  A wait in the compiled code after it
    # would not do: the compiler may move register-only work, such as the
    # last PV products that read the V^T operands, above it.
    tail = [mfma16(rs(1), ("v", SEL), ("v", pk(1, 0)), "R1.end"),
            mfma16(rs(1), ("v", SEL), ("v", pk(1, 1)), "R2.end"), Ins("s_waitcnt vmcnt(0)", "waitcnt"),
            Ins("s_waitcnt lgkmcnt(0)", "waitcnt")]
    entry = FENCE + [label("L_sp_top_%="),
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

    e0, e1 = s0 + advance(), s1 + advance()
    pe = plain_entry()
    for seq in (FENCE + e0 + e1 + e0 + tail + FENCE, FENCE + e1 + e0 + e1 + tail + FENCE,
                FENCE + e0 + tail + FENCE, FENCE + e1 + tail + FENCE, FENCE + pe + e0 + tail, FENCE + pe + e1 + tail):
        check_hazards(seq)
    for sl in (0, 1):
        phases = sp_phases[sl]
        for J in range(NBLK):
            if J == 0:
                befores = [FENCE + pre] + [v + [salu("s_add_u32"), branch("s_branch")] + pre
                                           for v in sp_phases[sl ^ 1][NBLK - 1].values()]
            else:
                befores = list(phases[J - 1].values())
            afters = (list(phases[J + 1].values()) if J < NBLK - 1 else
                      [pre + v for v in sp_phases[sl ^ 1][0].values()] + [pe + s0[:40], pe + s1[:40], tail + FENCE])
            for before in befores:
                for seq in phases[J].values():
                    for after in afters:
                        check_hazards(before[-40:] + seq + after[:60])
    # outstanding loads: entry state K(1) loads done, V(0) landed in slot 0
    # (each phase of two special steps on every path, the others on FGM)
    for first in (0, 1):
        slots = [(sl, J) for sl in (first, first ^ 1) for J in range(NBLK)]
        for at, pth in itertools.product(range(len(slots)), PATHS):
            seq = []
            for k, (sl, J) in enumerate(slots):
                seq += sp_phases[sl][J][pth if k == at else "FGM"]
            seq += pe + (s0 + s1 + s0 if first == 0 else s1 + s0 + s1)
            vm = check_waits(seq, [])
            assert len(vm) <= 8, vm
    # every exit (after the special steps, after an even or an odd plain
    # step) leaves nothing in flight
    for seq in (pe + tail, pe + s0 + advance() + tail, pe + s1 + advance() + tail,
                pe + s0 + advance() + s1 + advance() + tail):
        assert_quiet(seq)
    return loop, s0, c0


def render(seq):
    return " \\\n".join(f'  "{i.text}\\n\\t"' for i in seq)


def main():
    loop, s0, c0 = build()
    counts = {}
    for i in s0:
        counts[i.kind] = counts.get(i.kind, 0) + 1
    text = [
        "// flexrel_w64_step.inc -- generated by gen_w64_step.py (run by build.py); do not edit.",
        "// The key-step loop of flexrel_w64.hip.  One plain step: " + ", ".join(
            f"{v} {k}" for k, v in sorted(counts.items())) + f" instructions; modelled issue time {c0:.0f} cycles.",
        "#pragma once",
        "",
        "#define SIDON_W64_VGPR_CLOBBERS " + ", ".join(f'"{r}"' for r in VGPR_CLOBBERS),
        "#define SIDON_W64_SGPR_CLOBBERS " + ", ".join(f'"{r}"' for r in SGPR_CLOBBERS),
        "",
        "#define SIDON_W64_LOOP \\",
        render(loop),
        "",
    ]
    OUT.write_text("\n".join(text))
    print(f"wrote {OUT} ({len(loop)} instructions; one plain step {len(s0)}, modelled {c0:.0f} cycles)",
          file=sys.stderr)


if __name__ == "__main__":
    main()
