"""CPU oracle for the relative_key flash attention -- TEST INFRASTRUCTURE ONLY.

Nothing in the product path imports this module.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg use it,
and only as the checker / the timed CPU baseline, never as the thing measured
on the GPU.

The math (batch b, head h, query row i < L, key j < LK_b, D = 64):

    s_ij = (q_i . k_j + q_i . E[clamp(j - i, -64, 8) + 64]) / sqrt(D)
    o_i  = sum_{j < LK_b} softmax_j(s_ij) v_j

Sources restated here (read, not run):
  * src/sidon_triton/flexrel_triton.py:281-294 ``explicit_core_fp32``: the
    bias ``einsum(q, E)`` gathered by ``clamp(pos_j - pos_i, -64, 8) + 64`` and
    added to ``q k^T`` *before* the division by sqrt(d);
  * src/sidon_triton/flexrel_triton.py:297-328 ``torch_core_chunked``: the
    same per 512-row chunk (``torch_core_chunked`` below is its fp32 twin and
    is the timed CPU baseline);
  * src/sidon_triton/triton_encoder.py:219-226, :283, :304: keys j >= LENS[b]
    are masked (weight exactly 0); every query row < L is still computed;
  * transformers ``Wav2Vec2BertSelfAttention`` relative_key branch
    (modeling_wav2vec2_bert.py:308-327 in the installed 5.15.0; the reference
    pins transformers==4.56.1, pyproject.toml:16): distance = key - query.

Pinning (what checks each function, see tests/test_oracle.py):
  * ``flexrel_reference``: committed golden vectors written by the installed
    transformers module in float64 (tests/golden/make_golden.py), the
    pure-Python ``flexrel_bruteforce`` on tiny inputs, and closed-form special
    cases: E == 0 and E with equal rows reduce to
    ``torch.nn.functional.scaled_dot_product_attention``; LK == 1 gives v_0;
    heads are independent; valid rows do not depend on keys >= LK.
  * ``flexrel_tiled``: equals ``flexrel_reference`` in float64 over a sweep of
    (rows per block, keys per tile, key splits, L, LK).
  * ``torch_core_chunked``: equals ``flexrel_reference`` to fp32 rounding.
  * ``flexrel_bruteforce``: scalar loops with ``math.exp`` -- an independent
    statement, checked against the transformers golden vectors.
  * ``errors``: closed-form known answers (a constant reference scaled by
    1 + eps gives relative RMSE eps and SNR -20 log10 eps, exactly 60 dB at
    1e-3; a +-1 reference plus delta; an uneven two-element case whose RMS,
    mean |delta| and rms(actual) all differ; identical inputs hit the 1e-12
    noise floor), with planted variants (mean |delta|, 10 log10, signal from
    ``actual``) that the known answers reject.
  * ``attention_flops``: the 95.09 / 2.416 GFLOP figures of the c3 / c1
    configurations.
Planted-mistake tests mutate this module's formula (sign of the distance,
clamp bounds, scale placement, mask) and require the golden check to fail.

Convention beyond the reference: a batch item with LK == 0 produces zero
rows (the reference would divide 0 by 0).
"""

from __future__ import annotations

import math

import numpy as np

LEFT = 64
RIGHT = 8
NUM_POS = LEFT + RIGHT + 1  # 73
HEAD_DIM = 64


def rel_index(rows: np.ndarray, keys: np.ndarray, left: int = LEFT, right: int = RIGHT) -> np.ndarray:
    """clamp(j - i, -left, right) + left for every (row i, key j) pair.

    flexrel_triton.py:288-289 (``idx = clamp(pos_j - pos_i, -LEFT, RIGHT) + LEFT``).
    """
    return np.clip(keys[None, :] - rows[:, None], -left, right) + left


def _lens_of(lens, batch: int, length: int) -> list[int]:
    if lens is None:
        return [length] * batch
    out = [int(x) for x in np.asarray(lens).reshape(-1)]
    if len(out) != batch:
        raise ValueError(f"lens has {len(out)} entries for batch {batch}")
    return [min(max(x, 0), length) for x in out]


def flexrel_reference(q, k, v, rel, lens=None, chunk: int = 256, scale_before_bias: bool = False,
                      _distance_sign: int = 1, _left: int = LEFT, _right: int = RIGHT,
                      _mask: bool = True) -> np.ndarray:
    """Closed form in float64.  q/k/v: [B, H, L, D]; rel: [73, D]; lens: [B] or None.

    Returns float64 [B, H, L, D]; rows i >= LK_b are computed over keys < LK_b
    like every other row.  Underscored arguments exist only so tests can plant
    mistakes; the defaults are the reference's math.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    rel = np.asarray(rel, dtype=np.float64)
    batch, heads, length, dim = q.shape
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError("q, k and v must share one [B, H, L, D] shape")
    if rel.shape != (_left + _right + 1, dim):
        raise ValueError(f"rel must be [{_left + _right + 1}, {dim}]")
    out = np.zeros((batch, heads, length, dim), dtype=np.float64)
    inv = 1.0 / math.sqrt(dim)
    for b, lk in enumerate(_lens_of(lens, batch, length)):
        nk = lk if _mask else length
        if nk == 0:
            continue
        kb, vb = k[b, :, :nk], v[b, :, :nk]
        keys = np.arange(nk)
        for start in range(0, length, chunk):
            stop = min(start + chunk, length)
            qc = q[b, :, start:stop]                      # [H, c, D]
            rows = np.arange(start, stop)
            if _distance_sign > 0:
                idx = rel_index(rows, keys, _left, _right)
            else:
                idx = rel_index(keys, rows, _left, _right).T
            qr = qc @ rel.T                               # [H, c, 73]
            bias = np.take_along_axis(qr, np.broadcast_to(idx, (heads,) + idx.shape), axis=2)
            if scale_before_bias:
                s = (qc @ kb.transpose(0, 2, 1)) * inv + bias
            else:
                s = (qc @ kb.transpose(0, 2, 1) + bias) * inv
            s = s - s.max(axis=2, keepdims=True)
            p = np.exp(s)
            out[b, :, start:stop] = (p @ vb) / p.sum(axis=2, keepdims=True)
    return out


def flexrel_bruteforce(q, k, v, rel, lens=None) -> np.ndarray:
    """Scalar loops with math.exp -- tiny inputs only (an independent statement)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    rel = np.asarray(rel, dtype=np.float64)
    batch, heads, length, dim = q.shape
    out = np.zeros_like(q)
    for b, lk in enumerate(_lens_of(lens, batch, length)):
        for h in range(heads):
            for i in range(length):
                if lk == 0:
                    continue
                scores = []
                for j in range(lk):
                    d = min(max(j - i, -LEFT), RIGHT) + LEFT
                    dot = 0.0
                    for c in range(dim):
                        dot += q[b, h, i, c] * (k[b, h, j, c] + rel[d, c])
                    scores.append(dot / math.sqrt(dim))
                top = max(scores)
                weights = [math.exp(x - top) for x in scores]
                total = sum(weights)
                for c in range(dim):
                    out[b, h, i, c] = sum(w * v[b, h, j, c] for j, w in enumerate(weights)) / total
    return out


def flexrel_tiled(q, k, v, rel, lens=None, rows_per_block: int = 32, keys_per_tile: int = 64,
                  key_splits: int = 1, p_dtype=None) -> np.ndarray:
    """Emulation of the kernel's tile schedule in float64 (the GPU kernel's algorithm).

    Per block of ``rows_per_block`` query rows: key tiles [0, LK) of
    ``keys_per_tile`` keys are divided into ``key_splits`` contiguous ranges;
    each range runs an online softmax in base-2 units; tiles entirely left
    (j - i <= -64) or right (j - i >= 8) of every row use the per-row constant
    bias q.E[0] / q.E[72] folded into the exponent, the others gather the bias
    per score; keys >= LK in the straddling tile get -inf; the ranges are
    merged by rescaling to the common max.  ``p_dtype`` (e.g. np.float16)
    rounds the probabilities before the PV product as the kernel does.
    Structure follows triton_encoder.py:187-195 (online update) and :246-307
    (region split), with the split merge of a flash-decoding combine.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    rel = np.asarray(rel, dtype=np.float64)
    batch, heads, length, dim = q.shape
    c = math.log2(math.e) / math.sqrt(dim)
    bm, bn = rows_per_block, keys_per_tile
    out = np.zeros_like(q)
    for b, lk in enumerate(_lens_of(lens, batch, length)):
        ntiles = -(-lk // bn)
        for q0 in range(0, length, bm):
            q1 = min(q0 + bm, length)
            rows = np.arange(q0, q1)
            qb = q[b, :, q0:q1]                                 # [H, r, D]
            qr = qb @ rel.T                                     # [H, r, 73] raw
            parts = []
            for split in range(key_splits):
                t_lo, t_hi = split * ntiles // key_splits, (split + 1) * ntiles // key_splits
                m = np.full((heads, len(rows)), -np.inf)
                l = np.zeros((heads, len(rows)))
                acc = np.zeros((heads, len(rows), dim))
                for t in range(t_lo, t_hi):
                    n0 = t * bn
                    keys = np.arange(n0, n0 + bn)
                    kt = np.zeros((heads, bn, dim))
                    vt = np.zeros((heads, bn, dim))
                    valid = keys < lk
                    nv = min(n0 + bn, lk) - n0
                    kt[:, :nv] = k[b, :, n0:n0 + nv]
                    vt[:, :nv] = v[b, :, n0:n0 + nv]
                    s = qb @ kt.transpose(0, 2, 1)              # [H, r, bn] raw
                    left = n0 + bn - 1 + LEFT <= q0
                    right = n0 >= q0 + bm - 1 + RIGHT
                    off = np.zeros((heads, len(rows)))
                    if left:
                        off = qr[:, :, 0] * c
                    elif right:
                        off = qr[:, :, NUM_POS - 1] * c
                    else:
                        idx = rel_index(rows, keys)
                        s = s + np.take_along_axis(qr, np.broadcast_to(idx, (heads,) + idx.shape), axis=2)
                    s = np.where(valid[None, None, :], s, -np.inf)
                    m_new = np.maximum(m, s.max(axis=2) * c + off)
                    alpha = np.exp2(m - m_new)
                    p = np.exp2(s * c + (off - m_new)[:, :, None])
                    l = l * alpha + p.sum(axis=2)
                    if p_dtype is not None:
                        p = p.astype(p_dtype).astype(np.float64)
                    acc = acc * alpha[:, :, None] + p @ vt
                    m = m_new
                parts.append((m, l, acc))
            mmax = np.max(np.stack([pm for pm, _, _ in parts]), axis=0)
            l_tot = np.zeros_like(mmax)
            acc_tot = np.zeros((heads, len(rows), dim))
            for pm, pl, pa in parts:
                live = ~np.isneginf(pm)
                f = np.where(live, np.exp2(np.where(live, pm - np.where(live, mmax, 0.0), 0.0)), 0.0)
                l_tot += pl * f
                acc_tot += pa * f[:, :, None]
            with np.errstate(invalid="ignore", divide="ignore"):
                res = np.where(l_tot[:, :, None] > 0, acc_tot / l_tot[:, :, None], 0.0)
            out[b, :, q0:q1] = res
    return out


def torch_core_chunked(q, k, v, rel, lens=None, out=None, chunk: int = 512, dtype=None):
    """fp32 torch restatement of flexrel_triton.py:297-328 with the key mask.

    This is the CPU baseline the benchmark times (the reference's own
    CPU-capable fp32 path); tensors are torch tensors [B, H, L, D] on any
    device.  ``dtype`` (default float32) is the compute precision.
    """
    import torch

    batch, heads, length, dim = q.shape
    dtype = torch.float32 if dtype is None else dtype
    dev = q.device
    scale = 1.0 / math.sqrt(dim)
    if out is None:
        out = torch.zeros(q.shape, dtype=dtype, device=dev)
    rf = rel.to(dtype)
    for b, lk in enumerate(_lens_of(None if lens is None else [int(x) for x in lens], batch, length)):
        if lk == 0:
            out[b].zero_()
            continue
        kf = k[b:b + 1, :, :lk].to(dtype)
        vf = v[b:b + 1, :, :lk].to(dtype)
        pos_k = torch.arange(lk, device=dev)
        for start in range(0, length, chunk):
            stop = min(start + chunk, length)
            qc = q[b:b + 1, :, start:stop].to(dtype)
            idx = torch.clamp(pos_k[None, :] - torch.arange(start, stop, device=dev)[:, None], -LEFT, RIGHT) + LEFT
            bias = torch.gather(torch.einsum("bhld,rd->bhlr", qc, rf), 3,
                                idx.view(1, 1, stop - start, lk).expand(1, heads, -1, -1))
            scores = (qc @ kf.transpose(-2, -1) + bias) * scale
            out[b:b + 1, :, start:stop] = (torch.softmax(scores, dim=-1) @ vf).to(out.dtype)
    return out


def errors(reference, actual, *, _noise: str = "rms", _db_factor: float = 20.0,
           _signal_from: str = "reference") -> dict:
    """max_abs / relative RMSE / SNR dB as in src/sidon_triton/engines.py:47-55.

    signal = rms(reference), noise = rms(reference - actual) (the noise floor
    is clamped at 1e-12 as there; here also the signal at 1e-30, so an
    all-zero reference gives a finite, very negative SNR instead of a math
    error), snr_db = 20 log10(signal / noise).  Evaluated in float64.

    The underscored keywords exist only so tests can plant mistakes (mean
    |delta| instead of the RMS, a 10 log10 power ratio, the signal taken from
    ``actual``) and show that the closed-form known answers reject them.
    """
    ref = np.asarray(reference, dtype=np.float64)
    act = np.asarray(actual, dtype=np.float64)
    delta = np.abs(ref - act)
    sig_src = ref if _signal_from == "reference" else act
    signal = math.sqrt(float(np.mean(sig_src * sig_src))) if ref.size else 0.0
    if _noise == "rms":
        noise = math.sqrt(float(np.mean(delta * delta))) if ref.size else 0.0
    else:
        noise = float(np.mean(delta)) if ref.size else 0.0
    return {
        "max_abs": float(delta.max()) if delta.size else 0.0,
        "relative_rmse": noise / max(signal, 1e-12),
        "snr_db": _db_factor * math.log10(max(signal, 1e-30) / max(noise, 1e-12)),
    }


def attention_flops(heads_total: int, lq: int, lk: int, dim: int = HEAD_DIM) -> float:
    """Algorithmic FLOPs: 4*Lq*Lk*D (QK^T + PV) + 2*Lq*73*D (Q.E^T) per head."""
    return float(heads_total) * (4.0 * lq * lk * dim + 2.0 * lq * NUM_POS * dim)
