"""Write golden vectors for the relative_key attention with the installed
transformers ``Wav2Vec2BertSelfAttention`` (relative_key branch,
modeling_wav2vec2_bert.py:308-327 of transformers 5.15.0; the reference pins
transformers==4.56.1 at pyproject.toml:16 and uses this module as its fp32
reference in scripts/build_engines.py:76-83).

transformers is a third-party library, not the reference; it runs here in
float64 and its outputs are committed as data (.npz) so the tests do not need
it.  Run:  python tests/golden/make_golden.py

The module projects one hidden state h into q, k and v.  To get fp16-exact
q / k / v that are not copies of each other, h holds multiples of 1/64 in
[-4, 4] and the projections are small-integer matrices:
    q = h,   k[:, c] = h[:, pk(c)] - h[:, sk(c)],   v[:, c] = h[:, pv(c)] + h[:, sv(c)]
(pk, sk, pv, sv are seeded permutations; every value stays a multiple of
1/64 below 8 in magnitude, so it is exact in fp16).  linear_out is the
identity, so the module's output is the attention context itself.  The rel
table holds fp16 values.  Items with LK < L are evaluated at their exact
length (the reference's padding semantics, triton_encoder.py:219-226).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent

CASES = {
    # name: (batch, heads, length, lens, seed)
    "hf_b2_h2_l200": (2, 2, 200, [200, 173], 11),
    "hf_b1_h1_l520": (1, 1, 520, [487], 12),
    "hf_b1_h2_l40": (1, 2, 40, [40], 13),
}


def _module(heads: int):
    from transformers import Wav2Vec2BertConfig
    from transformers.models.wav2vec2_bert.modeling_wav2vec2_bert import Wav2Vec2BertSelfAttention

    cfg = Wav2Vec2BertConfig(hidden_size=64 * heads, num_attention_heads=heads,
                             position_embeddings_type="relative_key",
                             left_max_position_embeddings=64, right_max_position_embeddings=8,
                             attention_dropout=0.0)
    return Wav2Vec2BertSelfAttention(cfg).double().eval()


def make_case(batch: int, heads: int, length: int, lens: list[int], seed: int) -> dict:
    rng = np.random.default_rng(seed)
    hid = 64 * heads
    h = np.clip(np.round(rng.standard_normal((batch, length, hid)) * 64.0) / 64.0, -4.0, 4.0)
    perms = [rng.permutation(hid) for _ in range(4)]
    eye = np.eye(hid)
    wq = eye
    wk = eye[perms[0]] - eye[perms[1]]          # k[:, c] = h[:, p0(c)] - h[:, p1(c)]
    wv = eye[perms[2]] + eye[perms[3]]
    rel = rng.standard_normal((73, 64)) * 0.3
    rel = rel.astype(np.float16).astype(np.float64)
    mod = _module(heads)
    with torch.no_grad():
        mod.linear_q.weight.copy_(torch.from_numpy(wq))
        mod.linear_k.weight.copy_(torch.from_numpy(wk))
        mod.linear_v.weight.copy_(torch.from_numpy(wv))
        mod.linear_out.weight.copy_(torch.from_numpy(eye))
        for lin in (mod.linear_q, mod.linear_k, mod.linear_v, mod.linear_out):
            lin.bias.zero_()
        mod.distance_embedding.weight.copy_(torch.from_numpy(rel))
        expected = np.zeros((batch, length, hid))
        for b, lk in enumerate(lens):
            x = torch.from_numpy(h[b:b + 1, :lk])
            expected[b, :lk] = mod(x)[0][0].numpy()
    q = h
    k = h @ wk.T
    v = h @ wv.T
    for t in (q, k, v):
        assert np.array_equal(t.astype(np.float16).astype(np.float64), t), "inputs must be fp16-exact"

    return {
        "hidden": h.astype(np.float16),
        "perms": np.stack(perms).astype(np.int32),
        "heads": np.int32(heads),
        "rel": rel.astype(np.float16),
        "lens": np.asarray(lens, dtype=np.int32),
        # [B, L, H*64]; rows >= lens[b] are not defined by the exact-length
        # run and are left 0.
        "expected": expected.astype(np.float32),
    }


def load_case(path) -> dict:
    """Rebuild fp16 q / k / v [B, H, L, 64] and the expected context from a fixture."""
    d = np.load(path)
    h = d["hidden"].astype(np.float64)
    p0, p1, p2, p3 = d["perms"]
    heads = int(d["heads"])
    batch, length, _ = h.shape

    def bhld(t):
        return np.ascontiguousarray(t.reshape(batch, length, heads, 64).transpose(0, 2, 1, 3))

    return {
        "q": bhld(h).astype(np.float16),
        "k": bhld(h[..., p0] - h[..., p1]).astype(np.float16),
        "v": bhld(h[..., p2] + h[..., p3]).astype(np.float16),
        "rel": d["rel"],
        "lens": d["lens"],
        "expected": bhld(d["expected"].astype(np.float64)),
    }


def main() -> None:
    for name, (batch, heads, length, lens, seed) in CASES.items():
        data = make_case(batch, heads, length, lens, seed)
        path = HERE / f"{name}.npz"
        np.savez_compressed(path, **data)
        print(f"wrote {path.name}: {path.stat().st_size} bytes", flush=True)


if __name__ == "__main__":
    main()
