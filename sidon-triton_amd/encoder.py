"""The w2v-BERT conformer encoder (Sidon's 8 layers) on the MI355X library.

Mirrors src/sidon_triton/triton_encoder.py:

  * ``pack_encoder(model)`` (:394-445): the model's weights re-laid out for the
    encoder -- fused QKV, fp16 GEMM weights, FFN output weights pre-scaled by
    0.5, depthwise taps as [K, C] fp32, and the biases of the accumulating
    residual GEMMs as per-layer running sums (summed in float64) that the next
    norm adds;
  * ``HipEncoder(packed)(features, frames, out)`` (:448-511): fp32 features
    [B, L, 160] (+ valid frames [B]) -> hidden [B, L, C] fp32, with the
    residual stream kept in fp32 and every residual GEMM accumulating into it
    (fp16 operands, fp32 output), the norms fused with the bias adds;
  * ``save_encoder`` / ``load_encoder`` (:514-525): here a safetensors file
    with the scalars in its metadata, loaded without unpickling anything;
    ``load_encoder`` also reads the reference's own ``encoder_triton.pt``
    (with ``torch.load(weights_only=True)``).

Per layer the work is: res_norm (HIP), the QKV GEMM on hipBLASLt through
torch, the residual projections into the fp32 stream (one HIP kernel while
its 64 x 64 tiles fit one per CU, else hipBLASLt), the pointwise conv's first
GEMM on rocBLAS with the kernel chosen by timing (``blas.gemm_nt``), the
feed-forward input projections with bias and SiLU (one HIP GEMM kernel where
its tiles fill the chip, else hipBLASLt with the bias and SiLU in its epilogue),
the relative_key attention (HIP), and the conv module's GLU + causal
depthwise conv + LayerNorm + SiLU as one HIP kernel reading the pointwise
conv's output.  Every op launches on the current stream, reads no
device data on the host and, given a ``workspace``, allocates nothing, so a
whole encoder call can be captured into one HIP graph per length bucket.
"""

from __future__ import annotations

import json
from pathlib import Path

import torch

from .blas import gemm_nt
from .conformer import (glu_causal_dw_norm, linear_silu, linear_silu_lt, linear_silu_preferred, residual_gemm,
                        residual_gemm_preferred, silu_)
from .encoder_attention import flexrel_attention
from .encoder_block import res_norm
from .flexrel import HEAD_DIM, LEFT, NUM_POS, RIGHT

ENCODER_FILE = "encoder_mi355x.safetensors"
_FORMAT = "sidon-mi355x-encoder"
_NORMS = ("ffn1_ln", "attn_ln", "conv_ln", "dw_ln", "ffn2_ln", "final_ln")
_LAYER_TENSORS = ("ffn1_w1", "ffn1_b1", "ffn1_w2", "qkv_w", "qkv_b", "rel", "out_w", "pw1_w", "dwt", "pw2_w",
                  "ffn2_w1", "ffn2_b1", "ffn2_w2")


# ---- weights -------------------------------------------------------------------


def model_weights(model) -> dict:
    """Weights of a transformers ``Wav2Vec2BertModel`` with relative_key
    attention (or a wrapper holding one as ``.model``, as Sidon's encoder
    module does) in the model's own layout: per-projection q/k/v, unscaled
    FFN weights, depthwise taps [C, K]."""
    ssl = getattr(model, "model", model)
    cfg = ssl.config
    if cfg.position_embeddings_type != "relative_key":
        raise ValueError("the encoder needs relative_key attention")
    if int(cfg.left_max_position_embeddings) != LEFT or int(cfg.right_max_position_embeddings) != RIGHT:
        raise ValueError(f"the attention window must be -{LEFT}..+{RIGHT}")

    def ln(m):
        return (m.weight.detach(), m.bias.detach(), float(m.eps))

    def t(x):
        return x.detach()

    fp = ssl.feature_projection
    weights = {"heads": int(cfg.num_attention_heads), "fp_ln": ln(fp.layer_norm), "fp_w": t(fp.projection.weight),
               "fp_b": t(fp.projection.bias), "layers": []}
    for layer in ssl.encoder.layers:
        att, conv = layer.self_attn, layer.conv_module
        for m in (conv.pointwise_conv1, conv.depthwise_conv, conv.pointwise_conv2):
            if m.bias is not None:
                raise ValueError("the conv module's convolutions carry no bias")
        p = {"ffn1_ln": ln(layer.ffn1_layer_norm), "ffn1_w1": t(layer.ffn1.intermediate_dense.weight),
             "ffn1_b1": t(layer.ffn1.intermediate_dense.bias), "ffn1_w2": t(layer.ffn1.output_dense.weight),
             "ffn1_b2": t(layer.ffn1.output_dense.bias), "attn_ln": ln(layer.self_attn_layer_norm)}
        for name, lin in zip("qkv", (att.linear_q, att.linear_k, att.linear_v)):
            p[f"{name}_w"], p[f"{name}_b"] = t(lin.weight), t(lin.bias)
        p.update({"rel": t(att.distance_embedding.weight), "out_w": t(att.linear_out.weight),
                  "out_b": t(att.linear_out.bias), "conv_ln": ln(conv.layer_norm),
                  "pw1_w": t(conv.pointwise_conv1.weight)[:, :, 0], "dw_w": t(conv.depthwise_conv.weight)[:, 0, :],
                  "dw_ln": ln(conv.depthwise_layer_norm), "pw2_w": t(conv.pointwise_conv2.weight)[:, :, 0],
                  "ffn2_ln": ln(layer.ffn2_layer_norm), "ffn2_w1": t(layer.ffn2.intermediate_dense.weight),
                  "ffn2_b1": t(layer.ffn2.intermediate_dense.bias), "ffn2_w2": t(layer.ffn2.output_dense.weight),
                  "ffn2_b2": t(layer.ffn2.output_dense.bias), "final_ln": ln(layer.final_layer_norm)})
        weights["layers"].append(p)
    return weights


def pack_weights(weights: dict) -> dict:
    """Model-layout weights (``model_weights``) -> the packed encoder weights
    (CPU tensors): the layout of src/sidon_triton/triton_encoder.py:417-445."""

    def f32(x):
        return x.detach().float().contiguous().cpu()

    def h(x):
        return x.detach().to(torch.float16).contiguous().cpu()

    def ln(norm):
        return (f32(norm[0]), f32(norm[1]), float(norm[2]))

    heads = int(weights["heads"])
    packed = {"heads": heads, "fp_ln": ln(weights["fp_ln"]), "fp_w": f32(weights["fp_w"]),
              "fp_b": f32(weights["fp_b"]), "layers": []}
    for p in weights["layers"]:
        hid = p["out_w"].shape[0]
        if hid != heads * HEAD_DIM or tuple(p["rel"].shape) != (NUM_POS, HEAD_DIM):
            raise ValueError(f"hidden {hid} must be {HEAD_DIM} x {heads} heads and rel [{NUM_POS}, {HEAD_DIM}]")
        q = {name: ln(p[name]) for name in _NORMS}
        q.update({
            "ffn1_w1": h(p["ffn1_w1"]), "ffn1_b1": h(p["ffn1_b1"]), "ffn1_w2": h(p["ffn1_w2"] * 0.5),
            "qkv_w": h(torch.cat([p["q_w"], p["k_w"], p["v_w"]])),
            "qkv_b": h(torch.cat([p["q_b"], p["k_b"], p["v_b"]])),
            "rel": h(p["rel"]), "out_w": h(p["out_w"]), "pw1_w": h(p["pw1_w"]),
            "dwt": f32(p["dw_w"].t()), "pw2_w": h(p["pw2_w"]),
            "ffn2_w1": h(p["ffn2_w1"]), "ffn2_b1": h(p["ffn2_b1"]), "ffn2_w2": h(p["ffn2_w2"] * 0.5),
        })
        # The residual GEMMs skip their biases; the running sums (float64)
        # are added inside the next norm: after FFN1, after the attention (and
        # the conv module, which has none), after FFN2.
        b1 = p["ffn1_b2"].double() * 0.5
        b2 = b1 + p["out_b"].double()
        b4 = b2 + p["ffn2_b2"].double() * 0.5
        q["cum_bias"] = (f32(b1), f32(b2), f32(b4))
        packed["layers"].append(q)
    return packed


def pack_encoder(model) -> dict:
    """transformers Wav2Vec2BertModel (relative_key) -> packed weights."""
    return pack_weights(model_weights(model))


def _to(value, device):
    if isinstance(value, torch.Tensor):
        return value.to(device)
    if isinstance(value, (tuple, list)):
        return type(value)(_to(v, device) for v in value)
    if isinstance(value, dict):
        return {k: _to(v, device) for k, v in value.items()}
    return value


# ---- the encoder ---------------------------------------------------------------


class HipEncoder:
    """fp32 features [B, L, F] (+ valid frames [B]) -> hidden [B, L, C] fp32 on
    packed weights (``pack_encoder`` / ``pack_weights``)."""

    def __init__(self, packed: dict, device="cuda", fused_ffn: bool | str | None = None,
                 own_residual: bool | None = None) -> None:
        """fused_ffn: the feed-forward input projections as this library's
        GEMM + bias + SiLU kernel (True), as hipBLASLt with the bias and SiLU
        in its epilogue ("lt"), as torch.addmm followed by a SiLU pass
        (False), or chosen per call by shape (None: this library's kernel
        where it is expected to be faster, else "lt").  own_residual: the residual projections on this
        library's kernel (True, ``conformer.residual_gemm``), on torch.addmm
        (False), or chosen per call by shape (None)."""
        device = torch.device(device)
        if device.type == "cuda" and device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        packed = _to(packed, device)
        self.device = device
        self.heads = int(packed["heads"])
        self.fp_ln = packed["fp_ln"]
        self.fp_w, self.fp_b = packed["fp_w"], packed["fp_b"]
        self.layers = packed["layers"]
        self.hidden = self.fp_w.shape[0]
        self.features = self.fp_w.shape[1]
        self.inter = self.layers[0]["ffn1_w1"].shape[0]
        self.fused_ffn = fused_ffn
        self.own_residual = own_residual

    def workspace(self, rows: int) -> dict:
        """Buffers for calls of up to ``rows`` = B*L rows (graph capture
        reuses them): normalized features, the normed stream, one fp16 buffer
        for the FFN intermediate / fused QKV / pointwise conv output (their
        lifetimes do not overlap), and the attention context / conv output."""
        wide = max(self.inter, 3 * self.hidden)
        f16 = dict(device=self.device, dtype=torch.float16)
        return {"rows": rows, "fn": torch.empty(rows * self.features, device=self.device),
                "xn": torch.empty(rows * self.hidden, **f16), "wide": torch.empty(rows * wide, **f16),
                "ctx": torch.empty(rows * self.hidden, **f16)}

    @torch.no_grad()
    def __call__(self, features: torch.Tensor, frames: torch.Tensor | None = None,
                 out: torch.Tensor | None = None, workspace: dict | None = None) -> torch.Tensor:
        """out: optional fp32 [B, L, C] buffer the residual stream (and so the
        result) lives in.  frames: int32 [B] valid frames on the device (None:
        all L).  Rows past an item's valid frames hold finite values nobody
        should read."""
        batch, length, nfeat = features.shape
        if nfeat != self.features:
            raise ValueError(f"features must have {self.features} channels (got {nfeat})")
        rows = batch * length
        device = self.device
        if frames is None:
            lens = torch.full((batch,), length, dtype=torch.int32, device=device)
        else:
            lens = frames if frames.dtype == torch.int32 else frames.to(torch.int32)
        ws = workspace if workspace is not None else self.workspace(rows)
        if ws["rows"] < rows:
            raise ValueError(f"workspace holds {ws['rows']} rows, the call needs {rows}")
        hid = self.hidden
        fn = ws["fn"][:rows * nfeat].view(rows, nfeat)
        xn_buf = ws["xn"][:rows * hid].view(rows, hid)
        wide = ws["wide"]
        ctx = ws["ctx"][:rows * hid].view(rows, hid)
        h_buf = wide[:rows * self.inter].view(rows, self.inter)
        qkv_buf = wide[:rows * 3 * hid].view(rows, 3 * hid)
        pw1_buf = wide[:rows * 2 * hid].view(rows, 2 * hid)

        feats = features.reshape(rows, nfeat)
        if feats.dtype != torch.float32 or not feats.is_contiguous():
            feats = feats.float().contiguous()
        res_norm(feats, norm2=self.fp_ln, write_x=False, xn_dtype=torch.float32, xn=fn)
        x = torch.empty(rows, hid, device=device) if out is None else out.view(rows, hid)
        torch.addmm(self.fp_b, fn, self.fp_w.t(), out=x)  # fp32 stream
        layers = self.layers
        xn = res_norm(x, norm2=layers[0]["ffn1_ln"], write_x=False, xn=xn_buf)

        fused = self.fused_ffn
        if fused is None:
            fused = True if linear_silu_preferred(rows, self.inter, hid, device) else "lt"

        def ffn_in(w, b):
            if fused == "lt":
                return linear_silu_lt(xn, w, b, out=h_buf)
            if fused:
                return linear_silu(xn, w, b, out=h_buf)
            return silu_(torch.addmm(b, xn, w.t(), out=h_buf))

        own = {k: (residual_gemm_preferred(rows, hid, k, device) if self.own_residual is None
                   else self.own_residual) for k in (hid, self.inter)}

        def res(a, w, bias, **kw):
            # The residual projections: this library's kernel while its 64 x 64
            # tiles fit one per CU (short chunks), else torch.addmm (hipBLASLt);
            # rocBLAS's timed choice was no faster inside the encoder graph.
            if own[a.shape[1]]:
                residual_gemm(x, a, w)
            else:
                torch.addmm(x, a, w.t(), out_dtype=torch.float32, out=x)
            return res_norm(x, bias=bias, xn=xn_buf if kw.get("norm2") is not None else None, **kw)

        for i, p in enumerate(layers):
            b1, b2, b4 = p["cum_bias"]
            last = i + 1 == len(layers)
            h = ffn_in(p["ffn1_w1"], p["ffn1_b1"])
            xn = res(h, p["ffn1_w2"], b1, norm2=p["attn_ln"], write_x=False)
            qkv = torch.addmm(p["qkv_b"], xn, p["qkv_w"].t(), out=qkv_buf)
            c = flexrel_attention(qkv, batch, self.heads, p["rel"], lens, out=ctx)
            xn = res(c, p["out_w"], b2, norm2=p["conv_ln"], write_x=False)
            pw1 = gemm_nt(xn, p["pw1_w"], pw1_buf)
            s = glu_causal_dw_norm(pw1, batch, p["dwt"], *p["dw_ln"], out=ctx)
            xn = res(s, p["pw2_w"], b2, norm2=p["ffn2_ln"], write_x=False)
            h = ffn_in(p["ffn2_w1"], p["ffn2_b1"])
            xn = res(h, p["ffn2_w2"], b4, norm1=p["final_ln"],
                     norm2=None if last else layers[i + 1]["ffn1_ln"])
        return x.view(batch, length, hid)


# ---- file format ---------------------------------------------------------------


def save_encoder(packed: dict, max_batch: int, max_seconds: float, path) -> None:
    """Write packed weights (+ the runtime's maximum batch and seconds) as one
    safetensors file; the scalars (heads, norm eps) go into its metadata."""
    from safetensors.torch import save_file

    tensors = {"fp_ln.w": packed["fp_ln"][0], "fp_ln.b": packed["fp_ln"][1], "fp_w": packed["fp_w"],
               "fp_b": packed["fp_b"]}
    eps = {"fp_ln": packed["fp_ln"][2]}
    for i, p in enumerate(packed["layers"]):
        for name in _NORMS:
            tensors[f"layers.{i}.{name}.w"], tensors[f"layers.{i}.{name}.b"] = p[name][0], p[name][1]
            eps[f"layers.{i}.{name}"] = p[name][2]
        for name in _LAYER_TENSORS:
            tensors[f"layers.{i}.{name}"] = p[name]
        for j, b in enumerate(p["cum_bias"]):
            tensors[f"layers.{i}.cum_bias.{j}"] = b
    tensors = {k: v.detach().contiguous().cpu() for k, v in tensors.items()}
    meta = {"format": _FORMAT, "heads": str(int(packed["heads"])), "layers": str(len(packed["layers"])),
            "max_batch": str(int(max_batch)), "max_seconds": repr(float(max_seconds)), "eps": json.dumps(eps)}
    save_file(tensors, str(Path(path)), metadata=meta)


def read_encoder(path) -> tuple[dict, int, float]:
    """-> (packed weights on the CPU, max_batch, max_seconds)."""
    from safetensors import safe_open

    with safe_open(str(Path(path)), framework="pt") as f:
        meta = f.metadata() or {}
        if meta.get("format") != _FORMAT:
            raise ValueError(f"{path} is not a {_FORMAT} file")
        t = {k: f.get_tensor(k) for k in f.keys()}
    eps = json.loads(meta["eps"])
    packed = {"heads": int(meta["heads"]), "fp_ln": (t["fp_ln.w"], t["fp_ln.b"], float(eps["fp_ln"])),
              "fp_w": t["fp_w"], "fp_b": t["fp_b"], "layers": []}
    for i in range(int(meta["layers"])):
        p = {name: (t[f"layers.{i}.{name}.w"], t[f"layers.{i}.{name}.b"], float(eps[f"layers.{i}.{name}"]))
             for name in _NORMS}
        p.update({name: t[f"layers.{i}.{name}"] for name in _LAYER_TENSORS})
        p["cum_bias"] = tuple(t[f"layers.{i}.cum_bias.{j}"] for j in range(3))
        packed["layers"].append(p)
    return packed, int(meta["max_batch"]), float(meta["max_seconds"])


def read_triton_encoder(path) -> tuple[dict, int, float]:
    """Read the reference's own packed file (``encoder_triton.pt`` of
    ``save_encoder``, src/sidon_triton/triton_encoder.py:514-518): a dict of
    tensors, tuples and numbers, so it loads with ``weights_only=True`` (the
    reference's loader, :521-525, unpickles arbitrary objects; this one does
    not).  The packed layout is the one ``pack_weights`` writes, key for key.
    -> (packed weights on the CPU, max_batch, max_seconds)."""
    saved = torch.load(str(Path(path)), map_location="cpu", weights_only=True)
    if not isinstance(saved, dict) or "packed" not in saved:
        raise ValueError(f"{path} is not a packed encoder file")
    packed = saved["packed"]
    missing = {"heads", "fp_ln", "fp_w", "fp_b", "layers"} - set(packed)
    if missing:
        raise ValueError(f"{path}: packed weights lack {sorted(missing)}")
    layer_keys = set(_NORMS) | set(_LAYER_TENSORS) | {"cum_bias"}
    for i, layer in enumerate(packed["layers"]):
        if set(layer) != layer_keys:
            raise ValueError(f"{path}: layer {i} keys differ from the packed layout")
    return packed, int(saved["max_batch"]), float(saved["max_seconds"])


def load_encoder(path, device="cuda") -> tuple[HipEncoder, int, float]:
    """-> (HipEncoder, max_batch, max_seconds) from this library's
    safetensors file or from the reference's ``encoder_triton.pt``."""
    path = Path(path)
    with open(path, "rb") as f:
        zip_magic = f.read(2) == b"PK"   # torch.save writes a zip archive
    packed, max_batch, max_seconds = read_triton_encoder(path) if zip_magic else read_encoder(path)
    return HipEncoder(packed, device), max_batch, max_seconds
