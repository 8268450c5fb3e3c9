"""The fused feed-forward input projection (GEMM + bias + SiLU, csrc/gemm.hip;
hipBLASLt with the bias and SiLU in its epilogue, csrc/blaslt.hip) against
float32 torch and against hipBLASLt followed by the in-place SiLU, and the
residual GEMM (csrc/gemm_res.hip) (needs an MI355X)."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _inputs(m, n, k, seed, ldx=None):
    gen = torch.Generator().manual_seed(seed)
    ldx = k if ldx is None else ldx
    xs = torch.randn(m, ldx, generator=gen).half().to(DEV)
    w = (torch.randn(n, k, generator=gen) / k ** 0.5).half().to(DEV)
    b = (torch.randn(n, generator=gen) * 0.1).half().to(DEV)
    return xs[:, :k], w, b


def _reference(x, w, b, act):
    """fp32 sums, bias added, rounded to fp16 (as addmm stores it), SiLU in
    fp32, rounded to fp16."""
    h = x.float() @ w.float().t()
    if b is not None:
        h = h + b.float()
    h = h.half().float()
    return (torch.nn.functional.silu(h) if act else h).half()


@pytest.mark.parametrize("m,n,k,bias,act,ldx", [
    (4800, 4096, 1024, True, True, None),
    (1000, 512, 256, True, True, None),
    (333, 256, 64, False, False, None),
    (1, 256, 128, True, True, None),
    (650, 768, 128, True, True, 192),
])
def test_linear_silu_matches_fp32(sidon, m, n, k, bias, act, ldx):
    x, w, b = _inputs(m, n, k, seed=m + n + k, ldx=ldx)
    b = b if bias else None
    got = sidon.conformer.linear_silu(x, w, b, act=act)
    ref = _reference(x, w, b, act)
    torch.cuda.synchronize()
    err = (got.float() - ref.float()).abs()
    # the fp32 sums differ from torch's only in summation order: at most one
    # fp16 rounding step apart after the final rounding
    tol = 2e-3 + 2e-3 * ref.float().abs()
    assert torch.isfinite(got.float()).all()
    assert (err <= tol).all(), float(err.max())
    snr = 10 * torch.log10(ref.float().pow(2).sum() / (got.float() - ref.float()).pow(2).sum().clamp_min(1e-30))
    assert snr > 60, float(snr)


def test_linear_silu_matches_library_gemm_then_silu(sidon):
    """Same shape as the encoder's FFN input at a 96 s chunk; hipBLASLt's GEMM
    plus the in-place SiLU agree to within one fp16 rounding (measured: bit for bit)."""
    x, w, b = _inputs(4800, 4096, 1024, seed=7)
    fused = sidon.conformer.linear_silu(x, w, b)
    twostep = sidon.conformer.silu_(torch.addmm(b, x, w.t()))
    torch.cuda.synchronize()
    diff = (fused.float() - twostep.float()).abs()
    print(f"fused vs two-step: max {float(diff.max()):.3e}, differing {float((diff > 0).float().mean()):.4f}")
    assert torch.allclose(fused.float(), twostep.float(), atol=2e-3, rtol=2e-3)


def test_linear_silu_out_buffer_and_strides(sidon):
    """A strided output view: untouched columns stay untouched."""
    x, w, b = _inputs(500, 256, 128, seed=11)
    big = torch.full((500, 512), 5.0, dtype=torch.float16, device=DEV)
    out = big[:, 128:384]
    sidon.conformer.linear_silu(x, w, b, out=out)
    torch.cuda.synchronize()
    assert torch.all(big[:, :128] == 5.0) and torch.all(big[:, 384:] == 5.0)
    assert torch.allclose(out.float(), _reference(x, w, b, True).float(), atol=2e-3, rtol=2e-3)


def _reference_lt(x, w, b, act):
    """fp32 sums, bias added, SiLU in fp32, one rounding to fp16."""
    h = x.float() @ w.float().t()
    if b is not None:
        h = h + b.float()
    return (torch.nn.functional.silu(h) if act else h).half()


@pytest.mark.parametrize("m,n,k,bias,act,ldx", [
    (750, 4096, 1024, True, True, None),
    (1500, 4096, 1024, True, True, None),
    (333, 256, 64, False, False, None),
    (1, 256, 128, True, True, None),
    (650, 768, 128, True, True, 192),
    (7, 96, 40, True, True, None),
])
def test_linear_silu_lt_matches_fp32(sidon, m, n, k, bias, act, ldx):
    """hipBLASLt with the bias and SiLU in its epilogue against float32 torch,
    and five more calls bit-identical to the first."""
    x, w, b = _inputs(m, n, k, seed=m + n + k + 1, ldx=ldx)
    b = b if bias else None
    got = sidon.conformer.linear_silu_lt(x, w, b, act=act)
    ref = _reference_lt(x, w, b, act)
    torch.cuda.synchronize()
    err = (got.float() - ref.float()).abs()
    tol = 2e-3 + 2e-3 * ref.float().abs()
    assert torch.isfinite(got.float()).all()
    assert (err <= tol).all(), float(err.max())
    snr = 10 * torch.log10(ref.float().pow(2).sum() / (got.float() - ref.float()).pow(2).sum().clamp_min(1e-30))
    assert snr > 60, float(snr)
    for _ in range(5):
        again = sidon.conformer.linear_silu_lt(x, w, b, act=act)
        assert torch.equal(again, got)


def test_linear_silu_lt_out_buffer_and_strides(sidon):
    """A strided output view: untouched columns stay untouched."""
    x, w, b = _inputs(500, 256, 128, seed=12)
    big = torch.full((500, 512), 5.0, dtype=torch.float16, device=DEV)
    out = big[:, 128:384]
    sidon.conformer.linear_silu_lt(x, w, b, out=out)
    torch.cuda.synchronize()
    assert torch.all(big[:, :128] == 5.0) and torch.all(big[:, 384:] == 5.0)
    assert torch.allclose(out.float(), _reference_lt(x, w, b, True).float(), atol=2e-3, rtol=2e-3)


def test_linear_silu_lt_agrees_with_fused_kernel(sidon):
    """At the encoder's 15 s shape the epilogue SiLU (one rounding) and this
    library's kernel (SiLU of the fp16-rounded sum) differ by at most about
    one fp16 rounding step."""
    x, w, b = _inputs(750, 4096, 1024, seed=17)
    lt = sidon.conformer.linear_silu_lt(x, w, b)
    own = sidon.conformer.linear_silu(x, w, b)
    torch.cuda.synchronize()
    diff = (lt.float() - own.float()).abs()
    print(f"epilogue vs fused kernel: max {float(diff.max()):.3e}, differing {float((diff > 0).float().mean()):.4f}")
    assert torch.allclose(lt.float(), own.float(), atol=2e-3, rtol=2e-3)


def test_linear_silu_lt_graph_replays_match_eager(sidon):
    """Captured into a HIP graph (after an eager call of the same problem) and
    replayed three times, with eager work and synchronisations between the
    replays: every replay equals the eager call."""
    x, w, b = _inputs(1500, 4096, 1024, seed=19)
    out = torch.empty(1500, 4096, dtype=torch.float16, device=DEV)
    sidon.conformer.linear_silu_lt(x, w, b, out=out)
    torch.cuda.synchronize()
    eager = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        sidon.conformer.linear_silu_lt(x, w, b, out=out)
    for rep in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), rep
        _ = (x.float() * 2).sum().item()  # unrelated eager work


def test_encoder_fused_and_library_ffn_agree(sidon):
    """The whole encoder at Sidon's full width (8 layers, L=750) with the fused
    FFN input kernel forced on and forced off, and the fused one against the
    fp32 torch oracle."""
    import bench
    from oracle.encoder_oracle import encoder_reference
    from oracle.flexrel_oracle import errors

    weights = bench.encoder_model_weights(torch, seed=7, device=DEV)
    packed = sidon.encoder.pack_weights(weights)
    gen = torch.Generator().manual_seed(750)
    feats = torch.randn(1, 750, 160, generator=gen).to(DEV)
    frames = torch.tensor([750], dtype=torch.int32, device=DEV)
    on = sidon.encoder.HipEncoder(packed, DEV, fused_ffn=True)(feats, frames)
    off = sidon.encoder.HipEncoder(packed, DEV, fused_ffn=False)(feats, frames)
    lt = sidon.encoder.HipEncoder(packed, DEV, fused_ffn="lt")(feats, frames)
    default = sidon.encoder.HipEncoder(packed, DEV)(feats, frames)
    torch.cuda.synchronize()
    assert torch.equal(default, lt)  # at L = 750 the per-call choice is the epilogue path
    agree = errors(off[0].double().cpu().numpy(), on[0].double().cpu().numpy())
    want = encoder_reference(feats, weights, [750], dtype=torch.float32)
    err = errors(want[0].double().cpu().numpy(), on[0].double().cpu().numpy())
    # The epilogue path rounds the SiLU input differently (no fp16 rounding of
    # the biased sum), so it is held to the oracle, not to the other paths.
    err_lt = errors(want[0].double().cpu().numpy(), lt[0].double().cpu().numpy())
    err_off = errors(want[0].double().cpu().numpy(), off[0].double().cpu().numpy())
    print("fused vs library FFN input:", agree, "vs fp32 oracle: fused", err, "epilogue", err_lt, "addmm + SiLU",
          err_off)
    assert torch.isfinite(on).all() and torch.isfinite(lt).all()
    assert agree["snr_db"] > 80, agree
    assert err["snr_db"] > 58 and err["max_abs"] < 0.02 * want.abs().max().item(), err
    assert err_lt["snr_db"] > 58 and err_lt["max_abs"] < 0.02 * want.abs().max().item(), err_lt


def test_linear_silu_graph_replays_match_eager(sidon):
    """Captured into a HIP graph and replayed three times, with eager work and
    synchronisations between the replays: every replay equals the eager call."""
    x, w, b = _inputs(4800, 4096, 1024, seed=13)
    out = torch.empty(4800, 4096, dtype=torch.float16, device=DEV)
    sidon.conformer.linear_silu(x, w, b, out=out)
    torch.cuda.synchronize()
    eager = out.clone()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        sidon.conformer.linear_silu(x, w, b, out=out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        sidon.conformer.linear_silu(x, w, b, out=out)
    for rep in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), rep
        _ = (x.float() * 2).sum().item()  # unrelated eager work


def test_runtime_full_chunk_graph_replays_match_eager(sidon):
    """The encoder runtime at a full 96 s chunk (the fused FFN input kernel's
    shape): graph replays, with eager work between them, equal eager calls."""
    import bench

    weights = bench.encoder_model_weights(torch, seed=5, device=DEV)
    enc = sidon.encoder.HipEncoder(sidon.encoder.pack_weights(weights), DEV)
    assert sidon.conformer.linear_silu_preferred(4800, enc.inter, enc.hidden, DEV)
    rt = sidon.runtime.EncoderRuntime(enc, max_batch=1, max_seconds=96, max_graphs=2)
    gen = torch.Generator().manual_seed(6)
    for rep, frames in enumerate((4800, 4731, 4800)):
        feats = torch.randn(1, 4800, 160, generator=gen)
        got = rt.run(feats, [frames]).clone()
        want = enc(feats.to(DEV), torch.tensor([frames], dtype=torch.int32, device=DEV))
        torch.cuda.synchronize()
        assert torch.equal(got[0, :frames], want[0, :frames]), rep
        _ = (want * 2).sum().item()  # unrelated eager work between replays
    assert len(rt.graphs) == 1


# ---- the residual projection into the fp32 stream (csrc/gemm_res.hip) ----

@pytest.mark.parametrize("m,n,k,ldx,ldy", [
    (750, 1024, 4096, None, None),
    (750, 1024, 1024, None, None),
    (1500, 1024, 1024, None, None),
    (63, 64, 128, None, None),
    (1, 128, 256, None, None),
    (333, 192, 384, 400, 200),
])
def test_residual_gemm_matches_fp32(sidon, m, n, k, ldx, ldy):
    """x += a . w^T against float64 on the CPU from the same fp16 inputs and
    fp32 stream; columns past N and rows past M of a wider / taller stream
    buffer are left untouched; two calls from the same state give the same
    bits."""
    gen = torch.Generator().manual_seed(m + n + k)
    ldx = k if ldx is None else ldx
    ldy = n if ldy is None else ldy
    a_full = torch.randn(m, ldx, generator=gen).half()
    a = a_full[:, :k]
    w = (torch.randn(n, k, generator=gen) / k ** 0.5).half()
    x0 = torch.randn(m + 3, ldy, generator=gen)
    ref = x0.double().clone()
    ref[:m, :n] += a.double() @ w.double().t()
    buf = x0.to(DEV)
    x = buf[:m, :n]
    a_d, w_d = a_full.to(DEV)[:, :k], w.to(DEV)   # a keeps its row stride ldx on the device
    assert a_d.stride(0) == ldx
    got = sidon.conformer.residual_gemm(x, a_d, w_d)
    assert got.data_ptr() == x.data_ptr()
    out = buf.cpu()
    assert torch.equal(out[m:], x0[m:]) and torch.equal(out[:m, n:], x0[:m, n:])
    err = (out[:m, :n].double() - ref[:m, :n]).abs()
    # fp32 sums of k products: a few fp32 roundings of the running sum
    tol = 1e-5 * (1 + ref[:m, :n].abs()) * max(1.0, (k / 1024) ** 0.5)
    assert (err <= tol).all(), float(err.max())
    again = x0.to(DEV)
    sidon.conformer.residual_gemm(again[:m, :n], a_d, w_d)
    assert torch.equal(again.cpu(), out)


def test_residual_gemm_matches_addmm(sidon):
    """The encoder's feed-forward output at a 15 s chunk against the
    torch.addmm(x, a, w.t(), out_dtype=float32) it replaces: the same fp32
    sums in another order."""
    gen = torch.Generator().manual_seed(5)
    a = torch.randn(750, 4096, generator=gen).half().to(DEV)
    w = (torch.randn(1024, 4096, generator=gen) / 64).half().to(DEV)
    x = torch.randn(750, 1024, generator=gen).to(DEV)
    ref = torch.addmm(x, a, w.t(), out_dtype=torch.float32)
    got = sidon.conformer.residual_gemm(x.clone(), a, w)
    torch.cuda.synchronize()
    assert float((got - ref).abs().max()) <= 1e-4
