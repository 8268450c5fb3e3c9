"""Benchmark: 8-layer relative_key attention on a 96 s chunk (BASELINE config c3).

One step = one HIP-graph replay of the 8 attention calls of one 96 s chunk
(B=1, H=16, L=4800, D=64, fp16 in/out, fp32 softmax), each layer with its own
seeded 73x64 table.  Layer l's q/k/v are the RMS-normalised residual stream
times a seeded fused QKV projection, and layer l's output is added to the
stream before layer l+1 (computed once, untimed: the inputs of every layer
are resident in HBM before timing starts).  Prints ONE JSON line on stdout.

    python bench.py [--steps K] [--warmup W] [--no-cpu-baseline] [--no-check]

Timing follows src/sidon_triton/engines.py:26-44 (warm-up, then events on
the stream the work runs on).  The CPU baseline is the fp32 torch
restatement of flexrel_triton.py:297-328 (oracle/flexrel_oracle.py) timed on
a bounded sample of the same workload on this host's cores.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "ms per 96 s chunk (8-layer attn, L=4800); TFLOP/s and % fp16 MFMA peak"
PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
B, H, L, D, LAYERS = 1, 16, 4800, 64, 8
TRAFFIC_FILE = ROOT / "profiles" / "flexrel_fwd_c3_traffic.md"
COPY_PROBE_BYTES = 256 << 20  # --copy-probe: one device copy of this many bytes


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def attention_flops(heads_total, lq, lk, dim=D):
    return float(heads_total) * (4.0 * lq * lk * dim + 2.0 * lq * 73 * dim)


def build_inputs(torch, seed=0):
    """Residual stream h0 [L, 1024] fp32, per-layer tables [73, 64] fp16 and
    fused QKV projections [3072, 1024] fp16 (seeded)."""
    gen = torch.Generator().manual_seed(seed)
    hid = H * D
    h0 = torch.randn(B * L, hid, generator=gen)
    rels = [(torch.randn(73, D, generator=gen) * 0.02).half() for _ in range(LAYERS)]
    projs = [(torch.randn(3 * hid, hid, generator=gen) / math.sqrt(hid)).half() for _ in range(LAYERS)]
    return h0, rels, projs


def qkv_of(torch, h, proj, out=None):
    """q | k | v source of a layer: RMS-normalised residual stream times the
    layer's projection (fp16 GEMM), [B*L, 3*H*64]; q/k/v come out ~N(0, 1)."""
    x = h * torch.rsqrt(h.square().mean(dim=1, keepdim=True) + 1e-6)
    return torch.matmul(x.half(), proj.t(), out=out)


def cpu_baseline(torch, qkv0, rel0, heads):
    """Time the fp32 torch restatement on `heads` heads of layer 0; scale to a chunk."""
    from oracle.flexrel_oracle import torch_core_chunked

    hid = H * D
    view = qkv0.view(B, L, 3, H, D)
    q, k, v = (view[:, :, i, :heads].permute(0, 2, 1, 3).float().contiguous() for i in range(3))
    rel = rel0.float()
    torch_core_chunked(q, k, v, rel)  # warm-up
    samples = []
    for _ in range(3):
        t0 = time.perf_counter()
        torch_core_chunked(q, k, v, rel)
        samples.append(time.perf_counter() - t0)
    per_head_layer_ms = statistics.median(samples) * 1e3 / heads
    return {
        "value": per_head_layer_ms * H * LAYERS,
        "unit": "ms per 96 s chunk",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"layer 0, {heads} of {H} heads, L=4800, fp32 torch (oracle.torch_core_chunked, "
                   f"512-row chunks); median of 3 after 1 warm-up = {statistics.median(samples):.3f} s; "
                   f"scaled x{H * LAYERS // heads} to 8 layers x 16 heads"),
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-heads", type=int, default=4)
    ap.add_argument("--no-check", action="store_true")
    ap.add_argument("--no-projections", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run 3 plain device copies of 256 MiB (calibrates the HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py runs on one GPU only: this build has no multi-GPU path "
              "(each 96 s chunk is independent; see DESIGN.md for how it would shard)", file=sys.stderr)
        return 2

    import torch

    if args.copy_probe:
        src = torch.empty(COPY_PROBE_BYTES // 2, dtype=torch.float16, device="cuda:0").normal_()
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy probe: 3 x {COPY_PROBE_BYTES} bytes read and written")
        return 0

    from __graft_entry__ import load_package

    sidon = load_package()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    shape = sidon._lib.launch_shape(B, H, L)
    log(f"launch shape at L={L}: {shape}; {sidon._lib.version()}")

    h0, rels, projs = build_inputs(torch)
    rels_d = [r.to(dev) for r in rels]
    projs_d = [p.to(dev) for p in projs]
    outs = [torch.empty(B * L, H * D, dtype=torch.float16, device=dev) for _ in range(LAYERS)]
    lens = torch.full((B,), L, dtype=torch.int32, device=dev)
    attn = sidon.encoder_attention.flexrel_attention
    # Untimed: every layer's q/k/v, resident in HBM before timing starts.
    with torch.no_grad():
        h = h0.to(dev)
        qkv = []
        for i in range(LAYERS):
            qkv.append(qkv_of(torch, h, projs_d[i]))
            attn(qkv[i], B, H, rels_d[i], lens, out=outs[i])
            h = h + outs[i].float()
    torch.cuda.synchronize()

    def enqueue_attention():
        for i in range(LAYERS):
            attn(qkv[i], B, H, rels_d[i], lens, out=outs[i])

    graphs = sidon.graphs.BucketGraphs()
    graph = graphs.capture(("attn", L), enqueue_attention)
    stream = torch.cuda.current_stream()
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    per_step = []
    start.record(stream)
    for _ in range(args.steps):
        graph.replay()
    end.record(stream)
    end.synchronize()
    total_ms = start.elapsed_time(end)
    # per-step samples for the median (separate pass, same graph)
    for _ in range(min(args.steps, 30)):
        s0 = torch.cuda.Event(enable_timing=True)
        s1 = torch.cuda.Event(enable_timing=True)
        s0.record(stream)
        graph.replay()
        s1.record(stream)
        s1.synchronize()
        per_step.append(s0.elapsed_time(s1))
    torch.cuda.synchronize()
    ms_per_step = total_ms / args.steps
    launch_us = ms_per_step * 1e3 / LAYERS
    flops_launch = attention_flops(B * H, L, L)
    achieved = flops_launch / (launch_us * 1e-6) / 1e12

    extra = {"median_ms": statistics.median(per_step), "min_ms": min(per_step),
             "kernel_avg_us": launch_us, "tflops": achieved,
             "pct_fp16_peak": 100.0 * achieved / PEAK_TFLOPS, "launch": shape}

    if not args.no_projections:
        # Secondary: the same 8 layers with the residual update and the next
        # layer's projection between them (one graph).
        h_d = h0.to(dev)
        h_work = torch.empty_like(h_d)

        def enqueue_chain():
            h_work.copy_(h_d)
            for i in range(LAYERS):
                if i:
                    qkv_of(torch, h_work, projs_d[i], out=qkv[i])
                attn(qkv[i], B, H, rels_d[i], lens, out=outs[i])
                h_work.add_(outs[i])
        chain = graphs.capture(("chain", L), enqueue_chain)
        for _ in range(3):
            chain.replay()
        torch.cuda.synchronize()
        c0 = torch.cuda.Event(enable_timing=True)
        c1 = torch.cuda.Event(enable_timing=True)
        c0.record(stream)
        for _ in range(10):
            chain.replay()
        c1.record(stream)
        c1.synchronize()
        extra["with_projections_ms"] = c0.elapsed_time(c1) / 10

    if not args.no_check:
        from oracle.flexrel_oracle import errors, flexrel_reference
        heads = [0, 15]
        for layer in (0, LAYERS - 1):
            view = qkv[layer].view(B, L, 3, H, D).float().cpu().numpy()
            q, k, v = (view[:, :, i, heads].transpose(0, 2, 1, 3) for i in range(3))
            ref = flexrel_reference(q, k, v, rels[layer].float().numpy())
            got = outs[layer].view(B, L, H, D)[:, :, heads].permute(0, 2, 1, 3).float().cpu().numpy()
            err = errors(ref, got)
            extra[f"check_layer{layer}_heads_0_15"] = err
            log(f"parity (layer {layer}, heads {heads}): {err}")

    traffic = None
    if TRAFFIC_FILE.exists():
        import re
        m = re.search(r"HBM bytes per launch:\s*([0-9.eE+]+)", TRAFFIC_FILE.read_text())
        traffic = float(m.group(1)) if m else None

    result = {
        "metric": METRIC,
        "value": ms_per_step,
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded residual stream ~N(0,1) -> RMS norm -> seeded fused QKV projection per layer, so q/k/v ~N(0,1); tables ~N(0,0.02))",
        "config": {"workload": "c3: 8 layers of relative_key attention, one 96 s chunk, graph replay",
                   "batch": B, "heads": H, "seq_len": L, "head_dim": D, "layers": LAYERS,
                   "valid_len": L, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_TFLOPS, "traffic": traffic},
    }
    result.update(extra)
    if not args.no_cpu_baseline:
        log("timing the CPU baseline ...")
        result["cpu_baseline"] = cpu_baseline(torch, qkv[0].cpu(), rels[0], args.cpu_heads)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
