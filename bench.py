"""Causal self-attention fwd+bwd throughput on one MI355X.

Workload (the headline): one GPT-2 124M training
micro-step's attention, 12 layers, each forward + backward at B=16, T=256,
H=12, head_dim=64, fp32, packed qkv [B, T, 3C]. One "step" runs the 12
forwards in layer order then the 12 backwards in reverse order, through the
C ABI (gpt_amd/libgpt_hip_attn.so), with every input already resident in HBM.

value = algorithmic FLOPs / GPU time, FLOPs = 12 * 7 * B * H * d * T * (T+1)
(QK^T and PV forward; S recompute, dP, dV, dK, dQ backward; causal pairs
including the diagonal; exp and masking not counted).

Also reported:
  roofline      the backward op (the dominant cost), timed live with HIP
                events on the stream its kernels are launched on
  cpu_baseline  the reference's own CPUBackend attention (compiled from its
                sources into oracle/_ref, -O3) on a bounded sample of the
                same workload, one thread, on this host

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "causal attn fwd+bwd TFLOP/s & % fp32 MFMA peak, GPT-2 124M shape, 1 GPU"
PEAK_FP32_MFMA_TFLOPS = 157.3
LAYERS, B, T, C, H = 12, 16, 256, 768, 12
D_HEAD = C // H
CONFIG_SEED = 1237  # 1234 + config index 3


def attn_flops(b, t, h, d, fwd=True, bwd=True):
    pairs = b * h * d * t * (t + 1)
    return (2 * pairs if fwd else 0) + (5 * pairs if bwd else 0)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-layers", type=int, default=4,
                    help="layers of the workload timed on the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    return ap.parse_args()


def cpu_baseline(layers: int):
    """Reference CPUBackend attention fwd+bwd on `layers` layers of the same
    workload (B=16, T=256), single thread; returns the cpu_baseline object."""
    import numpy as np

    from gpt_amd import synth
    from oracle import pyoracle

    impl, kind = ("ref_fast", "reference") if pyoracle.ref_available(fast=True) else ("oracle", "port")
    scales = synth.layer_scales(LAYERS, CONFIG_SEED)
    total = 0.0
    for layer in range(layers):
        seed = CONFIG_SEED + layer
        x = synth.qkv(B, T, C, seed, scale=float(scales[layer]))
        g = synth.grad_out(B, T, C, seed)
        t0 = time.perf_counter()
        y, lse = pyoracle.forward(x, H, impl)
        pyoracle.backward(x, y, lse, g, H, impl)
        total += time.perf_counter() - t0
        assert np.isfinite(y).all()
    flops = layers * attn_flops(B, T, H, D_HEAD)
    return {
        "value": round(flops / total / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": 1,
        "kind": kind,
        "sample": f"{layers} of the 12 layers (B=16,T=256,H=12,d=64) fwd+bwd, "
                  f"{total:.2f} s on 1 thread ({'oracle/_ref/libref_cpu_attn_fast.so, -O3' if kind == 'reference' else 'oracle/liboracle_attn.so'})",
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}): the attention op "
              f"shards per (batch, head) with no communication; run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import gpt_amd
    from gpt_amd import synth

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    scales = synth.layer_scales(LAYERS, CONFIG_SEED)

    # Per-layer buffers, as GPT::set_size lays them out (gpt.cpp:101-214).
    qkv, dout, y, lse, gx, Dc = [], [], [], [], [], []
    for layer in range(LAYERS):
        seed = CONFIG_SEED + layer
        qkv.append(torch.from_numpy(synth.qkv(B, T, C, seed, scale=float(scales[layer]))).to(dev))
        dout.append(torch.from_numpy(synth.grad_out(B, T, C, seed)).to(dev))
        y.append(torch.empty(B, T, C, device=dev))
        lse.append(torch.empty(B, T, H, device=dev))
        gx.append(torch.empty(B, T, 3 * C, device=dev))
        Dc.append(torch.empty(B, T, H, device=dev))
    torch.cuda.synchronize()

    def step(ev=None):
        for layer in range(LAYERS):
            if ev is not None:
                ev[0][layer].record(stream)
            gpt_amd.device_flash_attention_forward(y[layer], lse[layer], qkv[layer], B, T, C, H, stream)
            if ev is not None:
                ev[1][layer].record(stream)
        for layer in reversed(range(LAYERS)):
            if ev is not None:
                ev[2][layer].record(stream)
            gpt_amd.device_flash_attention_backward(gx[layer], Dc[layer], lse[layer], dout[layer], y[layer],
                                                    qkv[layer], B, T, C, H, stream)
            if ev is not None:
                ev[3][layer].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    mk = lambda: [torch.cuda.Event(enable_timing=True) for _ in range(LAYERS)]  # noqa: E731
    evs = [[mk() for _ in range(4)] for _ in range(args.steps)]
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for k in range(args.steps):
        step(evs[k])
    end.record(stream)
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    fwd_ms = [e[0][i].elapsed_time(e[1][i]) for e in evs for i in range(LAYERS)]
    bwd_ms = [e[2][i].elapsed_time(e[3][i]) for e in evs for i in range(LAYERS)]

    ms_per_step = total_ms / args.steps
    step_flops = LAYERS * attn_flops(B, T, H, D_HEAD)
    tflops = step_flops / (ms_per_step * 1e-3) / 1e12
    bwd_avg_ms = float(np.mean(bwd_ms))
    fwd_avg_ms = float(np.mean(fwd_ms))
    bwd_flops = attn_flops(B, T, H, D_HEAD, fwd=False)
    fwd_flops = attn_flops(B, T, H, D_HEAD, bwd=False)
    bwd_tf = bwd_flops / (bwd_avg_ms * 1e-3) / 1e12
    fwd_tf = fwd_flops / (fwd_avg_ms * 1e-3) / 1e12

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "attn_bwd_c3_traffic.json")
    if os.path.exists(tpath):
        traffic = json.load(open(tpath)).get("hbm_bytes_per_launch")

    out = {
        "metric": METRIC,
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (splitmix64 Box-Muller; Q/K/V ~ N(0,1)*U[0.5,2] per layer, dO ~ N(0,1e-3))",
        "config": {
            "workload": "GPT-2 124M attention micro-step: 12 layers x causal fwd+bwd, B=16 T=256 H=12 d=64",
            "layers": LAYERS, "batch": B, "seq_len": T, "heads": H, "head_dim": D_HEAD,
            "flops_per_step": step_flops,
        },
        "pct_fp32_mfma_peak": round(100 * tflops / PEAK_FP32_MFMA_TFLOPS, 2),
        "fwd": {"avg_ms": round(fwd_avg_ms, 5), "tflops": round(fwd_tf, 3)},
        "bwd": {"avg_ms": round(bwd_avg_ms, 5), "tflops": round(bwd_tf, 3)},
        "roofline": {
            "kernel": "attention backward op: bwd_prep_kernel + bwd_d64_kernel<2>",
            "bound": "mfma",
            "achieved": round(bwd_tf, 3),
            "peak": PEAK_FP32_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(bwd_tf / PEAK_FP32_MFMA_TFLOPS, 4),
            "traffic": traffic,
        },
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.cpu_layers)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
