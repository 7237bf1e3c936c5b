#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-expert hot path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Workloads:
  * dequant: kernel (a) over one Qwen3-30B-A3B MoE layer's expert weights held
    as one flat 4-bit arena (gate_up [128,1536,2048] + down [128,2048,768] =
    603,979,776 elements, 1,528,823,808 algorithmic bytes per launch).
Synthetic data: weights ~ N(0, 0.02) quantized on the GPU with the reference's
scheme; inputs are resident in HBM before timing starts.  Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

METRIC = "dequant GB/s (% HBM peak); 4-bit MoE layer fwd+bwd tokens/sec, % MFMA peak"
HBM_PEAK_GBS = 8000.0            # MI355X HBM3E, 8 TB/s
MFMA_BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA

QWEN = dict(E=128, H=2048, I=768, k=8, T=4096)
LAYER_ELEMS = QWEN["E"] * 2 * QWEN["I"] * QWEN["H"] + QWEN["E"] * QWEN["H"] * QWEN["I"]  # 603,979,776
LAYER_GROUPS = LAYER_ELEMS // 128
DEQUANT_BYTES_PER_ELEM = 0.5 + 4.0 / 128 + 2.0            # codes + (scale, zero) + fp16/bf16 out


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class _Timer:
    """HIP-event timing on torch's current stream (the stream the kernels use)."""

    def __init__(self):
        self.a = torch.cuda.Event(enable_timing=True)
        self.b = torch.cuda.Event(enable_timing=True)

    def __enter__(self):
        torch.cuda.synchronize()
        self.a.record()
        return self

    def __exit__(self, *exc):
        self.b.record()
        torch.cuda.synchronize()
        self.ms = self.a.elapsed_time(self.b)


def bench_dequant(dev, steps: int, warmup: int, out_dtype=torch.bfloat16) -> dict:
    from usaf_amd import quantization as Q
    torch.manual_seed(1234)
    # quantize the layer in 8 slabs to bound the transient fp16 footprint
    packed = torch.empty((LAYER_GROUPS, 64), dtype=torch.int8, device=dev)
    scale = torch.empty(LAYER_GROUPS, dtype=torch.float16, device=dev)
    zero = torch.empty(LAYER_GROUPS, dtype=torch.float16, device=dev)
    slab = LAYER_GROUPS // 8
    for i in range(8):
        w = (torch.randn(slab * 128, device=dev) * 0.02).half()
        p, s, z, _ = Q.quantize_4bit(w, 128)
        packed[i * slab:(i + 1) * slab].copy_(p)
        scale[i * slab:(i + 1) * slab].copy_(s)
        zero[i * slab:(i + 1) * slab].copy_(z)
        del w, p, s, z
    out = torch.empty(LAYER_ELEMS, dtype=out_dtype, device=dev)
    shape = torch.Size([LAYER_ELEMS])
    for _ in range(warmup):
        Q.dequantize_4bit(packed, scale, zero, shape, 128, out_dtype=out_dtype, out=out)
    with _Timer() as t:
        for _ in range(steps):
            Q.dequantize_4bit(packed, scale, zero, shape, 128, out_dtype=out_dtype, out=out)
    ms = t.ms / steps
    nbytes = LAYER_ELEMS * DEQUANT_BYTES_PER_ELEM
    gbs = nbytes / (ms * 1e-3) / 1e9
    return dict(ms_per_launch=ms, gbs=gbs, bytes_per_launch=int(nbytes), elems=LAYER_ELEMS,
                out_dtype=str(out_dtype).replace("torch.", ""))


def cpu_baseline_dequant(max_seconds: float = 20.0) -> dict:
    """The reference's CPU dequant op sequence (oracle/codec_torch.py, torch CPU,
    all host cores) on a bounded sample: 16 of 128 experts of the layer."""
    from oracle.codec_torch import dequant_opseq
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(1234)
    parts = [(16 * 2 * QWEN["I"] * QWEN["H"]), (16 * QWEN["H"] * QWEN["I"])]  # 16 experts' gate_up + down
    data = []
    for n in parts:
        G = n // 128
        data.append((torch.randint(-128, 128, (G, 64), dtype=torch.int8, generator=g),
                     (torch.rand(G, generator=g) * 1e-2).half(), (torch.randn(G, generator=g) * 0.05).half(),
                     torch.Size([n])))
    elems = sum(parts)
    reps, t0 = 0, time.perf_counter()
    while True:
        for q, s, z, shp in data:
            dequant_opseq(q, s, z, shp, 128)
        reps += 1
        dt = time.perf_counter() - t0
        if dt > max_seconds or reps >= 50:
            break
    gbs = reps * elems * DEQUANT_BYTES_PER_ELEM / dt / 1e9
    return dict(value=round(gbs, 3), unit="GB/s", cores=threads, kind="port",
                sample=f"torch-CPU restatement of quantization.py:107-132 on 16 of 128 experts of one Qwen3 "
                       f"MoE layer ({elems:,} elements) x {reps} reps, {dt:.1f} s, fp16 output")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the hot path is benchmarked at one GPU's shard shape); run with --gpus 1.", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    from usaf_amd import _native
    _native.load()

    _log("dequant: one Qwen3 MoE layer (603,979,776 elements) -> bf16")
    dq = bench_dequant(dev, args.steps, args.warmup)
    _log(f"dequant: {dq['ms_per_launch']:.3f} ms/launch, {dq['gbs']:.1f} GB/s")
    cpu = None
    if not args.no_cpu_baseline:
        _log("cpu baseline: torch-CPU dequant sample")
        cpu = cpu_baseline_dequant()
        _log(f"cpu baseline: {cpu['value']} GB/s on {cpu['cores']} threads")

    line = {
        "metric": METRIC,
        "value": round(dq["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dq["ms_per_launch"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4->bf16",
        "data": "synthetic: expert weights ~N(0,0.02) quantized to 4-bit on the GPU (reference scheme, group 128)",
        "config": {"workload": "dequant one Qwen3-30B-A3B MoE layer (gate_up+down, 128 experts) as one 4-bit arena",
                   "elements": LAYER_ELEMS, "group_size": 128},
        "roofline": {"bound": "hbm", "achieved": round(dq["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dq["gbs"] / HBM_PEAK_GBS, 4), "traffic": None},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
