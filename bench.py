"""Benchmark of the MI355X FP32 attention path (one GPU).

A step is one launch of the 32-wide flash forward (attention_fp32_forward_flash_ex, causal) over BASELINE config 2:
24 independent sequences (B2 x H12) x 1024 tokens x d=32, Q/K/V iid N(0,1) (seeds 101-103), mask all ones.
The backward of the same batch (config 3) is timed the same way and reported beside it.

FLOP accounting:
  * value / tflops_*_convention: the reference's convention, 4*B*H*Lq*Lk*d forward and 8*... backward, regardless of
    the mask (ROCmKernels.Benchmark/src/AttentionBenchmarks.cpp:141-142,197);
  * roofline.achieved / tflops_*_visited: only (query, key) pairs inside the causal mask (L(L+1)/2 per sequence),
    4*d FLOPs per pair forward and 8*d backward -- the work the kernels actually have to do.
Timing: W warm-up launches, then K launches bracketed by HIP events on the launch stream, with device synchronisation
on both sides; inputs are resident in HBM before the timed region.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "TFLOP/s + ms/launch, FP32 flash attn fwd/bwd d=32 24x1024 on 1 MI355X"
PEAK_FP32_MFMA_TFLOPS = 157.3  # MI355X dense FP32 matrix peak (AMD public specification)
BATCH, HEADS, LENGTH, WIDTH = 2, 12, 1024, 32


def visited_pairs(length):
    return length * (length + 1) // 2


def time_launches(launch, steps, warmup, stream):
    import torch

    for _ in range(warmup):
        launch()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        launch()
    stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps  # ms per launch


def cpu_baseline(seconds):
    """The CPU oracle (a C port of the reference's CPU reference) timed on this host's cores on the same forward."""
    import numpy as np

    import oracle
    from rocmkernels_amd import inputs

    shape = (BATCH, HEADS, LENGTH, WIDTH)
    q, k, v = (inputs.normal(seed, shape) for seed in (101, 102, 103))
    mask = np.ones((BATCH, LENGTH), np.uint8)
    threads = min(os.cpu_count() or 1, 16)
    runs, elapsed = 0, 0.0
    while elapsed < seconds or runs == 0:
        begin = time.perf_counter()
        oracle.attention(q, k, v, mask, causal=True, threads=threads)
        elapsed += time.perf_counter() - begin
        runs += 1
    per_run = elapsed / runs
    convention = 4.0 * BATCH * HEADS * LENGTH * LENGTH * WIDTH
    return {
        "value": round(convention / per_run / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"full config-2 causal forward (24 x 1024 x 32) on the C oracle, {runs} run(s), {per_run * 1e3:.1f} ms/run",
    }


def load_traffic():
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as handle:
        data = json.load(handle)
    return data.get("attention_forward_kernel<32,false,true> config2", {}).get("hbm_bytes_per_launch")


def main():
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=500)
    parser.add_argument("--warmup", type=int, default=50)
    parser.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample length (0 skips it)")
    parser.add_argument("--no-backward", action="store_true")
    args = parser.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (every sequence is independent; "
              "sharding B*H across GPUs needs no communication). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    from rocmkernels_amd import attention, inputs

    if not torch.cuda.is_available():
        raise RuntimeError("bench.py needs a GPU")
    device = torch.device("cuda:0")
    shape = (BATCH, HEADS, LENGTH, WIDTH)
    q, k, v, du = (torch.from_numpy(inputs.normal(seed, shape)).to(device) for seed in (101, 102, 103, 104))
    mask = torch.ones((BATCH, LENGTH), dtype=torch.uint8, device=device)
    out = torch.empty(shape, device=device)
    lse = torch.empty((BATCH, HEADS, LENGTH, 2), device=device)
    grads = (torch.empty(shape, device=device), torch.empty(shape, device=device), torch.empty(shape, device=device),
             torch.empty((BATCH, HEADS, LENGTH), device=device))
    stream = torch.cuda.current_stream()

    def forward():
        attention.forward(q, k, v, mask, causal=True, output=out, lse=lse, stream=stream)

    def backward():
        attention.backward(q, k, v, mask, out, lse, du, causal=True, grads=grads, stream=stream)

    ms_fwd = time_launches(forward, args.steps, args.warmup, stream)
    convention_fwd = 4.0 * BATCH * HEADS * LENGTH * LENGTH * WIDTH
    visited_fwd = 4.0 * BATCH * HEADS * visited_pairs(LENGTH) * WIDTH
    tflops_conv = convention_fwd / (ms_fwd * 1e-3) / 1e12
    tflops_visited = visited_fwd / (ms_fwd * 1e-3) / 1e12
    result = {
        "metric": METRIC,
        "value": round(tflops_conv, 4),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_fwd, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "config 2: 32-wide flash forward, causal, B2 x H12 x L1024 x d32 (24 sequences)",
                   "batch": BATCH, "heads": HEADS, "seq_len": LENGTH, "head_dim": WIDTH, "mask": "causal",
                   "flop_basis_of_value": "reference convention 4*B*H*L^2*d"},
        "tflops_fwd_convention": round(tflops_conv, 4),
        "tflops_fwd_visited": round(tflops_visited, 4),
        "roofline": {"bound": "mfma", "achieved": round(tflops_visited, 4), "peak": PEAK_FP32_MFMA_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops_visited / PEAK_FP32_MFMA_TFLOPS, 4),
                     "traffic": load_traffic(), "kernel": "attention_forward_kernel<32,false,true>",
                     "flops_per_launch": visited_fwd},
    }
    if not args.no_backward:
        forward()
        ms_bwd = time_launches(backward, args.steps, args.warmup, stream)
        convention_bwd = 8.0 * BATCH * HEADS * LENGTH * LENGTH * WIDTH
        visited_bwd = 8.0 * BATCH * HEADS * visited_pairs(LENGTH) * WIDTH
        result["backward"] = {
            "workload": "config 3: backward of config 2 (delta + dQ kernel, then dK/dV kernel)",
            "ms_per_launch": round(ms_bwd, 6),
            "tflops_convention": round(convention_bwd / (ms_bwd * 1e-3) / 1e12, 4),
            "tflops_visited": round(visited_bwd / (ms_bwd * 1e-3) / 1e12, 4),
            "frac_of_fp32_mfma_peak_visited": round(visited_bwd / (ms_bwd * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4),
        }
    if args.cpu_seconds > 0:
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
