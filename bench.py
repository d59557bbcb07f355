"""Benchmark of the MI355X FP32 attention path (one GPU).

Default run (the driver's contract): a step is one launch of the 32-wide flash forward
(attention_fp32_forward_flash_ex, causal) over BASELINE config 2: 24 independent sequences (B2 x H12) x 1024 tokens
x d=32, Q/K/V iid N(0,1) (seeds 101-103), mask all ones. The backward of the same batch (config 3) is timed the same
way and reported beside it, and the CPU oracle is timed on the host for the cpu_baseline object.
``--config N`` (1-5) times BASELINE config N instead (forward and backward).

FLOP accounting:
  * value / tflops_*_convention: the reference's convention, 4*B*H*Lq*Lk*d forward and 8*... backward, regardless of
    the mask (ROCmKernels.Benchmark/src/AttentionBenchmarks.cpp:141-142,197);
  * roofline.achieved / tflops_*_visited: only (query, key) pairs inside the mask, 4*d FLOPs per pair forward and
    8*d backward -- the work the kernels actually have to do.
Timing: W warm-up launches, then K launches captured in one HIP graph and replayed once between two HIP events on
the launch stream (device synchronisation on both sides), so host launch gaps do not count; the same K launches
issued eagerly from Python through ctypes are timed too (``ms_per_launch_eager``). Inputs are resident in HBM.
Before each timed region the same launches run untimed for at least ``--settle-seconds`` of continuous load: under
sustained work the MI355X shader clock rises from about 2.0 GHz to about 2.34 GHz within the first ~20 ms (measured
with s_memtime against s_memrealtime inside the forward kernel; cycles per tile are unchanged), so without it the
first timed launches would run at the lower clock. The timed launches do the full work of every step.
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

# (batch, heads, length, width, radius, causal, padded key lengths)
CONFIGS = {
    1: dict(batch=4, heads=1, length=256, width=32, radius=-1, padding=False,
            workload="config 1: 32-wide forward, causal, B4 x H1 x L256 x d32"),
    2: dict(batch=2, heads=12, length=1024, width=32, radius=-1, padding=False,
            workload="config 2: 32-wide flash forward, causal, B2 x H12 x L1024 x d32 (24 sequences)"),
    3: dict(batch=2, heads=12, length=1024, width=32, radius=-1, padding=False,
            workload="config 3: 32-wide forward+backward, causal, B2 x H12 x L1024 x d32"),
    4: dict(batch=32, heads=1, length=2048, width=64, radius=-1, padding=True,
            workload="config 4: 64-wide fwd+bwd, causal + key padding (valid length U[1024,2048]), B32 x L2048 x d64"),
    5: dict(batch=16, heads=1, length=8192, width=64, radius=256, padding=False,
            workload="config 5: 64-wide local radius 256, causal in band, fwd+bwd, B16 x L8192 x d64"),
}


def key_lengths(cfg):
    import numpy as np

    from rocmkernels_amd import inputs

    if cfg["padding"]:
        return inputs.uniform_int(105, cfg["batch"], cfg["length"] // 2, cfg["length"])
    return np.full(cfg["batch"], cfg["length"], dtype=np.int64)


def visited_pairs(cfg, lengths):
    """(query, key) pairs inside the causal mask, the radius band and the key padding, summed over the batch:
    query q sees keys max(0, q - radius) .. min(q, valid - 1)."""
    import numpy as np

    q = np.arange(cfg["length"])
    lo = np.maximum(0, q - cfg["radius"]) if cfg["radius"] >= 0 else np.zeros_like(q)
    total = sum(int(np.maximum(np.minimum(q, int(valid) - 1) - lo + 1, 0).sum()) for valid in lengths)
    return total * cfg["heads"]


def make_inputs(cfg, device):
    import numpy as np
    import torch

    from rocmkernels_amd import inputs

    shape = (cfg["batch"], cfg["heads"], cfg["length"], cfg["width"])
    q, k, v, du = (torch.from_numpy(inputs.normal(seed, shape)).to(device) for seed in (101, 102, 103, 104))
    lengths = key_lengths(cfg)
    mask = torch.from_numpy((np.arange(cfg["length"])[None, :] < lengths[:, None]).astype(np.uint8)).to(device)
    return q, k, v, du, mask, lengths


SETTLE_SECONDS = 0.25


def settle(launch, per_check=20):
    """Untimed launches for at least SETTLE_SECONDS of continuous load (`per_check` launches between two looks at
    the clock), so that the timed launches run at the sustained shader clock rather than the one of an idle GPU."""
    import torch

    begin = time.perf_counter()
    while time.perf_counter() - begin < SETTLE_SECONDS:
        for _ in range(per_check):
            launch()
        torch.cuda.synchronize()


def time_eager(launch, steps, warmup, stream):
    import torch

    for _ in range(warmup):
        launch()
    settle(launch)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        launch()
    stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def time_graph(launch, steps, results, exact=True):
    """K launches captured into one graph; returns ms per launch of one replay. Checks every replay output
    against the eager result (``results`` are the eager outputs of the same launch): bit for bit, or, when
    ``exact`` is false (atomically accumulated outputs), within 1e-5 of the largest magnitude."""
    import torch

    reference = [r.clone() for r in results]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(steps):
            launch()
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    settle(graph.replay, per_check=1)
    times = []
    for _ in range(3):
        for r in results:
            r.fill_(float("nan"))
        torch.cuda.synchronize()
        start.record(stream)
        graph.replay()
        stop.record(stream)
        torch.cuda.synchronize()
        times.append(start.elapsed_time(stop) / steps)
        for r, ref in zip(results, reference):
            if exact and not torch.equal(r.view(torch.int32), ref.view(torch.int32)):
                raise RuntimeError("graph replay result differs bitwise from the eager launch")
            if not exact and float((r - ref).abs().max()) > 1e-5 * max(float(ref.abs().max()), 1e-30):
                raise RuntimeError("graph replay result differs from the eager launch")
    return min(times)


def measure_rotary(cfg, steps, warmup):
    """rotary_fp32 on the config's Q and K (32-wide heads only), token-major layout as the reference's bench
    (RotaryBenchmarks.cpp:52-53): HBM-bound, reported against the 8 TB/s HBM peak with
    the algorithmic bytes (Q, K read; oq, ok written; cos/sin tables read once)."""
    import torch

    from rocmkernels_amd import attention, inputs

    if cfg["width"] != 32:
        return None
    device = torch.device("cuda:0")
    batch, heads, length = cfg["batch"], cfg["heads"], cfg["length"]
    q, k = (torch.from_numpy(inputs.normal(seed, (batch, length, heads, 32))).to(device).permute(0, 2, 1, 3) for seed in (201, 202))
    cos, sin = (torch.from_numpy(inputs.normal(seed, (batch, length, 32))).to(device) for seed in (203, 204))
    oq = torch.empty((batch, length, heads, 32), device=device)
    ok = torch.empty_like(oq)

    def launch():
        attention.rotary(q, k, cos, sin, out_q=oq, out_k=ok)

    launch()
    ms = time_graph(launch, steps, [oq, ok])
    nbytes = 4 * 32 * (4 * batch * heads * length + 2 * batch * length)
    return {"ms_per_launch": round(ms, 6), "bytes_per_launch": nbytes, "gbps": round(nbytes / (ms * 1e-3) / 1e9, 2),
            "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / 8e12, 4), "shape": f"B{batch} H{heads} L{length} d32"}


def cpu_baseline(seconds):
    """The CPU oracle (a C port of the reference's CPU reference) timed on this host's cores on config 2."""
    import numpy as np

    import oracle
    from rocmkernels_amd import inputs

    cfg = CONFIGS[2]
    shape = (cfg["batch"], cfg["heads"], cfg["length"], cfg["width"])
    q, k, v = (inputs.normal(seed, shape) for seed in (101, 102, 103))
    mask = np.ones((cfg["batch"], cfg["length"]), np.uint8)
    threads = min(os.cpu_count() or 1, 16)
    runs, elapsed = 0, 0.0
    while elapsed < seconds or runs == 0:
        begin = time.perf_counter()
        oracle.attention(q, k, v, mask, causal=True, threads=threads)
        elapsed += time.perf_counter() - begin
        runs += 1
    per_run = elapsed / runs
    convention = 4.0 * cfg["batch"] * cfg["heads"] * cfg["length"] ** 2 * cfg["width"]
    return {
        "value": round(convention / per_run / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"full config-2 causal forward (24 x 1024 x 32) on the C oracle, {runs} run(s), {per_run * 1e3:.1f} ms/run",
    }


def forward_kernel_name(cfg, cus):
    """Name rocprofv3 reports for the forward kernel instance that runs on this config. Template arguments: head width,
    statistics-only, 16-byte vector loads, waves per 32-query item and items per persistent workgroup (0: dispatch
    order), chosen from the item count as rk::launch_mapped (rocmkernels_amd/csrc/attention_forward.hip) does."""
    items = (cfg["length"] + 31) // 32 * cfg["batch"] * cfg["heads"]
    resident = 3 if cfg["width"] == 32 else 2
    if cus < items <= resident * cus:
        bins = min(items, cus)
        rounds = -(-items // bins)
        return f"rk::attention_forward_kernel<{cfg['width']}, false, true, 4, {3 if rounds == 3 else 2}>"
    split = 1 if items >= 8192 else 2 if items >= 4096 else 4  # forward_split_for (attention_launch.hpp)
    return f"rk::attention_forward_kernel<{cfg['width']}, false, true, {split}, 0>"


def load_traffic(kernel_key):
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as handle:
        return json.load(handle).get(kernel_key, {}).get("hbm_bytes_per_launch")


def measure(cfg, steps, warmup, backward=True):
    import torch

    from rocmkernels_amd import attention

    device = torch.device("cuda:0")
    q, k, v, du, mask, lengths = make_inputs(cfg, device)
    shape = tuple(q.shape)
    out = torch.empty(shape, device=device)
    lse = torch.empty(shape[:3] + (2,), device=device)
    grads = (torch.empty(shape, device=device), torch.empty(shape, device=device), torch.empty(shape, device=device),
             torch.empty(shape[:3], device=device))

    def forward():
        attention.forward(q, k, v, mask, radius=cfg["radius"], causal=True, output=out, lse=lse)

    def backward_step():
        attention.backward(q, k, v, mask, out, lse, du, radius=cfg["radius"], causal=True, grads=grads)

    def backward_fused():
        attention.backward(q, k, v, mask, out, lse, du, radius=cfg["radius"], causal=True, grads=grads, fused=True)

    pairs = visited_pairs(cfg, lengths)
    full = cfg["batch"] * cfg["heads"] * cfg["length"] ** 2
    stream = torch.cuda.current_stream()
    result = {"visited_pairs": pairs}
    eager = time_eager(forward, steps, warmup, stream)
    graph = time_graph(forward, steps, [out, lse])
    result["forward"] = dict(ms_per_launch=graph, ms_per_launch_eager=eager,
                             tflops_convention=4.0 * full * cfg["width"] / (graph * 1e-3) / 1e12,
                             tflops_visited=4.0 * pairs * cfg["width"] / (graph * 1e-3) / 1e12,
                             flops_visited=4.0 * pairs * cfg["width"])
    if backward:
        forward()
        eager = time_eager(backward_step, steps, warmup, stream)
        graph = time_graph(backward_step, steps, list(grads))
        result["backward"] = dict(ms_per_launch=graph, ms_per_launch_eager=eager,
                                  tflops_convention=8.0 * full * cfg["width"] / (graph * 1e-3) / 1e12,
                                  tflops_visited=8.0 * pairs * cfg["width"] / (graph * 1e-3) / 1e12,
                                  flops_visited=8.0 * pairs * cfg["width"])
        backward_fused()
        eager = time_eager(backward_fused, steps, warmup, stream)
        graph = time_graph(backward_fused, steps, list(grads), exact=False)
        result["backward_fused"] = dict(ms_per_launch=graph, ms_per_launch_eager=eager,
                                        tflops_convention=8.0 * full * cfg["width"] / (graph * 1e-3) / 1e12,
                                        tflops_visited=8.0 * pairs * cfg["width"] / (graph * 1e-3) / 1e12,
                                        flops_visited=8.0 * pairs * cfg["width"])
    for part in ("forward", "backward", "backward_fused"):
        if part in result:
            result[part]["frac_of_fp32_mfma_peak_visited"] = result[part]["tflops_visited"] / PEAK_FP32_MFMA_TFLOPS
    return result


def rounded(d):
    return {k: (round(v, 6) if isinstance(v, float) else v) for k, v in d.items()}


def main():
    global SETTLE_SECONDS
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=400)
    parser.add_argument("--warmup", type=int, default=40)
    parser.add_argument("--config", type=int, default=2, choices=sorted(CONFIGS))
    parser.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample length (0 skips it)")
    parser.add_argument("--settle-seconds", type=float, default=SETTLE_SECONDS,
                        help="untimed continuous load before each timed region (sustained shader clock)")
    parser.add_argument("--no-backward", action="store_true")
    parser.add_argument("--calibrate-copy-mib", type=int, default=0,
                        help="first copy a buffer of this many MiB on the device (reference for rocprofv3 byte counters)")
    args = parser.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (every sequence is independent; "
              "sharding B*H across GPUs needs no communication). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("bench.py needs a GPU")
    if args.calibrate_copy_mib > 0:
        src = torch.ones(args.calibrate_copy_mib * 262144, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    SETTLE_SECONDS = args.settle_seconds
    cfg = CONFIGS[args.config]
    measured = measure(cfg, args.steps, args.warmup, backward=not args.no_backward)
    fwd = measured["forward"]
    kernel = forward_kernel_name(cfg, torch.cuda.get_device_properties(0).multi_processor_count)
    result = {
        "metric": METRIC,
        "value": round(fwd["tflops_convention"], 4),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(fwd["ms_per_launch"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": cfg["workload"], "batch": cfg["batch"], "heads": cfg["heads"], "seq_len": cfg["length"],
                   "head_dim": cfg["width"], "radius": cfg["radius"], "mask": "causal" + (" + key padding" if cfg["padding"] else ""),
                   "visited_pairs": measured["visited_pairs"], "flop_basis_of_value": "reference convention 4*B*H*L^2*d"},
        "tflops_fwd_convention": round(fwd["tflops_convention"], 4),
        "tflops_fwd_visited": round(fwd["tflops_visited"], 4),
        "ms_per_launch_eager": round(fwd["ms_per_launch_eager"], 6),
        "roofline": {"bound": "mfma", "achieved": round(fwd["tflops_visited"], 4), "peak": PEAK_FP32_MFMA_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(fwd["tflops_visited"] / PEAK_FP32_MFMA_TFLOPS, 4),
                     "traffic": load_traffic(f"{kernel} config{args.config}"), "kernel": kernel,
                     "flops_per_launch": fwd["flops_visited"]},
    }
    for part in ("backward", "backward_fused"):
        if part in measured:
            result[part] = rounded(measured[part])
    result["rotary"] = measure_rotary(cfg, args.steps, args.warmup)
    result["cpu_baseline"] = cpu_baseline(args.cpu_seconds) if args.cpu_seconds > 0 and args.config == 2 else None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
