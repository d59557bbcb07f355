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
Timing, after the reference harness (ROCmKernels.Benchmark/src/Harness.cpp:104-167): W warm-up launches, then
K launches issued eagerly through ctypes between two HIP events (``ms_per_launch_eager``, host gaps included). The
headline ``ms_per_step`` is the median over at least 20 samples (max(K, 20)); a sample flushes the caches (a 512 MiB
write, larger than the 256 MB Infinity Cache), then replays one HIP graph of L back-to-back launches, L chosen so a
sample lasts >= 10 ms, between two HIP events on the launch stream. ``ms_per_step_min`` and ``ms_per_step_p95`` give
the spread. Inputs are resident in HBM. Before each timed region the same launches run untimed for at least
``--settle-seconds`` of continuous load: under sustained work the MI355X shader clock rises from about 2.0 GHz to
about 2.34 GHz within the first ~20 ms (measured with s_memtime against s_memrealtime inside the forward kernel; cycles
per tile are unchanged), so without it the first timed launches would run at the lower clock. The timed launches do
the full work of every step, and every replay's output is checked against the eager launch's.
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


SETTLE_SECONDS = 1.0    # untimed load before each timed region (the clock settles within about 20 ms)
SAMPLES_MIN = 20       # timed samples per measurement (the reference harness records at least 20)
SAMPLE_MS = 10.0       # each sample is a graph of back-to-back launches lasting at least this long
FLUSH_MIB = 512        # written before every sample: larger than the 256 MB Infinity Cache plus the 8 x 4 MB L2s


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
    """W untimed warm-up launches, then exactly K launches issued eagerly (through ctypes, one by one) between two HIP
    events on the launch stream, device synchronisation on both sides: ms per launch including host launch gaps."""
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


_FLUSH = []


def flush_caches():
    """Overwrites a FLUSH_MIB buffer on the current stream, evicting the inputs from L2 and the Infinity Cache."""
    import torch

    if not _FLUSH:
        _FLUSH.append(torch.empty(FLUSH_MIB << 18, dtype=torch.float32, device="cuda"))
    _FLUSH[0].fill_(1.0)


def time_samples(launch, results, samples, exact=True):
    """The reference harness's protocol (ROCmKernels.Benchmark/src/Harness.cpp:104-167) on HIP graphs: L launches of
    the step, L chosen so one run lasts at least SAMPLE_MS, are captured in one graph; after a settle period every
    sample flushes the caches, then replays the graph between two HIP events on the launch stream. Returns ms per
    launch as the median, minimum and 95th percentile over the samples.

    Every replay's outputs (``results``, first overwritten with NaN) are checked against the eager result: bit for
    bit, or, when ``exact`` is false (atomically accumulated outputs), within 1e-5 of the largest magnitude."""
    import numpy as np
    import torch

    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    for _ in range(3):
        launch()
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(10):
        launch()
    stop.record(stream)
    torch.cuda.synchronize()
    estimate = max(start.elapsed_time(stop) / 10, 1e-4)
    per_sample = max(1, int(np.ceil(SAMPLE_MS / estimate)))

    reference = [r.clone() for r in results]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(per_sample):
            launch()
    settle(graph.replay, per_check=1)
    times = []
    for _ in range(max(samples, SAMPLES_MIN)):  # SAMPLES_MIN is lowered only for short profiler runs (--samples)
        for r in results:
            r.fill_(float("nan"))
        flush_caches()
        torch.cuda.synchronize()
        start.record(stream)
        graph.replay()
        stop.record(stream)
        torch.cuda.synchronize()
        times.append(start.elapsed_time(stop) / per_sample)
        for r, ref in zip(results, reference):
            if exact and not torch.equal(r.view(torch.int32), ref.view(torch.int32)):
                raise RuntimeError("graph replay result differs bitwise from the eager launch")
            if not exact and float((r - ref).abs().max()) > 1e-5 * max(float(ref.abs().max()), 1e-30):
                raise RuntimeError("graph replay result differs from the eager launch")
    times = np.asarray(times)
    return {"ms_per_launch": float(np.median(times)), "ms_min": float(times.min()), "ms_p95": float(np.percentile(times, 95)),
            "samples": int(times.size), "launches_per_sample": per_sample}


def time_graph(launch, steps, results, exact=True):
    """Median ms per launch under the sampled protocol of time_samples (kept for the tests' and profiles' callers)."""
    return time_samples(launch, results, steps, exact)["ms_per_launch"]


ROTARY_COLD_MIB = 768  # distinct rotary input/output sets cycled per sample: well over the 256 MB Infinity Cache


def measure_rotary(cfg, steps, warmup):
    """rotary_fp32 on the config's Q and K (32-wide heads only), token-major layout as the reference's bench
    (RotaryBenchmarks.cpp:52-53): HBM-bound, reported against the 8 TB/s HBM peak with the algorithmic bytes (Q, K
    read; oq, ok written; cos/sin tables read once). Consecutive launches cycle through enough copies of the inputs and
    outputs (ROTARY_COLD_MIB in all) that every launch reads its inputs from HBM, not from the Infinity Cache the
    previous launch filled: a sample replays a graph that launches every set in turn, R times (R such that the sample
    lasts at least SAMPLE_MS), after a cache flush. Every set's outputs are then checked bit for bit against an eager
    launch on set 0 (all sets hold the same inputs)."""
    import numpy as np
    import torch

    from rocmkernels_amd import attention, inputs

    if cfg["width"] != 32:
        return None
    device = torch.device("cuda:0")
    batch, heads, length = cfg["batch"], cfg["heads"], cfg["length"]
    q0, k0 = (torch.from_numpy(inputs.normal(seed, (batch, length, heads, 32))) for seed in (201, 202))
    cos0, sin0 = (torch.from_numpy(inputs.normal(seed, (batch, length, 32))) for seed in (203, 204))
    nbytes = 4 * 32 * (4 * batch * heads * length + 2 * batch * length)
    nsets = max(2, -(-(ROTARY_COLD_MIB << 20) // nbytes))
    sets = []
    for _ in range(nsets):
        q, k = (t.to(device).permute(0, 2, 1, 3) for t in (q0, k0))
        cos, sin = cos0.to(device), sin0.to(device)
        oq = torch.empty((batch, length, heads, 32), device=device)
        sets.append((q, k, cos, sin, oq, torch.empty_like(oq)))

    def launch(i):
        q, k, cos, sin, oq, ok = sets[i]
        attention.rotary(q, k, cos, sin, out_q=oq, out_k=ok)

    launch(0)
    torch.cuda.synchronize()
    want = [t.clone() for t in sets[0][4:]]
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(nsets):
        launch(i)
    stop.record(stream)
    torch.cuda.synchronize()
    reps = max(1, int(np.ceil(SAMPLE_MS / max(start.elapsed_time(stop), 1e-3))))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            for i in range(nsets):
                launch(i)
    settle(graph.replay, per_check=1)
    times = []
    for _ in range(max(steps, SAMPLES_MIN)):
        flush_caches()
        torch.cuda.synchronize()
        start.record(stream)
        graph.replay()
        stop.record(stream)
        torch.cuda.synchronize()
        times.append(start.elapsed_time(stop) / (reps * nsets))
    for st in sets:
        for got, ref in zip(st[4:], want):
            if not torch.equal(got.view(torch.int32), ref.view(torch.int32)):
                raise RuntimeError("rotary: a replayed launch differs from the eager one")
    ms = float(np.median(times))
    return {"ms_per_launch": round(ms, 6), "bytes_per_launch": nbytes, "gbps": round(nbytes / (ms * 1e-3) / 1e9, 2),
            "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / 8e12, 4), "shape": f"B{batch} H{heads} L{length} d32",
            "samples": len(times), "launches_per_sample": reps * nsets,
            "inputs": f"{nsets} distinct input/output sets of {nbytes / 2**20:.1f} MiB launched in turn, so each launch reads HBM"}


def cpu_threads():
    """(visible cores, threads used). The visible count is this process's CPU affinity; the threads used are capped by
    OMP_NUM_THREADS when it is set (the GPU box exports the CPU share it grants one GPU there, and asks that worker
    pools stay within it)."""
    visible = len(os.sched_getaffinity(0))
    try:
        limit = int(os.environ.get("OMP_NUM_THREADS", "0"))
    except ValueError:
        limit = 0
    return visible, (min(visible, limit) if limit > 0 else visible)


def cpu_baseline(config, seconds):
    """The C oracle (a C port of the reference's CPU reference, AttentionTests.cpp:28-125) on the same workload as the
    GPU line, timed on this host: single-threaded and on every core this process may use, in the same process.
    Configs 1-3 are run in full (config 3 forward and backward); configs 4-5 once each on all cores (forward and
    backward), as planned for the CPU side. Returns the all-core rate in the GPU line's unit (convention TFLOP/s)."""
    import numpy as np

    import oracle

    cfg = CONFIGS[config]
    shape = (cfg["batch"], cfg["heads"], cfg["length"], cfg["width"])
    from rocmkernels_amd import inputs

    q, k, v, du = (inputs.normal(seed, shape) for seed in (101, 102, 103, 104))
    lengths = key_lengths(cfg)
    mask = (np.arange(cfg["length"])[None, :] < lengths[:, None]).astype(np.uint8)
    with_backward = config >= 3
    upstream = du if with_backward else None
    visible, threads = cpu_threads()

    def run(nthreads):
        begin = time.perf_counter()
        oracle.attention(q, k, v, mask, upstream, radius=cfg["radius"], causal=True, threads=nthreads)
        return time.perf_counter() - begin

    def timed(nthreads, budget, once=False):
        runs, elapsed = 0, 0.0
        while runs == 0 or (not once and elapsed < budget):
            elapsed += run(nthreads)
            runs += 1
        return elapsed / runs, runs

    full = cfg["batch"] * cfg["heads"] * cfg["length"] ** 2
    flops = (4.0 + (8.0 if with_backward else 0.0)) * full * cfg["width"]
    pairs = visited_pairs(cfg, lengths)
    flops_visited = (4.0 + (8.0 if with_backward else 0.0)) * pairs * cfg["width"]
    many, many_runs = timed(threads, seconds / 2, once=config >= 4)
    result = {
        "value": round(flops / many / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"full {cfg['workload']} {'forward+backward' if with_backward else 'forward'} on the C oracle "
                   f"(double scores, float gradients); {many_runs} run(s) on {threads} threads, {many * 1e3:.1f} ms/run"),
        "ms_per_run_all_cores": round(many * 1e3, 3),
        "tflops_visited_all_cores": round(flops_visited / many / 1e12, 6),
        "host_cores_visible": visible,
        "thread_limit": "OMP_NUM_THREADS" if threads < visible else "affinity",
    }
    if config <= 3:
        single, single_runs = timed(1, seconds / 2)
        result["single_thread"] = {"ms_per_run": round(single * 1e3, 3), "runs": single_runs,
                                   "tflops_convention": round(flops / single / 1e12, 6),
                                   "tflops_visited": round(flops_visited / single / 1e12, 6)}
    return result


def forward_kernel_name(cfg, cus):
    """Name rocprofv3 reports for the forward kernel instance that runs on this config (every config is causal).
    Template arguments: head width, statistics-only, 16-byte vector loads, waves per 32-query item and items per
    persistent workgroup (0: dispatch order), chosen as rk::launch_mapped and rk::dispatch_split
    (rocmkernels_amd/csrc/attention_forward.hip) choose them."""
    items = (cfg["length"] + 31) // 32 * cfg["batch"] * cfg["heads"]
    resident = 3 if cfg["width"] <= 32 else 2  # resident_items_per_cu
    if cus < items <= resident * cus:
        bins = min(items, cus)
        rounds = -(-items // bins)
        return f"rk::attention_forward_kernel<{cfg['width']}, false, true, 4, {3 if rounds == 3 else 2}>"
    # dispatch_split: item costs vary (causal without a radius window, or a window wider than a quarter of the
    # sequence): forward_split_for; otherwise the fewest waves per item that fill every SIMD's resident slots.
    radius, length = cfg["radius"], cfg["length"]
    if radius < 0 or 4 * radius > length:
        split = 1 if items >= 8192 else 2 if items >= 4096 else 4  # forward_split_for (attention_launch.hpp)
    else:
        slots = cus * 4 * (2 if cfg["width"] == 64 else 3)
        split = 1 if items >= slots else 2 if 2 * items >= slots else 4
    return f"rk::attention_forward_kernel<{cfg['width']}, false, true, {split}, 0>"


def traffic_table():
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return {}
    with open(path) as handle:
        return json.load(handle)


def profile_config(config):
    """Configs 2 and 3 share their workload (forward at config 2, backward at config 3), profiled together as config 2."""
    return 2 if config == 3 else config


def load_traffic(kernel, config):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter summary (profiles/traffic.json), or None."""
    return traffic_table().get(f"{kernel} config{profile_config(config)}", {}).get("hbm_bytes_per_launch")


def backward_traffic(config, part):
    """HBM and algorithmic bytes per launch of the kernels one backward call runs, from profiles/traffic.json: the fused
    pre-pass and the fused (no radius window) or band kernel (radius window) for the default backward, which the library
    takes for inputs with 128-bit access, as every bench input has (rk::run in attention_backward.hip); the dQ and
    dK/dV kernels for the deterministic backward."""
    suffix = f" config{profile_config(config)}"
    rows = {k[:-len(suffix)]: v for k, v in traffic_table().items() if k.endswith(suffix) and "forward_kernel" not in k}
    fused = part == "backward"
    names = sorted(n for n in rows if ("fused" in n or "band" in n) == fused)
    if not names:
        return None
    return {"kernels": names, "hbm_bytes_per_launch": sum(rows[n]["hbm_bytes_per_launch"] for n in names),
            "algorithmic_bytes_per_launch": sum(rows[n]["algorithmic_bytes_per_launch"] for n in names)}


def rates(timing, flops_convention, flops_visited, eager=None):
    """ms statistics of time_samples plus the TFLOP/s and roofline fraction they imply (median time)."""
    ms = timing["ms_per_launch"]
    out = dict(timing)
    if eager is not None:
        out["ms_per_launch_eager"] = eager
    out.update(tflops_convention=flops_convention / (ms * 1e-3) / 1e12, tflops_visited=flops_visited / (ms * 1e-3) / 1e12,
               flops_visited=flops_visited)
    out["frac_of_fp32_mfma_peak_visited"] = out["tflops_visited"] / PEAK_FP32_MFMA_TFLOPS
    return out


def measure(cfg, steps, warmup, backward=True, forward_timed=True):
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

    def backward_step():  # the _ex default: the faster backward for the call (fused where it exists)
        attention.backward(q, k, v, mask, out, lse, du, radius=cfg["radius"], causal=True, grads=grads)

    def backward_deterministic():
        attention.backward(q, k, v, mask, out, lse, du, radius=cfg["radius"], causal=True, grads=grads, deterministic=True)

    pairs = visited_pairs(cfg, lengths)
    full = cfg["batch"] * cfg["heads"] * cfg["length"] ** 2
    stream = torch.cuda.current_stream()
    result = {"visited_pairs": pairs}
    width = cfg["width"]
    if forward_timed:
        eager = time_eager(forward, steps, warmup, stream)
        result["forward"] = rates(time_samples(forward, [out, lse], steps), 4.0 * full * width, 4.0 * pairs * width, eager)
    if backward:
        # The default backward may accumulate dQ with atomics (checked against the eager result within 1e-5); the
        # deterministic one is checked bit for bit.
        forward()
        eager = time_eager(backward_step, steps, warmup, stream)
        result["backward"] = rates(time_samples(backward_step, list(grads), steps, exact=False), 8.0 * full * width,
                                   8.0 * pairs * width, eager)
        backward_deterministic()
        eager = time_eager(backward_deterministic, steps, warmup, stream)
        result["backward_deterministic"] = rates(time_samples(backward_deterministic, list(grads), steps), 8.0 * full * width,
                                                 8.0 * pairs * width, eager)
    return result


# The reference's registered benchmark cases (ROCmKernels.Benchmark/src/AttentionBenchmarks.cpp:205-211), each through the
# entry point it calls: (name, width, batch, heads, length, entry, backward).
REFERENCE_CASES = (
    ("Attention32 flash forward b2 h12 l1024", 32, 2, 12, 1024, "flash", False),
    ("Attention32 forward b2 h12 l1024", 32, 2, 12, 1024, "simple", False),
    ("Attention32 backward b2 h12 l1024", 32, 2, 12, 1024, "simple", True),
    ("Attention32 tiled forward b2 h12 l1024", 32, 2, 12, 1024, "tiled", False),
    ("Attention32 tiled backward b2 h12 l1024", 32, 2, 12, 1024, "tiled", True),
    ("Attention64 forward b1 h4 l512", 64, 1, 4, 512, "simple", False),
    ("Attention64 backward b1 h4 l512", 64, 1, 4, 512, "simple", True),
)


def measure_reference_cases(steps):
    """The reference's own benchmark cases (AttentionBenchmarks.cpp:17-47,124-211): constant inputs Q = dO = 0.5,
    K = V = 0.25, mask all ones, radius -1, no causal mask, each through the reference entry point it names (the
    backward cases after one forward, as its State::Initialize does). FLOPs on its convention, 4*B*H*L^2*d forward and
    8*... backward (every pair is visited). Constant inputs fix the results exactly: O = 0.25; every score of a row is
    equal, so dP = dO.V = delta and dS = 0, giving dQ = dK = 0 and dV = sum_q P dO = 0.5, checked before timing.
    Returns {case name: timing} and the flash case alone (the headline reference case)."""
    import torch

    from rocmkernels_amd import attention

    device = torch.device("cuda:0")
    out_cases = {}
    for name, width, batch, heads, length, entry, with_backward in REFERENCE_CASES:
        shape = (batch, heads, length, width)
        q = torch.full(shape, 0.5, device=device)
        k = torch.full(shape, 0.25, device=device)
        v = torch.full(shape, 0.25, device=device)
        du = torch.full(shape, 0.5, device=device)
        mask = torch.ones((batch, length), dtype=torch.uint8, device=device)
        out = torch.empty(shape, device=device)
        lse = torch.empty(shape[:3] + (2,), device=device)
        grads = (torch.empty(shape, device=device), torch.empty(shape, device=device), torch.empty(shape, device=device),
                 torch.empty(shape[:3], device=device))

        def forward():
            attention.forward(q, k, v, mask, radius=-1, causal=False, output=out, lse=lse, entry=entry)

        def backward():
            attention.backward(q, k, v, mask, out, lse, du, radius=-1, causal=False, entry=entry, grads=grads)

        forward()
        launch, results = forward, [out, lse]
        if with_backward:
            backward()
            launch, results = backward, list(grads)
        torch.cuda.synchronize()
        if not bool((out == 0.25).all()):
            raise RuntimeError(f"{name}: output is not 0.25")
        if with_backward:
            gq, gk, gv, _ = grads
            worst = max(float(gq.abs().max()), float(gk.abs().max()), float((gv - 0.5).abs().max()))
            if worst > 1e-5:
                raise RuntimeError(f"{name}: gradients off their closed form by {worst:.3e}")
        flops = (8.0 if with_backward else 4.0) * batch * heads * length * length * width
        timing = rates(time_samples(launch, results, steps), flops, flops)
        timing["entry"] = {"flash": "attention_fp32_forward_flash", "simple": "attention_fp32_forward",
                           "tiled": "attention_fp32_forward_tiled"}[entry] if not with_backward else (
            "attention_fp32_backward_tiled" if entry == "tiled" else "attention_fp32_backward")
        if width == 64:
            timing["entry"] = "attention64_fp32_backward" if with_backward else "attention64_fp32_forward"
        out_cases[name] = rounded(timing)
    flash = dict(out_cases[REFERENCE_CASES[0][0]])
    flash["workload"] = "reference bench case: B2 x H12 x L1024 x d32, Q=0.5, K=V=0.25, no mask, not causal (flash entry)"
    flash["reference_rx6700"] = {"ms_per_launch": 0.96, "tflops": 3.36, "source": "README.md:63 (RX 6700, gfx1031)"}
    return out_cases, flash


PEAK_FP16_MFMA_TFLOPS = 2500.0  # MI355X dense FP16 matrix peak (AMD public specification; no sparsity)
# Softmax work of one 32 x 32 score tile on one wave, the fewest instructions the online softmax needs per tile:
# 8 three-input maxima and 1 compare (row maximum, re-base test), 16 FMAs (scale and offset), 16 exponentials,
# 16 adds (row sum), 8 packed conversions to fp16; measured issue costs on gfx950: 4 cycles per VALU instruction,
# 8 per v_exp_f32. FP16 MFMAs co-issue with VALU work, so this is the fp16 forward's ALU bound.
F16_TILE_VALU = 49
F16_TILE_TRANS = 16
F16_TILE_CYCLES = 4 * F16_TILE_VALU + 8 * F16_TILE_TRANS
SIMDS = 1024          # 256 CUs x 4 SIMDs
CLOCK_GHZ = 2.4       # the clock of the published peaks


def computed_tiles(queries, keys, radius, seqs):
    """32 x 32 score tiles the forward kernels compute: for each 32-query tile, the whole key tiles from the first key
    any of its queries sees to the last (no causal flag: the generic entry point has none)."""
    total = 0
    for q0 in range(0, queries, 32):
        first, last = 0, keys
        if radius >= 0:
            first, last = max(0, q0 - radius), min(keys, q0 + 32 + radius)
        total += -(-(last - first) // 32) if last > first else 0
    return total * seqs


def f16_valu_ceiling_us(tiles):
    """ALU bound of the fp16 forward: every SIMD issuing the softmax work of its share of the tiles, nothing else."""
    return tiles / SIMDS * F16_TILE_CYCLES / (CLOCK_GHZ * 1e3)


def measure_generic(cfg, steps):
    """attention_generic_forward (the reference's Generic/Attention/AttentionGeneric.hip:36-309) on the config's Q, K,
    V and radius with fp32 and fp16 storage. The generic entry point has no causal flag, so every (query, key) pair
    inside the radius window is visited. fp32 storage runs the FP32 MFMA kernel; fp16 storage runs v_mfma_f32_32x32x16_f16, whose matrix work per
    tile is 1/16 of the FP32 kernel's, so it is bound by the softmax VALU work (exp, max, sum: about 62 operations
    and 16 exponentials per 32 x 32 tile and wave) rather than by the FP16 matrix peak it is reported against."""
    import torch

    from rocmkernels_amd import attention

    device = torch.device("cuda:0")
    q32, k32, v32, _, _, _ = make_inputs(cfg, device)
    batch, heads, length, width = q32.shape
    mask = torch.ones((batch, length), dtype=torch.uint8, device=device)
    radius = cfg["radius"]
    if radius < 0:
        pairs = batch * heads * length * length
    else:
        per_query = [min(length - 1, i + radius) - max(0, i - radius) + 1 for i in range(length)]
        pairs = batch * heads * sum(per_query)
    flops = 4.0 * width * pairs
    out = {}
    for name, dtype, peak in (("f32", torch.float32, PEAK_FP32_MFMA_TFLOPS), ("f16", torch.float16, PEAK_FP16_MFMA_TFLOPS)):
        q, k, v = (t.to(dtype) for t in (q32, k32, v32))
        o = torch.empty_like(q)
        lse = torch.empty((batch, heads, length, 2), device=device)

        def launch():
            attention.generic_forward(q, k, v, mask, radius=radius, output=o, lse=lse)

        launch()
        timing = time_samples(launch, [o, lse], steps)
        tflops = flops / (timing["ms_per_launch"] * 1e-3) / 1e12
        out[name] = {"ms_per_launch": round(timing["ms_per_launch"], 6), "ms_min": round(timing["ms_min"], 6),
                     "ms_p95": round(timing["ms_p95"], 6), "tflops_visited": round(tflops, 4), "peak_tflops": peak,
                     "frac_of_mfma_peak": round(tflops / peak, 4), "samples": timing["samples"],
                     "launches_per_sample": timing["launches_per_sample"]}
        if name == "f16":
            tiles = computed_tiles(length, length, radius, batch * heads)
            ceiling = f16_valu_ceiling_us(tiles)
            out[name]["valu_ceiling"] = {
                "us": round(ceiling, 4), "frac": round(ceiling / (timing["ms_per_launch"] * 1e3), 4), "tiles": tiles,
                "cycles_per_tile": F16_TILE_CYCLES,
                "basis": f"{F16_TILE_VALU} VALU x 4 cycles + {F16_TILE_TRANS} v_exp_f32 x 8 cycles per 32x32 wave-tile, "
                         f"{SIMDS} SIMDs at {CLOCK_GHZ} GHz; FP16 MFMAs co-issue"}
    out["workload"] = (f"generic forward: B{batch} x H{heads} x L{length} x d{width}, radius {radius}, not causal "
                       f"(the generic entry point has no causal flag), {pairs} visited pairs")
    return out


def measure_part(part, cfg, args):
    """One part of the line alone, for profiler runs (rocprofv3 then sees only its kernels): the forward and the
    backward of the config (the backward after one forward, both backward implementations), the generic forward, the
    reference cases or rotary."""
    if part in ("forward", "backward"):
        measured = measure(cfg, args.steps, args.warmup, backward=part == "backward", forward_timed=part == "forward")
        return {k: rounded(v) if isinstance(v, dict) else v for k, v in measured.items()}
    if part == "generic":
        return measure_generic(cfg, args.steps)
    if part == "reference":
        return measure_reference_cases(args.steps)[0]
    return measure_rotary(cfg, args.steps, args.warmup)


def rounded(d):
    return {k: (round(v, 6) if isinstance(v, float) else v) for k, v in d.items()}


def main():
    global SETTLE_SECONDS, SAMPLES_MIN, SAMPLE_MS
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20,
                        help="eager launches timed back to back, and timed samples (at least 20) of >= 10 ms each")
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--config", type=int, default=2, choices=sorted(CONFIGS))
    parser.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample length (0 skips it)")
    parser.add_argument("--settle-seconds", type=float, default=SETTLE_SECONDS,
                        help="untimed continuous load before each timed region (sustained shader clock)")
    parser.add_argument("--no-backward", action="store_true")
    parser.add_argument("--samples", type=int, default=SAMPLES_MIN,
                        help="timed samples per measurement (default 20, the harness's minimum; fewer only for profiler runs)")
    parser.add_argument("--sample-ms", type=float, default=SAMPLE_MS, help="minimum length of one sample in ms")
    parser.add_argument("--only", choices=("forward", "backward", "generic", "reference", "rotary"), default=None,
                        help="time one part alone and print its figures (for profiler runs; not the driver's line)")
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
    SAMPLES_MIN = max(1, args.samples)
    SAMPLE_MS = args.sample_ms
    cfg = CONFIGS[args.config]
    if args.only is not None:
        print(json.dumps({"only": args.only, "config": cfg["workload"], "result": measure_part(args.only, cfg, args)}), flush=True)
        return
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
        "ms_per_step_min": round(fwd["ms_min"], 6),
        "ms_per_step_p95": round(fwd["ms_p95"], 6),
        "timing": {"samples": fwd["samples"], "launches_per_sample": fwd["launches_per_sample"],
                   "statistic": "median over samples of ms per launch; each sample: cache flush (512 MiB write), then "
                                "one HIP-graph replay of back-to-back launches lasting >= 10 ms, between HIP events",
                   "eager_steps_timed": args.steps},
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
                     "traffic": load_traffic(kernel, args.config), "kernel": kernel,
                     "flops_per_launch": fwd["flops_visited"]},
    }
    for part in ("backward", "backward_deterministic"):
        if part in measured:
            result[part] = rounded(measured[part])
            result[part]["traffic"] = backward_traffic(args.config, part)
    result["rotary"] = measure_rotary(cfg, args.steps, args.warmup)
    result["generic_forward"] = measure_generic(cfg, args.steps)
    if args.config == 2:
        result["reference_bench_cases"], result["reference_bench_case"] = measure_reference_cases(args.steps)
    result["cpu_baseline"] = cpu_baseline(args.config, args.cpu_seconds) if args.cpu_seconds > 0 else None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
