"""bench.py bookkeeping on the CPU: the one-GPU contract, visited-pair counts against closed forms, and the name of the
forward kernel instance whose launch the roofline object describes."""
import os
import subprocess
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    run = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         timeout=120)
    assert run.returncode == 2
    assert "one GPU" in run.stderr


def test_visited_pairs_closed_forms():
    # Causal without padding: L(L+1)/2 pairs per sequence (config 2: 24 x 524800).
    cfg = bench.CONFIGS[2]
    assert bench.visited_pairs(cfg, bench.key_lengths(cfg)) == 24 * 1024 * 1025 // 2
    # Radius 256 inside the causal band: query q sees min(q, 256) + 1 keys (config 5: 2,072,448 per sequence).
    cfg = bench.CONFIGS[5]
    per_sequence = sum(min(q, 256) + 1 for q in range(8192))
    assert per_sequence == 2072448
    assert bench.visited_pairs(cfg, bench.key_lengths(cfg)) == 16 * per_sequence
    # Key padding: query q sees min(q, valid - 1) + 1 keys.
    cfg = bench.CONFIGS[4]
    lengths = bench.key_lengths(cfg)
    assert np.all((lengths >= 1024) & (lengths <= 2048))
    want = sum(int(np.minimum(np.arange(2048), valid - 1).sum()) + 2048 for valid in lengths)
    assert bench.visited_pairs(cfg, lengths) == want


def test_forward_kernel_names_follow_the_launch_policy():
    # 256 CUs: config 2 has 768 query tiles (3 per CU, persistent); config 4 has 2048 causal items (costs vary: four
    # waves per item); config 5 has 4096 items under a radius-256 window (uniform costs, 2048 resident slots at d = 64:
    # one wave per item).
    assert bench.forward_kernel_name(bench.CONFIGS[2], 256) == "rk::attention_forward_kernel<32, false, true, 4, 3>"
    assert bench.forward_kernel_name(bench.CONFIGS[1], 256) == "rk::attention_forward_kernel<32, false, true, 4, 0>"
    assert bench.forward_kernel_name(bench.CONFIGS[4], 256) == "rk::attention_forward_kernel<64, false, true, 4, 0>"
    assert bench.forward_kernel_name(bench.CONFIGS[5], 256) == "rk::attention_forward_kernel<64, false, true, 1, 0>"


def test_roofline_kernels_have_profiled_traffic():
    # The kernel each config's roofline names, and every kernel of each backward, has a counter row in
    # profiles/traffic.json (rocprofv3 FETCH_SIZE / WRITE_SIZE of the same instance).
    for config in (2, 3, 4, 5):
        name = bench.forward_kernel_name(bench.CONFIGS[config], 256)
        assert bench.load_traffic(name, config) is not None, (config, name)
        for part in ("backward", "backward_deterministic"):
            rows = bench.backward_traffic(config, part)
            assert rows is not None and len(rows["kernels"]) == 2, (config, part)
            fused = any("fused_backward" in n or "band" in n for n in rows["kernels"])
            assert fused == (part == "backward"), (config, part, rows["kernels"])


def test_cpu_baseline_reports_single_thread_and_all_core_rates():
    # Config 1 is small enough to time here; the GPU box runs the same code on its own cores.
    result = bench.cpu_baseline(1, 0.2)
    visible, threads = bench.cpu_threads()
    assert result["kind"] == "port" and result["unit"] == "TFLOP/s" and result["value"] > 0
    assert result["cores"] == threads and result["host_cores_visible"] == visible == len(os.sched_getaffinity(0))
    assert result["single_thread"]["runs"] >= 1 and result["single_thread"]["tflops_convention"] > 0


def test_cpu_threads_respects_the_openmp_share(monkeypatch):
    monkeypatch.setenv("OMP_NUM_THREADS", "1")
    assert bench.cpu_threads()[1] == 1
    monkeypatch.delenv("OMP_NUM_THREADS")
    assert bench.cpu_threads()[1] == len(os.sched_getaffinity(0))
