"""Concurrent launches: two shapes interleaved on two streams, and two host threads each with its own stream, give the
single-stream results.

The library keeps no device state between calls and only host-side caches keyed by the launch's shape (the
persistent grid's item table and the backward's piece plan, per host thread): interleaving shapes on one thread
rebuilds them on every call, and other threads keep their own. Each launch's outputs are checked against a
single-stream run of the same call: bit for bit, except the atomically summed gradients of the default backward
(1e-5 of the tensor's largest element). Streams are created at the default priority.
"""
import threading

import numpy as np
import pytest
import torch

from parity import normal_case, padding_mask, to_dev
from rocmkernels_amd import attention

pytestmark = pytest.mark.gpu

SHAPES = [(32, 2, 12, 1024, -1), (64, 4, 6, 1024, 100)]
ROUNDS = 3


def _inputs(device, width, batch, heads, length, radius):
    q, k, v, u = normal_case(6100 + width, width, batch, heads, length, length)
    mask = padding_mask(6200 + width, batch, length, length * 3 // 4)
    return dict(zip(("q", "k", "v", "u", "mask"), to_dev(device, q, k, v, u, mask)), radius=radius)


def _run(x, stream=None):
    """Forward, default backward and deterministic backward of one call; returns the outputs by name."""
    o, lse = attention.forward(x["q"], x["k"], x["v"], x["mask"], radius=x["radius"], causal=True, stream=stream)
    fused = attention.backward(x["q"], x["k"], x["v"], x["mask"], o, lse, x["u"], radius=x["radius"], causal=True,
                               stream=stream)
    det = attention.backward(x["q"], x["k"], x["v"], x["mask"], o, lse, x["u"], radius=x["radius"], causal=True,
                             deterministic=True, stream=stream)
    names = ("dq", "dk", "dv", "delta")
    out = {"o": o, "lse": lse}
    out.update({f"fused {n}": t for n, t in zip(names, fused)})
    out.update({f"det {n}": t for n, t in zip(names, det)})
    return out


def _compare(got, want, label):
    for name, t in got.items():
        a = t.cpu().numpy()
        b = want[name].cpu().numpy()
        if name in ("fused dq", "fused dk", "fused dv"):
            err = float(np.abs(a.astype(np.float64) - b).max()) / (float(np.abs(b).max()) or 1.0)
            assert err <= 1e-5, f"{label} {name}: {err:.3e} of the largest element"
        else:
            assert np.array_equal(a, b), f"{label} {name}: differs from the single-stream run"


def test_two_shapes_interleaved_on_two_streams(device):
    xs = [_inputs(device, *shape) for shape in SHAPES]
    want = [_run(x) for x in xs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    results = []
    for _ in range(ROUNDS):
        for i, x in enumerate(xs):
            with torch.cuda.stream(streams[i]):
                results.append((i, _run(x, stream=streams[i])))
    torch.cuda.synchronize()
    for n, (i, got) in enumerate(results):
        _compare(got, want[i], f"launch {n} (shape {SHAPES[i]})")


def test_two_host_threads(device):
    xs = [_inputs(device, *shape) for shape in SHAPES]
    want = [_run(x) for x in xs]
    torch.cuda.synchronize()
    results, errors = {}, []

    def worker(i):
        try:
            stream = torch.cuda.Stream()
            stream.wait_stream(torch.cuda.default_stream())
            with torch.cuda.stream(stream):
                got = [_run(xs[i], stream=stream) for _ in range(ROUNDS)]
            stream.synchronize()
            results[i] = got
        except Exception as error:  # reported on the main thread
            errors.append(repr(error))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(xs))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not errors, errors
    assert sorted(results) == [0, 1]
    torch.cuda.synchronize()
    for i, runs in results.items():
        for n, got in enumerate(runs):
            _compare(got, want[i], f"thread {i} run {n}")
