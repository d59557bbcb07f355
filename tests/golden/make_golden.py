"""Writes the golden fixtures in this folder (run: python tests/golden/make_golden.py).

The reference holds no golden vectors; its tests regenerate inputs at run time and compare the GPU against its CPU
``ReferenceAttention`` (ROCmKernels.Tests/AttentionTests.cpp:127-286). These fixtures pin the same cases
independently of our oracle:

* shapes, radius and the ``mask[3] = 0`` convention of the reference's TEST_CASE sections (AttentionTests.cpp:272-286,
  :136-137, :232-233);
* inputs Q/K/V/upstream drawn exactly as a Linux build of the reference draws them: std::mt19937 seeds 101-104 through
  libstdc++'s uniform_real_distribution<float>(-1, 1) (TestSupport.hpp:11-21; see rocmkernels_amd.inputs);
* expected outputs from torch in float64 -- softmax(QKᵀ/√D + mask)V for O, {max, Σexp(s - max)} for lse, and
  autograd for dQ/dK/dV -- an implementation that shares no code with oracle/attention_oracle.c.

Two extra cases exercise the causal extension (no reference counterpart) with the same inputs.

The generic cases follow ROCmKernels.Tests/Generic/AttentionGenericTests.cpp:105-188: head widths 16, 32 and 64,
shapes (1, 2, 40, 48, radius -1) and (2, 1, 33, 37, radius 3), mask[3] = 0, Q/K/V from seeds 101-103 narrowed to
the storage type (fp16: round to nearest even, as __float2half_rn does) and the expected forward computed in
float64 on the narrowed values, as the reference's ComputeReference does (:44-101). Index: generic_cases.json.

The rotary cases follow ROCmKernels.Tests/PositionalTests.cpp:53-140: forward (batch 2, heads 3, length 4; Q/K
seeds 21/22 in [-2, 2), cos/sin seeds 23/24 in [-1, 1)) and backward (1, 2, 3; seeds 31-34), token-major inputs, the
expected rotation computed in float64 (an evaluation independent of the float32 oracle).
"""
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.abspath(os.path.join(HERE, "..", "..")))

from rocmkernels_amd.inputs import reference_uniform  # noqa: E402

CASES = [
    # name, width, batch, heads, queries, keys, radius, causal   (reference section)
    ("ref_d32_b2h2_q4k6", 32, 2, 2, 4, 6, -1, False),        # "32-wide heads"
    ("ref_d32_b1h1_q40k40", 32, 1, 1, 40, 40, -1, False),    # "32-wide tiled"
    ("ref_d32_b1h2_q40k40", 32, 1, 2, 40, 40, -1, False),    # "32-wide flash"
    ("ref_d32_b1h2_q64k64_r5", 32, 1, 2, 64, 64, 5, False),  # "32-wide flash banded"
    ("ref_d64_b1h2_q4k6", 64, 1, 2, 4, 6, -1, False),        # "64-wide heads"
    ("causal_d32_b1h2_q40k40", 32, 1, 2, 40, 40, -1, True),
    ("causal_d64_b1h2_q64k64_r5", 64, 1, 2, 64, 64, 5, True),
]


GENERIC_CASES = [
    # width, dtype, batch, heads, queries, keys, radius   (AttentionGenericTests.cpp:153-188)
    (w, dt, *shape) for w in (16, 32, 64) for dt in ("f32", "f16") for shape in ((1, 2, 40, 48, -1), (2, 1, 33, 37, 3))
]


def reference_inputs(width, batch, heads, queries, keys):
    qn, kn = batch * heads * queries * width, batch * heads * keys * width
    q = reference_uniform(101, qn).reshape(batch, heads, queries, width)
    k = reference_uniform(102, kn).reshape(batch, heads, keys, width)
    v = reference_uniform(103, kn).reshape(batch, heads, keys, width)
    upstream = reference_uniform(104, qn).reshape(batch, heads, queries, width)
    mask = np.ones((batch, keys), dtype=np.uint8)
    mask.reshape(-1)[3] = 0
    return q, k, v, upstream, mask


def torch_attention(q, k, v, upstream, mask, radius, causal):
    q64, k64, v64 = (torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (q, k, v))
    width = q.shape[-1]
    queries, keys = q.shape[2], k.shape[2]
    qi = torch.arange(queries)[:, None]
    ki = torch.arange(keys)[None, :]
    visible = torch.tensor(mask != 0)[:, None, None, :].expand(q.shape[0], 1, queries, keys)
    window = torch.ones(queries, keys, dtype=torch.bool)
    if radius >= 0:
        window &= (qi - ki).abs() <= radius
    if causal:
        window &= ki <= qi
    visible = visible & window
    scores = torch.matmul(q64, k64.transpose(-1, -2).contiguous()) / np.sqrt(width)
    scores = scores.masked_fill(~visible, float("-inf"))
    maximum = scores.max(dim=-1, keepdim=True).values
    weights = torch.exp(scores - maximum)
    total = weights.sum(dim=-1, keepdim=True)
    output = torch.matmul(weights / total, v64)
    (output * torch.tensor(upstream, dtype=torch.float64)).sum().backward()
    lse = torch.cat([maximum, total], dim=-1)
    return {
        "output": output.detach().numpy(),
        "lse": lse.detach().numpy(),
        "gq": q64.grad.numpy(),
        "gk": k64.grad.numpy(),
        "gv": v64.grad.numpy(),
    }


def generic_case(width, dtype, batch, heads, queries, keys, radius):
    q, k, v, _, mask = reference_inputs(width, batch, heads, queries, keys)
    if dtype == "f16":
        q, k, v = (a.astype(np.float16) for a in (q, k, v))
    wide = [a.astype(np.float32) for a in (q, k, v)]
    expected = torch_attention(*wide, np.zeros_like(wide[0]), mask, radius, False)
    return dict(q=q, k=k, v=v, mask=mask, output=expected["output"], lse=expected["lse"])


ROTARY_CASES = [  # name, backward, batch, heads, length, seeds (q, k, cos, sin)
    ("rotary_forward_b2h3l4", False, 2, 3, 4, (21, 22, 23, 24)),
    ("rotary_backward_b1h2l3", True, 1, 2, 3, (31, 32, 33, 34)),
]


def rotary_float64(x, cos, sin, backward):
    x, cos, sin = (np.asarray(a, dtype=np.float64) for a in (x, cos, sin))
    low, high = x[..., :16], x[..., 16:]
    c_lo, c_hi, s_lo, s_hi = cos[..., :16], cos[..., 16:], sin[..., :16], sin[..., 16:]
    if backward:
        return np.concatenate([low * c_lo + high * s_hi, high * c_hi - low * s_lo], axis=-1)
    return np.concatenate([low * c_lo - high * s_lo, high * c_hi + low * s_hi], axis=-1)


def main():
    for name, backward, batch, heads, length, seeds in ROTARY_CASES:
        # Token-major [batch][token][head][32] inputs, as the reference's test lays them out; tables [batch][token][32].
        q, k = (reference_uniform(seed, batch * length * heads * 32, -2.0, 2.0).reshape(batch, length, heads, 32) for seed in seeds[:2])
        cos, sin = (reference_uniform(seed, batch * length * 32, -1.0, 1.0).reshape(batch, length, 32) for seed in seeds[2:])
        expected_q = rotary_float64(q, cos[:, :, None, :], sin[:, :, None, :], backward)
        expected_k = rotary_float64(k, cos[:, :, None, :], sin[:, :, None, :], backward)
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), q=q, k=k, cos=cos, sin=sin, backward=np.array(backward),
                            expected_q=expected_q, expected_k=expected_k)
        print(name, "written")
    generic = {}
    for width, dtype, batch, heads, queries, keys, radius in GENERIC_CASES:
        name = f"generic_d{width}_{dtype}_b{batch}h{heads}_q{queries}k{keys}" + (f"_r{radius}" if radius >= 0 else "")
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **generic_case(width, dtype, batch, heads, queries, keys, radius))
        generic[name] = dict(width=width, dtype=dtype, batch=batch, heads=heads, queries=queries, keys=keys, radius=radius)
        print(name, "written")
    with open(os.path.join(HERE, "generic_cases.json"), "w") as handle:
        json.dump(generic, handle, indent=1, sort_keys=True)
        handle.write("\n")
    index = {}
    for name, width, batch, heads, queries, keys, radius, causal in CASES:
        q, k, v, upstream, mask = reference_inputs(width, batch, heads, queries, keys)
        expected = torch_attention(q, k, v, upstream, mask, radius, causal)
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), q=q, k=k, v=v, upstream=upstream, mask=mask, **expected)
        index[name] = dict(width=width, batch=batch, heads=heads, queries=queries, keys=keys, radius=radius, causal=causal)
        print(name, "written")
    with open(os.path.join(HERE, "cases.json"), "w") as handle:
        json.dump(index, handle, indent=1, sort_keys=True)
        handle.write("\n")


if __name__ == "__main__":
    main()
