"""GPU checks of the torch autograd binding (rocmkernels_amd.autograd): gradients that torch's backward produces
through attention_fp32() match the CPU oracle's at the BASELINE tolerances, for packed tensors and for the
[batch][token][head][D] layout that training code holds (a permuted view, passed by strides)."""
import numpy as np
import pytest
import torch

import oracle
from rocmkernels_amd import autograd, inputs

pytestmark = pytest.mark.gpu


def rel(a, b):
    scale = np.abs(b).max(initial=0.0)
    return float(np.abs(np.asarray(a, np.float64) - b).max(initial=0.0) / (scale if scale > 0 else 1.0))


@pytest.mark.parametrize("width,batch,heads,length,radius,causal,deterministic,layout", [
    (32, 2, 3, 100, -1, True, False, "packed"),
    (32, 2, 2, 130, 11, False, False, "bthd"),
    (64, 1, 2, 90, -1, True, True, "bthd"),
    (64, 2, 1, 64, 5, True, False, "packed"),
    (32, 1, 4, 257, -1, False, True, "packed"),
    (32, 2, 2, 300, -1, True, True, "bthd"),
    (64, 1, 3, 200, -1, False, False, "bthd"),
])
def test_autograd_gradients_match_oracle(device, width, batch, heads, length, radius, causal, deterministic, layout):
    shape = (batch, heads, length, width)
    q, k, v, du = (inputs.normal(seed, shape) for seed in (31, 32, 33, 34))
    lengths = inputs.uniform_int(35, batch, length // 2, length)
    mask = (np.arange(length)[None, :] < lengths[:, None]).astype(np.uint8)
    want = oracle.attention(q, k, v, mask, du, radius=radius, causal=causal)

    def leaf(a):
        if layout == "packed":
            return torch.from_numpy(a).to(device).requires_grad_()
        # Training layout [batch][token][head][D]; the kernels take the permuted [b][h][t][d] view by strides.
        return torch.from_numpy(np.ascontiguousarray(a.transpose(0, 2, 1, 3))).to(device).requires_grad_()

    tq, tk, tv = leaf(q), leaf(k), leaf(v)
    view = (lambda t: t) if layout == "packed" else (lambda t: t.permute(0, 2, 1, 3))
    tm = torch.from_numpy(mask).to(device)
    out = autograd.attention_fp32(view(tq), view(tk), view(tv), tm, radius=radius, causal=causal, deterministic=deterministic)
    tdu = torch.from_numpy(du).to(device)
    (out * tdu).sum().backward()
    torch.cuda.synchronize()
    back = (lambda a: a) if layout == "packed" else (lambda a: a.transpose(0, 2, 1, 3))
    assert np.abs(out.detach().cpu().numpy() - want["output"]).max() <= 1e-5
    for name, t in (("gq", tq), ("gk", tk), ("gv", tv)):
        err = rel(back(t.grad.cpu().numpy()), want[name])
        assert err <= 1e-4, f"{name} rel {err:.3e}"


def test_autograd_lse_is_not_differentiable_and_second_call_reuses_nothing(device):
    q, k, v = (torch.from_numpy(inputs.normal(s, (1, 2, 40, 32))).to(device).requires_grad_() for s in (1, 2, 3))
    out, lse = autograd.attention_fp32(q, k, v, return_lse=True, deterministic=True)
    assert not lse.requires_grad
    out.sum().backward()
    first = q.grad.clone()
    q.grad = None
    autograd.attention_fp32(q, k, v, deterministic=True).sum().backward()
    assert torch.equal(first, q.grad)  # the deterministic backward is bit-reproducible


def test_autograd_follows_torch_deterministic_mode(device):
    # With torch's deterministic mode on, the default call runs the bit-reproducible backward: its gradients equal those
    # of deterministic=True bit for bit (the fused default, whose dQ is summed with atomics, need not).
    q, k, v = (torch.from_numpy(inputs.normal(s, (2, 3, 200, 32))).to(device).requires_grad_() for s in (41, 42, 43))
    autograd.attention_fp32(q, k, v, causal=True, deterministic=True).sum().backward()
    want = [t.grad.clone() for t in (q, k, v)]
    previous = torch.are_deterministic_algorithms_enabled()
    try:
        torch.use_deterministic_algorithms(True)
        for t in (q, k, v):
            t.grad = None
        autograd.attention_fp32(q, k, v, causal=True).sum().backward()
    finally:
        torch.use_deterministic_algorithms(previous)
    for got, ref in zip((q.grad, k.grad, v.grad), want):
        assert torch.equal(got, ref)


def test_autograd_fused_backward_alias(device):
    # The first version's keyword still works (with a DeprecationWarning): fused_backward=True runs the fused kernels,
    # whose gradients meet the same tolerance as the deterministic ones.
    shape = (1, 2, 96, 64)
    q, k, v, du = (inputs.normal(seed, shape) for seed in (51, 52, 53, 54))
    mask = np.ones((1, 96), np.uint8)
    want = oracle.attention(q, k, v, mask, du, causal=True)
    tq, tk, tv = (torch.from_numpy(a).to(device).requires_grad_() for a in (q, k, v))
    with pytest.warns(DeprecationWarning):
        out = autograd.attention_fp32(tq, tk, tv, causal=True, fused_backward=True)
    (out * torch.from_numpy(du).to(device)).sum().backward()
    for name, t in (("gq", tq), ("gk", tk), ("gv", tv)):
        assert rel(t.grad.cpu().numpy(), want[name]) <= 1e-4, name

