"""torch autograd over the library's FP32 attention entry points, the way the reference wraps its kernels for
training code (tools/Autograd/layernorm_scale_add.py: a torch.autograd.Function whose forward saves the kernel's
statistics and whose backward calls the backward entry point with them; tools/TorchCompare/compare_ops.py:29-56 for
the ctypes binding).

``attention_fp32(q, k, v, mask, radius, causal)`` returns O = softmax(QKᵀ/√D + mask) V for q/k/v [B][H][L][D]
float32 CUDA tensors (D = 32 or 64). The forward keeps O and the {max, sum} statistics; the backward runs the
library's *_ex backward entry point on them. Which backward: ``deterministic=True`` the bit-reproducible two-kernel
one, ``deterministic=False`` the faster one for the call (the fused one, whose dQ is accumulated with atomics, for
128-bit aligned inputs); left at None, the bit-reproducible one exactly when torch's deterministic mode is on
(``torch.use_deterministic_algorithms(True)``).
Everything runs on the GPU through the C ABI; there is no CPU path.
"""
import warnings

import torch

from . import attention


class AttentionFP32(torch.autograd.Function):
    """Autograd Function over attention_fp32_forward_flash / attention64_fp32_forward (and their *_ex forms)."""

    @staticmethod
    def forward(ctx, q, k, v, mask, radius, causal, deterministic, fused):
        for name, t in (("q", q), ("k", k), ("v", v)):
            if t.dim() != 4 or t.dtype != torch.float32 or not t.is_cuda:
                raise ValueError(f"{name} must be a float32 [batch][head][token][D] tensor on the GPU")
        if q.shape[-1] not in (32, 64) or k.shape[-1] != q.shape[-1] or v.shape != k.shape:
            raise ValueError("q, k and v must share D = 32 or 64, and k and v their shape")
        q, k, v = (t if t.stride(-1) == 1 else t.contiguous() for t in (q, k, v))
        out, lse = attention.forward(q, k, v, mask, radius=radius, causal=causal)
        ctx.save_for_backward(q, k, v, mask, out, lse)
        ctx.radius, ctx.causal, ctx.deterministic, ctx.fused = radius, causal, deterministic, fused
        ctx.mark_non_differentiable(lse)
        return out, lse

    @staticmethod
    def backward(ctx, grad_out, grad_lse):
        q, k, v, mask, out, lse = ctx.saved_tensors
        if grad_out is None:
            return None, None, None, None, None, None, None, None
        if grad_out.stride(-1) != 1:
            grad_out = grad_out.contiguous()
        gq, gk, gv, _ = attention.backward(q, k, v, mask, out, lse, grad_out, radius=ctx.radius, causal=ctx.causal,
                                           entry="ex", deterministic=ctx.deterministic, fused=ctx.fused)
        return gq, gk, gv, None, None, None, None, None


def backward_mode(deterministic=None, fused_backward=None):
    """(deterministic, fused) flags of the *_ex backward for attention_fp32's arguments.

    ``deterministic`` None follows torch.are_deterministic_algorithms_enabled(). ``fused_backward`` is the first
    version's spelling, kept as a deprecated alias: True asked for the fused backward (the fused flag), False for the
    bit-reproducible one; it may be combined with a ``deterministic`` that agrees with it, and raises ValueError
    otherwise."""
    fused = False
    if fused_backward is not None:
        warnings.warn("attention_fp32(fused_backward=...) is deprecated; pass deterministic=True or False instead",
                      DeprecationWarning, stacklevel=3)
        if deterministic is not None and bool(deterministic) == bool(fused_backward):
            raise ValueError("fused_backward and deterministic ask for different backward implementations")
        fused = bool(fused_backward)
        deterministic = not fused
    if deterministic is None:
        deterministic = torch.are_deterministic_algorithms_enabled()
    return bool(deterministic), fused


def attention_fp32(q, k, v, mask=None, radius=-1, causal=False, deterministic=None, return_lse=False, fused_backward=None):
    """Differentiable FP32 attention. mask: [B][keys] bool/uint8 on the GPU (None = every key visible).
    ``deterministic``: True for bit-reproducible gradients, False for the faster backward, None (default) to follow
    torch.are_deterministic_algorithms_enabled(). ``fused_backward`` is a deprecated alias (see backward_mode)."""
    deterministic, fused = backward_mode(deterministic, fused_backward)
    if mask is None:
        mask = torch.ones((q.shape[0], k.shape[2]), dtype=torch.uint8, device=q.device)
    elif mask.dtype == torch.bool:
        mask = mask.to(torch.uint8)
    out, lse = AttentionFP32.apply(q, k, v, mask.contiguous(), int(radius), bool(causal), deterministic, fused)
    return (out, lse) if return_lse else out
