"""ctypes binding of libROCmKernels.Kernels.Shared.so, the way the reference's training loop binds it.

The reference documents its Python caller as ``ctypes.CDLL`` on the shared library with one ``bind(name,
argtypes)`` per entry point, raw pointers, a by-value ``Strides`` struct and the torch stream handle
(README.md:67-81, tools/TorchCompare/compare_ops.py:29-56). This module keeps that shape: ``lib()`` returns the
bound library, ``Strides`` is the ctypes mirror of the C struct, and ``ENTRY_POINTS`` lists every exported symbol
with its argument types. The torch helpers below (``forward``, ``backward``, ``statistics``) are thin
conveniences over the same calls; they never compute anything on the host and raise when the library is missing
or a tensor is not on the GPU.
"""
import ctypes
import os

LIBRARY_NAME = "libROCmKernels.Kernels.Shared.so"
_HERE = os.path.dirname(os.path.abspath(__file__))

P, I = ctypes.c_void_p, ctypes.c_int
CAUSAL = 1
FUSED_BACKWARD = 2
DETERMINISTIC = 4
DTYPE_FLOAT32 = 0  # rocmkernels_dtype / ROCmKernels::Kernels::DType::Float32
DTYPE_FLOAT16 = 1
HIP_ERROR_INVALID_VALUE = 1


class Strides(ctypes.Structure):
    """Element strides of a [batch][head][token] tensor (C struct rocmkernels_strides)."""

    _fields_ = [("batch", I), ("head", I), ("token", I)]


S = Strides
_FORWARD = [P, P, P, P, P, P, I, I, I, I, I, S, S, S, S, P]
_FORWARD_CODE = [P, P, P, P, P, P, I, I, I, I, I, I, S, S, S, S, P]
_BACKWARD = [P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, S, S, S, S, S, P]
_BACKWARD_CODE = [P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, I, S, S, S, S, S, P]

ENTRY_POINTS = {
    "attention_fp32_forward": _FORWARD,
    "attention_fp32_forward_tiled": _FORWARD,
    "attention_fp32_statistics": [P, P, P, P, I, I, I, I, I, S, S, P],
    "attention_fp32_forward_tuned": _FORWARD_CODE,
    "attention_fp32_forward_flash": _FORWARD,
    "attention_fp32_forward_flash_tuned": _FORWARD_CODE,
    "attention_fp32_backward": _BACKWARD,
    "attention_fp32_backward_tiled": _BACKWARD,
    "attention_fp32_backward_tuned": _BACKWARD_CODE,
    "attention_fp32_backward_profile": _BACKWARD_CODE,
    "attention_fp32_query_profile": _BACKWARD_CODE,
    "attention64_fp32_forward": _FORWARD,
    "attention64_fp32_backward": _BACKWARD,
    "attention_fp32_forward_flash_ex": _FORWARD_CODE,
    "attention_fp32_backward_ex": _BACKWARD_CODE,
    "attention64_fp32_forward_ex": _FORWARD_CODE,
    "attention64_fp32_backward_ex": _BACKWARD_CODE,
    "attention_generic_forward": [P, P, P, P, P, P, I, I, I, I, I, I, S, S, S, S, ctypes.c_ubyte, P],
    "rotary_fp32": [P, P, P, P, P, P, I, I, I, I, S, S, S, S, P],
}

_lib = None


class HipError(RuntimeError):
    """Non-zero hipError_t returned by an entry point (mirrors ROCmKernels::HipError)."""

    def __init__(self, status, name):
        super().__init__(f"{name} returned hipError_t {status}")
        self.status = status


def library_path():
    return os.environ.get("ROCMKERNELS_LIBRARY") or os.path.join(_HERE, "lib", LIBRARY_NAME)


def lib():
    """The bound shared library; raises if it has not been built."""
    global _lib
    if _lib is None:
        path = library_path()
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: build it with __graft_entry__.build() (hipcc, gfx950)")
        handle = ctypes.CDLL(path)
        for name, argtypes in ENTRY_POINTS.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = I
        _lib = handle
    return _lib


def call(name, *args):
    """Calls entry point ``name`` and returns its int status without raising."""
    return getattr(lib(), name)(*args)


def check(name, *args):
    status = call(name, *args)
    if status != 0:
        raise HipError(status, name)


# ---- torch conveniences -------------------------------------------------------------------------------------


def _torch():
    import torch

    return torch


def strides(t):
    """Strides of a 4-D [batch][head][token][D] view with contiguous features."""
    if t.dim() != 4 or t.stride(3) != 1:
        raise ValueError("expected a [batch][head][token][D] tensor with contiguous features")
    return Strides(t.stride(0), t.stride(1), t.stride(2))


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _device_check(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("the attention kernels run on the GPU only; move the tensor to a HIP device")
        if t is not None and t.dtype not in (_torch().float32, _torch().float16, _torch().bool, _torch().uint8):
            raise ValueError(f"unsupported dtype {t.dtype}")


def _stream(stream):
    torch = _torch()
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


_FORWARD_NAMES = {
    ("simple", 32): "attention_fp32_forward",
    ("tiled", 32): "attention_fp32_forward_tiled",
    ("flash", 32): "attention_fp32_forward_flash",
    ("simple", 64): "attention64_fp32_forward",
}


def forward(q, k, v, mask, radius=-1, causal=False, output=None, lse=None, entry="flash", code=None, stream=None):
    """O, lse = attention(q, k, v) with q/k/v [B][H][L][D] float32 views on the GPU and mask [B][keys].

    ``entry`` picks the reference entry point ("simple", "tiled", "flash", "tuned", "flash_tuned"); causal uses
    the *_ex extension. Returns (output, lse) with lse packed [B][H][Lq][2].
    """
    torch = _torch()
    _device_check(q, k, v, mask)
    batch, heads, queries, width = q.shape
    keys = k.shape[2]
    if output is None:
        output = torch.empty((batch, heads, queries, width), device=q.device, dtype=torch.float32)
    if lse is None:
        lse = torch.empty((batch, heads, queries, 2), device=q.device, dtype=torch.float32)
    common = (_ptr(q), _ptr(k), _ptr(v), _ptr(mask), _ptr(output), _ptr(lse), batch, heads, queries, keys, radius)
    views = (strides(q), strides(k), strides(v), strides(output), _stream(stream))
    if causal:
        name = "attention_fp32_forward_flash_ex" if width == 32 else "attention64_fp32_forward_ex"
        check(name, *common, CAUSAL, *views)
    elif entry in ("tuned", "flash_tuned"):
        check("attention_fp32_forward_tuned" if entry == "tuned" else "attention_fp32_forward_flash_tuned", *common, code, *views)
    else:
        check(_FORWARD_NAMES[(entry if width == 32 else "simple", width)], *common, *views)
    return output, lse


def generic_forward(q, k, v, mask, radius=-1, output=None, lse=None, stream=None):
    """attention_generic_forward: q/k/v [B][H][L][D] float32 or float16 views (D = 16, 32 or 64) on the GPU, mask
    [B][keys]. Returns (output, lse): output has q's dtype, lse is float32 [B][H][Lq][2]."""
    torch = _torch()
    _device_check(q, k, v, mask)
    if not (q.dtype == k.dtype == v.dtype) or q.dtype not in (torch.float32, torch.float16):
        raise ValueError("q, k and v must all be float32 or all float16")
    batch, heads, queries, width = q.shape
    if output is None:
        output = torch.empty((batch, heads, queries, width), device=q.device, dtype=q.dtype)
    if lse is None:
        lse = torch.empty((batch, heads, queries, 2), device=q.device, dtype=torch.float32)
    dtype = DTYPE_FLOAT16 if q.dtype == torch.float16 else DTYPE_FLOAT32
    check("attention_generic_forward", _ptr(q), _ptr(k), _ptr(v), _ptr(mask), _ptr(output), _ptr(lse), batch, heads, queries,
          k.shape[2], width, radius, strides(q), strides(k), strides(v), strides(output), dtype, _stream(stream))
    return output, lse


def table_strides(t):
    """Strides of a [B][L][32] cos/sin table (the head entry is unused)."""
    if t.dim() != 3 or t.stride(2) != 1:
        raise ValueError("expected a [batch][token][32] table with contiguous columns")
    return Strides(t.stride(0), 0, t.stride(1))


def rotary(q, k, cos, sin, backward=False, out_q=None, out_k=None, stream=None):
    """rotary_fp32 on q/k [B][H][L][32] float32 views and cos/sin [B][L][32] tables; returns (oq, ok) token-major
    [B][L][H][32]."""
    torch = _torch()
    _device_check(q, k, cos, sin)
    batch, heads, length, width = q.shape
    if width != 32 or k.shape != q.shape:
        raise ValueError("rotary_fp32 takes 32-wide q and k of the same shape")
    if out_q is None:
        out_q = torch.empty((batch, length, heads, 32), device=q.device, dtype=torch.float32)
    if out_k is None:
        out_k = torch.empty((batch, length, heads, 32), device=q.device, dtype=torch.float32)
    check("rotary_fp32", _ptr(q), _ptr(k), _ptr(cos), _ptr(sin), _ptr(out_q), _ptr(out_k), batch, heads, length,
          1 if backward else 0, strides(q), strides(k), table_strides(cos), table_strides(sin), _stream(stream))
    return out_q, out_k


def statistics(q, k, mask, radius=-1, lse=None, stream=None):
    """Softmax statistics only (32-wide): lse packed [B][H][Lq][2]."""
    torch = _torch()
    _device_check(q, k, mask)
    batch, heads, queries, _ = q.shape
    if lse is None:
        lse = torch.empty((batch, heads, queries, 2), device=q.device, dtype=torch.float32)
    check("attention_fp32_statistics", _ptr(q), _ptr(k), _ptr(mask), _ptr(lse), batch, heads, queries, k.shape[2], radius,
          strides(q), strides(k), _stream(stream))
    return lse


def backward(q, k, v, mask, output, lse, upstream, radius=-1, causal=False, entry="simple", code=None, grads=None, stream=None,
             fused=False, deterministic=False):
    """dQ, dK, dV, delta of attention; gradients packed [B][H][L][D], delta [B][H][Lq].

    A causal mask, ``entry="ex"``, ``fused`` or ``deterministic`` go through the *_ex entry points, whose default
    takes the faster backward for the call (the fused one, whose dQ is accumulated with atomics, for 128-bit aligned
    inputs); ``fused`` asks for the fused backward, ``deterministic`` for the bit-reproducible two-kernel one. Otherwise
    ``entry`` picks the reference entry point ("simple", "tiled", "tuned", "profile", "query_profile"), which always
    runs the deterministic kernels."""
    torch = _torch()
    _device_check(q, k, v, mask, output, lse, upstream)
    batch, heads, queries, width = q.shape
    keys = k.shape[2]
    if grads is None:
        grads = (torch.empty((batch, heads, queries, width), device=q.device, dtype=torch.float32),
                 torch.empty((batch, heads, keys, width), device=q.device, dtype=torch.float32),
                 torch.empty((batch, heads, keys, width), device=q.device, dtype=torch.float32),
                 torch.empty((batch, heads, queries), device=q.device, dtype=torch.float32))
    gq, gk, gv, delta = grads
    common = (_ptr(q), _ptr(k), _ptr(v), _ptr(mask), _ptr(output), _ptr(lse), _ptr(upstream), _ptr(gq), _ptr(gk), _ptr(gv),
              _ptr(delta), batch, heads, queries, keys, radius)
    views = (strides(q), strides(k), strides(v), strides(output), strides(upstream), _stream(stream))
    if causal or fused or deterministic or entry == "ex":
        name = "attention_fp32_backward_ex" if width == 32 else "attention64_fp32_backward_ex"
        flags = (CAUSAL if causal else 0) | (FUSED_BACKWARD if fused else 0) | (DETERMINISTIC if deterministic else 0)
        check(name, *common, flags, *views)
    elif width == 64:
        check("attention64_fp32_backward", *common, *views)
    elif entry in ("tuned", "profile", "query_profile"):
        name = {"tuned": "attention_fp32_backward_tuned", "profile": "attention_fp32_backward_profile",
                "query_profile": "attention_fp32_query_profile"}[entry]
        check(name, *common, code, *views)
    else:
        check("attention_fp32_backward_tiled" if entry == "tiled" else "attention_fp32_backward", *common, *views)
    return gq, gk, gv, delta
