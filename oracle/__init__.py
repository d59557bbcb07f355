"""CPU oracle for the FP32 attention path -- test infrastructure only.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may import this package, and only
as the checker (or as the timed CPU port for the baseline). The product path never calls it.

``attention()`` wraps ``oracle_attention`` in attention_oracle.c, a C restatement of the reference's CPU
reference ``ReferenceAttention`` (ROCmKernels.Tests/AttentionTests.cpp:28-125) extended with a causal flag.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(_HERE, "lib", "liboracle.so")
_libs = {}


def build():
    """Compile liboracle.so with the host C compiler (make)."""
    subprocess.run(["make", "-B", "-C", _HERE], check=True, stdout=subprocess.DEVNULL)


def build_mutant(mutation, directory):
    """Compile a copy of the oracle with one planted mistake (ORACLE_MUTATION=mutation) into ``directory``."""
    path = os.path.join(directory, f"liboracle_mutant{mutation}.so")
    subprocess.run(["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", f"-DORACLE_MUTATION={mutation}",
                    os.path.join(_HERE, "attention_oracle.c"), "-o", path, "-lm", "-lpthread"], check=True)
    return path


def _load(path=LIBRARY):
    if path not in _libs:
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library missing: {path} (run __graft_entry__.build())")
        lib = ctypes.CDLL(path)
        P, I = ctypes.c_void_p, ctypes.c_int
        lib.oracle_attention.argtypes = [P, P, P, P, P, I, I, I, I, I, I, I, P, P, P, P, P, P, I]
        lib.oracle_attention.restype = I
        _libs[path] = lib
    return _libs[path]


def _ptr(array):
    return None if array is None else array.ctypes.data_as(ctypes.c_void_p)


def attention(q, k, v, mask, upstream=None, radius=-1, causal=False, threads=None, library=LIBRARY):
    """Reference-order FP32 attention on packed [B][H][L][D] float32 arrays.

    mask is [B][keys] (any integer/bool dtype, nonzero = visible). Returns a dict with ``output``, ``lse``
    ([B][H][Lq][2]) and, when ``upstream`` is given, ``gq``, ``gk``, ``gv`` and ``delta``.
    """
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    batch, heads, queries, width = q.shape
    keys = k.shape[2]
    assert k.shape == (batch, heads, keys, width) and v.shape == k.shape
    m = np.ascontiguousarray(np.asarray(mask) != 0, dtype=np.uint8)
    assert m.shape == (batch, keys)
    out = {
        "output": np.empty_like(q),
        "lse": np.empty((batch, heads, queries, 2), dtype=np.float32),
    }
    if upstream is not None:
        upstream = np.ascontiguousarray(upstream, dtype=np.float32)
        assert upstream.shape == q.shape
        out.update(gq=np.empty_like(q), gk=np.empty_like(k), gv=np.empty_like(v),
                   delta=np.empty((batch, heads, queries), dtype=np.float32))
    if threads is None:
        threads = min(os.cpu_count() or 1, 16)
    rc = _load(library).oracle_attention(
        _ptr(q), _ptr(k), _ptr(v), _ptr(m), _ptr(upstream), width, batch, heads, queries, keys, int(radius),
        1 if causal else 0, _ptr(out["output"]), _ptr(out["lse"]), _ptr(out.get("gq")), _ptr(out.get("gk")),
        _ptr(out.get("gv")), _ptr(out.get("delta")), int(threads))
    if rc != 0:
        raise RuntimeError("oracle_attention failed")
    return out


def rotary(x, cos, sin, backward=False):
    """Reference-order rotary embedding of x [B][H][L][32] with cos/sin [B][L][32], returned token-major [B][L][H][32].

    Restates ReferenceRotary (ROCmKernels.Tests/PositionalTests.cpp:18-51) in float32 numpy: each product is rounded to
    float32 before the sum, as the C++ expression ``low * cosineLow - high * sineLow`` is evaluated there:
    forward  out[c] = x[c]cos[c] - x[c+16]sin[c],   out[c+16] = x[c+16]cos[c+16] + x[c]sin[c+16];
    backward out[c] = x[c]cos[c] + x[c+16]sin[c+16], out[c+16] = x[c+16]cos[c+16] - x[c]sin[c].
    """
    x = np.asarray(x, dtype=np.float32).transpose(0, 2, 1, 3)  # [B][L][H][32]
    cos = np.asarray(cos, dtype=np.float32)[:, :, None, :]
    sin = np.asarray(sin, dtype=np.float32)[:, :, None, :]
    low, high = x[..., :16], x[..., 16:]
    c_lo, c_hi, s_lo, s_hi = cos[..., :16], cos[..., 16:], sin[..., :16], sin[..., 16:]
    out = np.empty_like(x)
    if backward:
        out[..., :16] = (low * c_lo).astype(np.float32) + (high * s_hi).astype(np.float32)
        out[..., 16:] = (high * c_hi).astype(np.float32) - (low * s_lo).astype(np.float32)
    else:
        out[..., :16] = (low * c_lo).astype(np.float32) - (high * s_lo).astype(np.float32)
        out[..., 16:] = (high * c_hi).astype(np.float32) + (low * s_hi).astype(np.float32)
    return np.ascontiguousarray(out)
