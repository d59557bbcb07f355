"""GPU run of the namespaced C++ wrappers (include/ROCmKernels/...), the layer the reference's own tests call
(ROCmKernels.Tests/AttentionTests.cpp:162-224,254-264).

tests/cpp/wrapper_gpu_check.cpp (built by the CMake project next to the library as librocmkernels_wrapper_gpu_check.so)
calls every wrapper once on device buffers: Q and V token-major, K, dO and the outputs packed, so swapped or dropped
stride and pointer arguments change the results. This test writes its inputs, calls it in this process through ctypes
(a process that has initialised the GPU starts no other program), makes the same calls through the C entry points and
requires every output to match bit for bit; a few are also checked against the CPU oracle.
"""
import ctypes
import os

import numpy as np
import pytest
import torch

import oracle
from parity import check_backward, check_forward
from rocmkernels_amd import attention, inputs

pytestmark = pytest.mark.gpu

B, H, L = 2, 3, 70
CHECK_LIBRARY = os.path.join(os.path.dirname(attention.library_path()), "librocmkernels_wrapper_gpu_check.so")


def _tensors(device):
    data = {}
    for width in (32, 64):
        for i, name in enumerate("qkvu"):
            data[f"{name}{width}"] = inputs.normal(1300 + 10 * width + i, (B, H, L, width))
    for i, name in enumerate("qkv"):
        data[f"h64{name}"] = inputs.normal(1400 + i, (B, H, L, 64)).astype(np.float16)
    data["cos"] = np.cos(inputs.normal(1410, (B, L, 32))).astype(np.float32)
    data["sin"] = np.sin(inputs.normal(1411, (B, L, 32))).astype(np.float32)
    mask = np.ones((B, L), np.uint8)
    mask[1, 50:] = 0
    mask[0, 3] = 0
    data["mask"] = mask
    return data


def _token_major(device, a):
    """[B][H][L][D] values stored token-major [B][L][H][D] on the device, returned as the [B][H][L][D] view."""
    return torch.from_numpy(np.ascontiguousarray(a.transpose(0, 2, 1, 3))).to(device).permute(0, 2, 1, 3)


def test_cpp_wrappers_match_c_entry_points(device, tmp_path):
    if not os.path.exists(CHECK_LIBRARY):
        pytest.fail(f"{CHECK_LIBRARY} is missing: build it with __graft_entry__.build() (CMake)")
    data = _tensors(device)
    for name, a in data.items():
        # Q and V files hold the token-major storage [B][L][H][D] the program views through strides.
        stored = a.transpose(0, 2, 1, 3) if name in ("q32", "v32", "q64", "v64") else a
        np.ascontiguousarray(stored).tofile(tmp_path / name)
    attention.lib()  # the library the wrappers call is the one the ctypes calls below use
    check_library = ctypes.CDLL(CHECK_LIBRARY)
    check_library.wrapper_gpu_check.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    check_library.wrapper_gpu_check.restype = ctypes.c_int
    torch.cuda.synchronize()
    written = check_library.wrapper_gpu_check(str(tmp_path).encode(), B, H, L)
    assert written > 0, "wrapper_gpu_check failed (see stderr)"

    def out(name, shape, dtype=np.float32):
        return np.fromfile(tmp_path / f"out_{name}", dtype=dtype).reshape(shape)

    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    mask = dev(data["mask"])
    q32, v32 = _token_major(device, data["q32"]), _token_major(device, data["v32"])
    k32, u32 = dev(data["k32"]), dev(data["u32"])
    q64, v64 = _token_major(device, data["q64"]), _token_major(device, data["v64"])
    k64, u64 = dev(data["k64"]), dev(data["u64"])
    s32, s64, stats = (B, H, L, 32), (B, H, L, 64), (B, H, L, 2)
    checked = 0

    def same(name, got_device, shape, dtype=np.float32):
        nonlocal checked
        torch.cuda.synchronize()
        want = np.ascontiguousarray(got_device.cpu().numpy())
        got = out(name, shape, dtype)
        identical = got.tobytes() == want.tobytes()
        if not identical:
            differ = int((got.view(np.uint8) != want.view(np.uint8)).sum())
            pytest.fail(f"{name}: wrapper and C entry point differ in {differ} bytes")
        checked += 1

    forward_cases = [("forward", "simple", -1, None), ("forward_tiled", "tiled", 5, None), ("forward_flash", "flash", -1, None),
                     ("forward_flash_tuned", "flash_tuned", 7, 13), ("forward_tuned", "tuned", -1, 84)]
    for name, entry, radius, code in forward_cases:
        o, lse = attention.forward(q32, k32, v32, mask, radius=radius, entry=entry, code=code)
        same(f"{name}_o", o, s32)
        same(f"{name}_lse", lse, stats)
    same("statistics_lse", attention.statistics(q32, k32, mask, radius=9), stats)
    o_flash, lse_flash = attention.forward(q32, k32, v32, mask)
    o_causal, lse_causal = attention.forward(q32, k32, v32, mask, causal=True)
    same("forward_flash_ex_o", o_causal, s32)
    same("forward_flash_ex_lse", lse_causal, stats)

    backward_cases = [("backward", "simple", None, False), ("backward_tiled", "tiled", None, False),
                      ("backward_tuned", "tuned", 164, False), ("backward_ex", None, None, True)]
    for name, entry, code, causal in backward_cases:
        o, lse = (o_causal, lse_causal) if causal else (o_flash, lse_flash)
        grads = attention.backward(q32, k32, v32, mask, o, lse, u32, causal=causal, entry=entry or "simple", code=code,
                                   deterministic=causal)
        for part, g in zip(("gq", "gk", "gv"), grads[:3]):
            same(f"{name}_{part}", g, s32)
        same(f"{name}_delta", grads[3], (B, H, L))

    o64, lse64 = attention.forward(q64, k64, v64, mask, radius=11)
    same("forward64_o", o64, s64)
    same("forward64_lse", lse64, stats)
    grads = attention.backward(q64, k64, v64, mask, o64, lse64, u64, radius=11)
    for part, g in zip(("gq", "gk", "gv", "delta"), grads):
        same(f"backward64_{part}", g, s64 if part != "delta" else (B, H, L))
    o64c, lse64c = attention.forward(q64, k64, v64, mask, causal=True)
    same("forward64_ex_o", o64c, s64)
    same("forward64_ex_lse", lse64c, stats)
    grads = attention.backward(q64, k64, v64, mask, o64c, lse64c, u64, causal=True, deterministic=True)
    for part, g in zip(("gq", "gk", "gv", "delta"), grads):
        same(f"backward64_ex_{part}", g, s64 if part != "delta" else (B, H, L))

    go, glse = attention.generic_forward(q32, k32, v32, mask, radius=3)
    same("generic32_o", go, s32)
    same("generic32_lse", glse, stats)
    hq, hk, hv = (dev(data[f"h64{n}"]) for n in "qkv")
    ho, hlse = attention.generic_forward(hq, hk, hv, mask)
    same("generic16_o", ho, s64, np.float16)
    same("generic16_lse", hlse, stats)

    cos, sin = dev(data["cos"]), dev(data["sin"])
    for name, backward in (("rotary", False), ("rotary_back", True)):
        rq, rk = attention.rotary(q32, k32, cos, sin, backward=backward)
        same(f"{name}_q", rq, (B, L, H, 32))
        same(f"{name}_k", rk, (B, L, H, 32))
    assert checked == written == 49  # every wrapper output compared

    # The wrapper outputs also meet the oracle (the C entry points' parity is covered in test_attention_gpu.py).
    want = oracle.attention(data["q32"], data["k32"], data["v32"], data["mask"], data["u32"])
    check_forward(out("forward_flash_o", s32), out("forward_flash_lse", stats), want, "AttentionForwardFlash")
    check_backward(out("backward_gq", s32), out("backward_gk", s32), out("backward_gv", s32), out("backward_delta", (B, H, L)),
                   want, "AttentionBackward")
    want = oracle.attention(data["q64"], data["k64"], data["v64"], data["mask"], data["u64"], causal=True)
    check_backward(out("backward64_ex_gq", s64), out("backward64_ex_gk", s64), out("backward64_ex_gv", s64),
                   out("backward64_ex_delta", (B, H, L)), want, "Attention64BackwardEx")
