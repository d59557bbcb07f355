"""GPU parity of attention_generic_forward (16-, 32- and 64-wide heads, fp32 or fp16 storage) through the C ABI.

The reference checks this entry point against a double-precision forward on the values the device reads
(ROCmKernels.Tests/Generic/AttentionGenericTests.cpp:44-146) with max-abs 5e-4 (fp32) and 2e-3 (fp16). Here:
  fp32: O max-abs <= 1e-5 (the BASELINE tolerance), lse as in test_attention_gpu.py;
  fp16: O max-abs <= 2e-3 (the reference's, covering the fp16 rounding of P and of O), lse max max-abs <= 1e-5 and
        lse sum relative <= 1e-5 (scores and sums stay fp32 on fp16 inputs).
Expected values: golden fixtures at the reference's cases (tests/golden/generic_*.npz) and the CPU oracle run on the
fp16 inputs widened to float.
"""
import json
import os

import numpy as np
import pytest
import torch

import oracle
from rocmkernels_amd import attention, inputs

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
with open(os.path.join(GOLDEN, "generic_cases.json")) as _handle:
    GENERIC_CASES = json.load(_handle)

TOL = {"f32": 1e-5, "f16": 2e-3}
LSE_TOL = 1e-5
DTYPES = {"f32": (np.float32, torch.float32), "f16": (np.float16, torch.float16)}


def check(output, lse, want, dtype, label):
    output = np.asarray(output, dtype=np.float64)
    err = np.abs(output - want["output"]).max()
    assert err <= TOL[dtype], f"{label} O max-abs {err:.3e}"
    finite = np.isfinite(want["lse"][..., 0])
    assert np.array_equal(np.isfinite(lse[..., 0]), finite), f"{label} lse finiteness"
    err_m = np.abs(lse[..., 0][finite] - want["lse"][..., 0][finite]).max(initial=0.0)
    assert err_m <= LSE_TOL, f"{label} lse max max-abs {err_m:.3e}"
    assert np.all(lse[..., 1][~finite] == 0.0)
    scale = max(float(np.abs(want["lse"][..., 1]).max()), 1e-30)
    err_s = float(np.abs(lse[..., 1] - want["lse"][..., 1]).max()) / scale
    assert err_s <= LSE_TOL, f"{label} lse sum rel {err_s:.3e}"


def run(device, q, k, v, mask, radius=-1, output=None):
    tq, tk, tv = (torch.from_numpy(np.ascontiguousarray(a)).to(device) for a in (q, k, v))
    tm = torch.from_numpy(np.ascontiguousarray(mask)).to(device)
    out, lse = attention.generic_forward(tq, tk, tv, tm, radius=radius, output=output)
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), lse.cpu().numpy()


@pytest.mark.parametrize("name", sorted(GENERIC_CASES))
def test_generic_reference_cases(device, name):
    case = GENERIC_CASES[name]
    data = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    out, lse = run(device, data["q"], data["k"], data["v"], data["mask"], radius=case["radius"])
    check(out, lse, {"output": data["output"], "lse": data["lse"]}, case["dtype"], name + " vs golden")
    wide = [data[key].astype(np.float32) for key in ("q", "k", "v")]
    want = oracle.attention(*wide, data["mask"], radius=case["radius"])
    check(out, lse, want, case["dtype"], name + " vs oracle")


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("width", [16, 32, 64])
@pytest.mark.parametrize("batch,heads,queries,keys,radius,pad", [
    (2, 3, 100, 70, -1, True),
    (1, 2, 257, 300, 9, False),
    (3, 1, 1, 45, -1, True),
    (1, 1, 64, 64, 0, False),
    (2, 2, 33, 1, -1, False),
])
def test_generic_matches_oracle(device, dtype, width, batch, heads, queries, keys, radius, pad):
    np_type, _ = DTYPES[dtype]
    seed = 900 + width + queries
    q = inputs.normal(seed, (batch, heads, queries, width)).astype(np_type)
    k = inputs.normal(seed + 1, (batch, heads, keys, width)).astype(np_type)
    v = inputs.normal(seed + 2, (batch, heads, keys, width)).astype(np_type)
    mask = np.ones((batch, keys), np.uint8)
    if pad:
        lengths = inputs.uniform_int(seed + 3, batch, max(1, keys // 2), keys)
        mask = (np.arange(keys)[None, :] < lengths[:, None]).astype(np.uint8)
        mask[0, 0] = 0
    want = oracle.attention(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), mask, radius=radius)
    out, lse = run(device, q, k, v, mask, radius=radius)
    check(out, lse, want, dtype, f"d{width} {dtype}")


@pytest.mark.parametrize("width", [32, 64])
def test_generic_fp32_is_the_flash_forward(device, width):
    # fp32 storage at 32/64-wide heads runs the same kernel as attention_fp32_forward / attention64_fp32_forward.
    q, k, v = (inputs.normal(seed, (2, 2, 150, width)) for seed in (11, 12, 13))
    mask = np.ones((2, 150), np.uint8)
    mask[1, 140:] = 0
    tq, tk, tv, tm = (torch.from_numpy(a).to(device) for a in (q, k, v, mask))
    a_out, a_lse = attention.generic_forward(tq, tk, tv, tm, radius=20)
    b_out, b_lse = attention.forward(tq, tk, tv, tm, radius=20, entry="simple")
    torch.cuda.synchronize()
    assert torch.equal(a_out.view(torch.int32), b_out.view(torch.int32))
    assert torch.equal(a_lse.view(torch.int32), b_lse.view(torch.int32))


@pytest.mark.parametrize("width", [16, 32, 64])
def test_generic_fp16_strided_and_unaligned(device, width):
    # Rows of 2*width halves with an odd element offset: neither 16-byte aligned nor a stride multiple of 8, so the
    # kernel takes its 16-bit load path; the output is a strided view too.
    batch, heads, queries, keys = 2, 2, 70, 90
    base = [inputs.normal(40 + i, (batch, heads, n, 2 * width + 1)).astype(np.float16) for i, n in enumerate((queries, keys, keys))]
    views = [torch.from_numpy(a).to(device)[..., 1:width + 1] for a in base]
    mask = np.ones((batch, keys), np.uint8)
    mask[0, 50:] = 0
    tm = torch.from_numpy(mask).to(device)
    out_store = torch.zeros(batch, heads, queries, 3 * width, dtype=torch.float16, device=device)
    out_view = out_store[..., width:2 * width]
    out, lse = attention.generic_forward(*views, tm, radius=-1, output=out_view)
    torch.cuda.synchronize()
    want = oracle.attention(*(v.float().cpu().numpy() for v in views), mask)
    check(out.float().cpu().numpy(), lse.cpu().numpy(), want, "f16", f"d{width} strided")
    assert torch.count_nonzero(out_store[..., :width]) == 0 and torch.count_nonzero(out_store[..., 2 * width:]) == 0


def test_generic_fully_masked_batch(device):
    q, k, v = (inputs.normal(seed, (2, 1, 40, 16)).astype(np.float16) for seed in (1, 2, 3))
    mask = np.ones((2, 40), np.uint8)
    mask[1] = 0
    out, lse = run(device, q, k, v, mask)
    assert np.all(out[1] == 0.0)
    assert np.all(lse[1, ..., 0] == -np.inf) and np.all(lse[1, ..., 1] == 0.0)
    want = oracle.attention(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), mask)
    check(out, lse, want, "f16", "masked batch")


@pytest.mark.parametrize("width", [16, 32, 64])
def test_generic_fp16_masked_keys_with_garbage_values_are_ignored(device, width):
    # Masked keys contribute exactly nothing whatever their rows hold: the staged V path (d = 32, 64) writes zeros
    # for their rows, the 16-bit path zeroes their operand elements. The masked keys sit inside and at the end of
    # tiles, in every query tile's key range.
    batch, heads, queries, keys = 2, 2, 96, 100
    q, k, v = (inputs.normal(70 + i, (batch, heads, n, width)).astype(np.float16) for i, n in enumerate((queries, keys, keys)))
    mask = np.ones((batch, keys), np.uint8)
    mask[0, 40:48] = 0
    mask[0, 90:] = 0
    mask[1, 5] = 0
    want = oracle.attention(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), mask)
    hidden = mask[:, None, :, None] == 0
    k = np.where(hidden, np.float16(np.inf), k)
    v = np.where(hidden, np.float16(np.nan), v)
    out, lse = run(device, q, k, v, mask)
    check(out, lse, want, "f16", f"d{width} garbage in masked rows")


@pytest.mark.parametrize("width", [32, 64])
def test_generic_fp16_one_wave_per_item(device, width):
    # 8192 query tiles (one wave per item, forward_split_for) with a radius window; odd key count so the last tile is
    # partial and its missing rows come from the range check.
    batch, heads, queries, keys = 8, 32, 1024, 1023
    seed = 800 + width
    q = inputs.normal(seed, (batch, heads, queries, width)).astype(np.float16)
    k = inputs.normal(seed + 1, (batch, heads, keys, width)).astype(np.float16)
    v = inputs.normal(seed + 2, (batch, heads, keys, width)).astype(np.float16)
    mask = np.ones((batch, keys), np.uint8)
    mask[3, 500:] = 0
    want = oracle.attention(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), mask, radius=40)
    out, lse = run(device, q, k, v, mask, radius=40)
    check(out, lse, want, "f16", f"d{width} 8192 items")


@pytest.mark.parametrize("width", [32, 64])
def test_generic_fp16_token_major_aligned(device, width):
    # [B][T][H][D] storage viewed as [B][H][T][D]: token stride H*D halves, rows 16-byte aligned, so K and V take
    # the 128-bit paths (V staged through LDS) with a row step other than the head width.
    batch, heads, queries, keys = 2, 3, 130, 97
    arrays = [inputs.normal(60 + i, (batch, n, heads, width)).astype(np.float16) for i, n in enumerate((queries, keys, keys))]
    views = [torch.from_numpy(a).to(device).permute(0, 2, 1, 3) for a in arrays]
    assert views[2].stride(2) == heads * width
    mask = np.ones((batch, keys), np.uint8)
    mask[1, 60:] = 0
    tm = torch.from_numpy(mask).to(device)
    out, lse = attention.generic_forward(*views, tm, radius=33)
    torch.cuda.synchronize()
    want = oracle.attention(*(a.transpose(0, 2, 1, 3).astype(np.float32) for a in arrays), mask, radius=33)
    check(out.float().cpu().numpy(), lse.cpu().numpy(), want, "f16", f"d{width} token-major")


@pytest.mark.parametrize("batch,heads,length,width,radius", [
    (2, 12, 1024, 32, -1),   # config 2's shape (no causal flag in this API: every pair)
    (32, 1, 2048, 64, -1),   # config 4's
    (16, 1, 8192, 64, 256),  # config 5's
])
def test_generic_fp16_benchmark_shapes(device, batch, heads, length, width, radius):
    # The shapes bench.py times the generic forward on, in full, against the oracle on the fp16 inputs.
    seed = 500 + width + length
    q, k, v = (inputs.normal(seed + i, (batch, heads, length, width)).astype(np.float16) for i in range(3))
    mask = np.ones((batch, length), np.uint8)
    want = oracle.attention(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), mask, radius=radius)
    out, lse = run(device, q, k, v, mask, radius=radius)
    check(out, lse, want, "f16", f"{batch}x{heads}x{length} d{width} r{radius}")


@pytest.mark.parametrize("width", [32, 64])
def test_generic_fp16_staged_v_is_bit_identical(device, width):
    # The staged V path (128-bit loads, LDS, transposing reads) feeds the MFMAs the same operands as the 16-bit path:
    # the same inputs with V as an unaligned view (16-bit loads) give the same bits, padding and radius included.
    batch, heads, queries, keys = 2, 2, 150, 133
    q, k, v = (inputs.normal(80 + i, (batch, heads, n, width)).astype(np.float16) for i, n in enumerate((queries, keys, keys)))
    mask = np.ones((batch, keys), np.uint8)
    mask[0, 100:] = 0
    mask[1, 7] = 0
    tq, tk, tv = (torch.from_numpy(a).to(device) for a in (q, k, v))
    tm = torch.from_numpy(mask).to(device)
    wide = torch.zeros(batch, heads, keys, width + 1, dtype=torch.float16, device=device)
    wide[..., 1:] = tv
    tv_unaligned = wide[..., 1:]
    assert tv_unaligned.data_ptr() % 16 != 0
    staged, staged_lse = attention.generic_forward(tq, tk, tv, tm, radius=40)
    plain, plain_lse = attention.generic_forward(tq, tk, tv_unaligned, tm, radius=40)
    torch.cuda.synchronize()
    assert torch.equal(staged.view(torch.int16), plain.view(torch.int16))
    assert torch.equal(staged_lse.view(torch.int32), plain_lse.view(torch.int32))


@pytest.mark.parametrize("batch,heads,length,width,radius", [
    (2, 12, 2048, 64, -1),   # 1536 query tiles at d = 64: two waves per item
    (2, 16, 2048, 32, 300),  # 2048 at d = 32: two waves per item, radius window
    (1, 64, 1024, 16, -1),   # 2048 at d = 16: two waves per item
])
def test_generic_fp16_two_waves_per_item(device, batch, heads, length, width, radius):
    # Item counts between half and all of the resident wave slots take two waves per query tile (f16_split_for).
    seed = 600 + width + length
    q, k, v = (inputs.normal(seed + i, (batch, heads, length, width)).astype(np.float16) for i in range(3))
    mask = np.ones((batch, length), np.uint8)
    mask[-1, length // 3:] = 0
    want = oracle.attention(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), mask, radius=radius)
    out, lse = run(device, q, k, v, mask, radius=radius)
    check(out, lse, want, "f16", f"{batch}x{heads}x{length} d{width} r{radius}")


SHARED_CASES = [
    (64, 4, 100, 77, -1, True),     # 256 sequences x 4 query tiles (the last partial): four tiles per workgroup
    (32, 8, 130, 300, 21, True),    # 5 query tiles (a half-empty second workgroup), radius window, more keys than queries
    (130, 1, 128, 128, -1, False),  # 130 workgroups, fewer than the CUs: the per-wave kernel at both widths
    (65, 4, 33, 20, 5, True),       # 2 query tiles, fewer keys than one tile, the window wider than the keys
    (16, 16, 256, 256, 64, False),  # radius window: each workgroup streams the union of its four tiles' windows
    (64, 16, 128, 64, 7, True),     # 1024 workgroups (four per CU): one key stream
]


@pytest.mark.parametrize("width", [32, 64])
@pytest.mark.parametrize("batch,heads,queries,keys,radius,pad", SHARED_CASES)
def test_generic_fp16_shared_kv_tiles(device, width, batch, heads, queries, keys, radius, pad):
    # At d = 64, grids of at least one workgroup of four query tiles per CU take the shared K/V kernel (the waves of a
    # workgroup stream its K/V tiles through LDS once for all of them; two key streams per workgroup below four
    # workgroups per CU); the shapes cover partial workgroups, Lq != Lk, radius windows and key padding, with one and two
    # streams. At d = 32 the same shapes run the per-wave kernel.
    seed = 1000 + width + queries + keys
    q = inputs.normal(seed, (batch, heads, queries, width)).astype(np.float16)
    k = inputs.normal(seed + 1, (batch, heads, keys, width)).astype(np.float16)
    v = inputs.normal(seed + 2, (batch, heads, keys, width)).astype(np.float16)
    mask = np.ones((batch, keys), np.uint8)
    if pad:
        lengths = inputs.uniform_int(seed + 3, batch, 1, keys)
        mask = (np.arange(keys)[None, :] < lengths[:, None]).astype(np.uint8)
        mask[0, 0] = 0
    want = oracle.attention(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), mask, radius=radius)
    out, lse = run(device, q, k, v, mask, radius=radius)
    check(out, lse, want, "f16", f"{batch}x{heads} {queries}x{keys} d{width} r{radius} shared")


@pytest.mark.parametrize("width", [32, 64])
def test_generic_fp16_shared_kv_tiles_garbage_and_masked_batch(device, width):
    # Masked keys holding inf (K) and NaN (V) contribute nothing through the shared stages (their V elements are zeroed
    # in the operand registers, their scores dropped), and a fully masked batch gives O = 0, lse = {-inf, 0}.
    batch, heads, queries, keys = 32, 8, 96, 100
    q, k, v = (inputs.normal(1100 + i, (batch, heads, n, width)).astype(np.float16) for i, n in enumerate((queries, keys, keys)))
    mask = np.ones((batch, keys), np.uint8)
    mask[0, 40:48] = 0
    mask[0, 90:] = 0
    mask[1, 5] = 0
    mask[2] = 0
    want = oracle.attention(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), mask)
    hidden = mask[:, None, :, None] == 0
    k = np.where(hidden, np.float16(np.inf), k)
    v = np.where(hidden, np.float16(np.nan), v)
    out, lse = run(device, q, k, v, mask)
    check(out, lse, want, "f16", f"d{width} shared, garbage in masked rows")
    assert np.all(out[2] == 0.0) and np.all(lse[2, ..., 0] == -np.inf) and np.all(lse[2, ..., 1] == 0.0)


@pytest.mark.parametrize("case", range(12))
def test_generic_fp16_shared_kv_tiles_random_shapes(device, case):
    # Seeded random shapes on the shared K/V kernel (d = 64, at least one workgroup of four query tiles per CU): query
    # and key counts that leave partial tiles and partial workgroups, radius windows, key padding; both stream counts.
    rng = np.random.default_rng(7000 + case)
    seqs = int(rng.choice([256, 320, 512, 1024]))
    heads = int(rng.choice([1, 2, 4, 8]))
    batch = seqs // heads
    queries = int(rng.integers(1, 3)) * 128 - int(rng.integers(0, 100))
    keys = int(rng.integers(1, 300))
    radius = -1 if rng.random() < 0.4 else int(rng.integers(0, 160))
    seed = 7100 + 10 * case
    q = inputs.normal(seed, (batch, heads, queries, 64)).astype(np.float16)
    k = inputs.normal(seed + 1, (batch, heads, keys, 64)).astype(np.float16)
    v = inputs.normal(seed + 2, (batch, heads, keys, 64)).astype(np.float16)
    mask = np.ones((batch, keys), np.uint8)
    if rng.random() < 0.6:
        lengths = inputs.uniform_int(seed + 3, batch, 1, keys)
        mask = (np.arange(keys)[None, :] < lengths[:, None]).astype(np.uint8)
    want = oracle.attention(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), mask, radius=radius)
    out, lse = run(device, q, k, v, mask, radius=radius)
    check(out, lse, want, "f16", f"case {case}: {batch}x{heads} {queries}x{keys} d64 r{radius} shared")


@pytest.mark.parametrize("radius", [-1, 20])
def test_generic_fp16_shared_kv_tiles_token_major(device, radius):
    # [B][T][H][D] storage viewed as [B][H][T][D] on the shared K/V kernel (256 sequences): the stage loads step by the
    # token stride H*D, not the head width.
    batch, heads, queries, keys, width = 64, 4, 100, 90, 64
    arrays = [inputs.normal(7300 + i, (batch, n, heads, width)).astype(np.float16) for i, n in enumerate((queries, keys, keys))]
    views = [torch.from_numpy(a).to(device).permute(0, 2, 1, 3) for a in arrays]
    assert views[1].stride(2) == heads * width
    mask = np.ones((batch, keys), np.uint8)
    mask[3, 70:] = 0
    mask[5, :10] = 0
    out, lse = attention.generic_forward(*views, torch.from_numpy(mask).to(device), radius=radius)
    torch.cuda.synchronize()
    want = oracle.attention(*(a.transpose(0, 2, 1, 3).astype(np.float32) for a in arrays), mask, radius=radius)
    check(out.float().cpu().numpy(), lse.cpu().numpy(), want, "f16", f"d64 token-major shared r{radius}")
