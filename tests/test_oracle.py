"""Pins the CPU oracle (oracle/attention_oracle.c) before it is trusted as the checker of the HIP kernels.

The reference ships no golden vectors and its CPU reference cannot be built here (it sits in a Catch2 test
translation unit), so the oracle is pinned by checks that do not restate its loop:

* golden fixtures from torch float64 autograd at the reference's own test shapes and inputs (tests/golden/);
* an independent float64 matrix formulation (softmax(QKᵀ/√D)V and its closed-form gradients) on random shapes
  with key masks, radius windows and the causal extension;
* closed forms: constant inputs, radius 0, a single visible key, fully masked rows;
* invariants of a row-stochastic softmax: Σ_k dV_k = Σ_q dO_q and Σ_k dK_k = 0;
* central finite differences in float64 of Σ O·dO against the oracle's analytic gradients;
* thread-count invariance (bit-identical);
* mutation sensitivity: the same checks fail on oracle builds with one planted mistake each.
"""
import json
import os

import numpy as np
import pytest

import oracle
from rocmkernels_amd import inputs

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
with open(os.path.join(GOLDEN, "cases.json")) as handle:
    GOLDEN_CASES = json.load(handle)


def dense_reference(q, k, v, mask, upstream, radius=-1, causal=False):
    """float64 matrix-form attention and its analytic gradients (independent of the oracle's loops)."""
    q, k, v, du = (np.asarray(a, dtype=np.float64) for a in (q, k, v, upstream))
    width = q.shape[-1]
    scale = 1.0 / np.sqrt(width)
    queries, keys = q.shape[2], k.shape[2]
    qi = np.arange(queries)[:, None]
    ki = np.arange(keys)[None, :]
    window = np.ones((queries, keys), dtype=bool)
    if radius >= 0:
        window &= np.abs(qi - ki) <= radius
    if causal:
        window &= ki <= qi
    visible = (np.asarray(mask) != 0)[:, None, None, :] & window[None, None]
    s = np.where(visible, q @ np.swapaxes(k, -1, -2) * scale, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    m_safe = np.where(np.isfinite(m), m, 0.0)
    e = np.where(visible, np.exp(s - m_safe), 0.0)
    total = e.sum(axis=-1, keepdims=True)
    p = np.divide(e, total, out=np.zeros_like(e), where=total > 0)
    o = p @ v
    delta = (du * o).sum(axis=-1)
    dp = du @ np.swapaxes(v, -1, -2)
    ds = p * (dp - delta[..., None])
    return {
        "output": o,
        "lse": np.concatenate([np.where(np.isfinite(m), m, -np.inf), total], axis=-1),
        "gq": ds @ k * scale,
        "gk": np.swapaxes(ds, -1, -2) @ q * scale,
        "gv": np.swapaxes(p, -1, -2) @ du,
        "delta": delta,
    }


def rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    scale = np.abs(b).max()
    return float(np.abs(a - b).max() / (scale if scale > 0 else 1.0))


def assert_matches(got, want, o_tol=2e-6, g_tol=2e-5):
    assert np.abs(got["output"] - want["output"]).max() <= o_tol
    finite = np.isfinite(want["lse"][..., 0])
    assert np.array_equal(np.isfinite(got["lse"][..., 0]), finite)
    assert np.abs(got["lse"][..., 0][finite] - want["lse"][..., 0][finite]).max(initial=0.0) <= o_tol
    assert rel(got["lse"][..., 1], want["lse"][..., 1]) <= o_tol
    for name in ("gq", "gk", "gv"):
        if name in got and name in want:
            assert rel(got[name], want[name]) <= g_tol, name


def random_case(seed, width, batch, heads, queries, keys, padding=False):
    shape_q = (batch, heads, queries, width)
    shape_k = (batch, heads, keys, width)
    q = inputs.normal(seed, shape_q)
    k = inputs.normal(seed + 1, shape_k)
    v = inputs.normal(seed + 2, shape_k)
    du = inputs.normal(seed + 3, shape_q)
    mask = np.ones((batch, keys), dtype=np.uint8)
    if padding:
        lengths = inputs.uniform_int(seed + 4, batch, max(1, keys // 2), keys)
        mask = (np.arange(keys)[None, :] < lengths[:, None]).astype(np.uint8)
    return q, k, v, du, mask


@pytest.mark.parametrize("name", sorted(GOLDEN_CASES))
def test_oracle_matches_torch_golden(name):
    case = GOLDEN_CASES[name]
    data = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    got = oracle.attention(data["q"], data["k"], data["v"], data["mask"], data["upstream"], radius=case["radius"],
                           causal=case["causal"])
    assert_matches(got, {key: data[key] for key in ("output", "lse", "gq", "gk", "gv")})


with open(os.path.join(GOLDEN, "generic_cases.json")) as handle:
    GENERIC_CASES = json.load(handle)


@pytest.mark.parametrize("name", sorted(GENERIC_CASES))
def test_oracle_matches_generic_golden(name):
    # The generic forward's reference (AttentionGenericTests.cpp:44-101) is the same double-precision forward as
    # ReferenceAttention, applied to the values the device reads (fp16 inputs widened to float).
    case = GENERIC_CASES[name]
    data = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    wide = [data[key].astype(np.float32) for key in ("q", "k", "v")]
    got = oracle.attention(*wide, data["mask"], radius=case["radius"])
    assert np.abs(got["output"] - data["output"]).max() <= 1e-6
    finite = np.isfinite(data["lse"][..., 0])
    assert np.array_equal(np.isfinite(got["lse"][..., 0]), finite)
    assert np.abs(got["lse"][..., 0][finite] - data["lse"][..., 0][finite]).max() <= 1e-6
    assert np.abs(got["lse"][..., 1] - data["lse"][..., 1]).max() <= 1e-6 * np.abs(data["lse"][..., 1]).max()


@pytest.mark.parametrize("width,batch,heads,queries,keys,radius,causal,padding", [
    (32, 2, 3, 37, 53, -1, False, True),
    (32, 1, 2, 64, 64, 7, False, False),
    (32, 2, 1, 70, 70, -1, True, True),
    (64, 1, 2, 33, 65, 5, True, False),
    (64, 2, 2, 48, 31, -1, False, True),
    (16, 1, 1, 9, 11, 2, False, False),
])
def test_oracle_matches_dense_formulation(width, batch, heads, queries, keys, radius, causal, padding):
    q, k, v, du, mask = random_case(11 + width + queries, width, batch, heads, queries, keys, padding)
    got = oracle.attention(q, k, v, mask, du, radius=radius, causal=causal)
    want = dense_reference(q, k, v, mask, du, radius, causal)
    assert_matches(got, want)
    assert np.abs(got["delta"] - want["delta"]).max() <= 2e-6


def test_constant_inputs_closed_form():
    # The reference benchmark's inputs (AttentionBenchmarks.cpp:36-43): Q = 0.5, K = V = 0.25. Every score is
    # 0.125*D/sqrt(D) = 0.125*sqrt(D), so O = 0.25 exactly and lse = {0.125*sqrt(D), visible keys}.
    for width in (32, 64):
        shape = (1, 2, 40, width)
        q = np.full(shape, 0.5, np.float32)
        k = np.full(shape, 0.25, np.float32)
        v = np.full(shape, 0.25, np.float32)
        mask = np.ones((1, 40), np.uint8)
        mask[0, 3] = 0
        got = oracle.attention(q, k, v, mask, causal=True)
        assert np.all(got["output"] == np.float32(0.25))
        assert np.allclose(got["lse"][..., 0], 0.125 * np.sqrt(width), rtol=0, atol=1e-6)
        visible = np.array([sum(1 for key in range(query + 1) if key != 3) for query in range(40)], np.float32)
        assert np.array_equal(got["lse"][0, 0, :, 1], visible)


def test_radius_zero_is_identity():
    q, k, v, du, mask = random_case(5, 32, 1, 2, 24, 24)
    got = oracle.attention(q, k, v, mask, du, radius=0)
    assert np.array_equal(got["output"], v)
    assert np.all(got["lse"][..., 1] == 1.0)
    assert np.all(got["gq"] == 0.0) and np.all(got["gk"] == 0.0)
    assert np.array_equal(got["gv"], du)


def test_single_visible_key():
    q, k, v, du, mask = random_case(6, 64, 2, 1, 10, 10)
    mask[:] = 0
    mask[:, 4] = 1
    got = oracle.attention(q, k, v, mask, du)
    assert np.array_equal(got["output"], np.broadcast_to(v[:, :, 4:5, :], q.shape))
    assert np.all(got["gq"] == 0.0)
    assert np.all(np.abs(got["gk"]) <= 1e-6)  # exactly derivative*(dO.v - dO.v) = 0 up to double rounding
    assert np.allclose(got["gv"][:, :, 4], du.sum(axis=2), rtol=1e-6, atol=1e-6)
    assert np.all(np.delete(got["gv"], 4, axis=2) == 0.0)


def test_fully_masked_rows():
    q, k, v, du, mask = random_case(7, 32, 2, 2, 12, 12)
    mask[1, :] = 0
    got = oracle.attention(q, k, v, mask, du)
    assert np.all(got["output"][1] == 0.0)
    assert np.all(got["lse"][1, ..., 0] == -np.inf) and np.all(got["lse"][1, ..., 1] == 0.0)
    assert np.all(got["gq"][1] == 0.0) and np.all(got["gk"][1] == 0.0) and np.all(got["gv"][1] == 0.0)
    # causal: query 0 sees key 0 only when key 0 is visible
    mask[0, 0] = 0
    got = oracle.attention(q, k, v, mask, du, causal=True)
    assert np.all(got["output"][0, :, 0] == 0.0) and np.all(got["lse"][0, :, 0, 0] == -np.inf)


def test_row_stochastic_invariants():
    q, k, v, du, mask = random_case(8, 32, 2, 2, 50, 50, padding=True)
    got = oracle.attention(q, k, v, mask, du, radius=9, causal=True)
    attending = (got["lse"][..., 1] > 0)[..., None]  # rows with at least one visible key
    assert not attending.all()
    assert np.allclose(got["gv"].sum(axis=2), (du * attending).sum(axis=2), rtol=0, atol=2e-5)
    assert np.abs(got["gk"].sum(axis=2)).max() <= 2e-5


def test_finite_differences():
    q, k, v, du, mask = random_case(9, 32, 1, 1, 6, 7)
    mask[0, 2] = 0
    got = oracle.attention(q, k, v, mask, du, radius=4)

    def loss(qq, kk, vv):
        out = dense_reference(qq, kk, vv, mask, du, radius=4)["output"]
        return float((out * du.astype(np.float64)).sum())

    h = 1e-6
    base = [a.astype(np.float64) for a in (q, k, v)]
    for which, name in enumerate(("gq", "gk", "gv")):
        numeric = np.zeros_like(base[which])
        for index in np.ndindex(base[which].shape):
            plus = [a.copy() for a in base]
            minus = [a.copy() for a in base]
            plus[which][index] += h
            minus[which][index] -= h
            numeric[index] = (loss(*plus) - loss(*minus)) / (2 * h)
        assert rel(got[name], numeric) <= 1e-5, name


def test_thread_count_is_bit_identical():
    q, k, v, du, mask = random_case(10, 32, 3, 3, 40, 40, padding=True)
    one = oracle.attention(q, k, v, mask, du, causal=True, threads=1)
    many = oracle.attention(q, k, v, mask, du, causal=True, threads=8)
    for name in one:
        assert np.array_equal(one[name], many[name]), name


@pytest.mark.parametrize("mutation", [1, 2, 3, 4])
def test_pins_catch_planted_mistakes(mutation, tmp_path):
    library = oracle.build_mutant(mutation, str(tmp_path))
    failures = 0
    for name, case in GOLDEN_CASES.items():
        data = np.load(os.path.join(GOLDEN, f"{name}.npz"))
        got = oracle.attention(data["q"], data["k"], data["v"], data["mask"], data["upstream"], radius=case["radius"],
                               causal=case["causal"], library=library)
        try:
            assert_matches(got, {key: data[key] for key in ("output", "lse", "gq", "gk", "gv")})
        except AssertionError:
            failures += 1
    assert failures == len(GOLDEN_CASES)


# ---- rotary (ReferenceRotary, PositionalTests.cpp:18-51) ---------------------------------------------------------

@pytest.mark.parametrize("name", ["rotary_forward_b2h3l4", "rotary_backward_b1h2l3"])
def test_rotary_oracle_matches_float64_golden(name):
    # The reference's own cases and tolerance (PositionalTests.cpp:53-140, CheckClose 1e-6); inputs token-major.
    data = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    backward = bool(data["backward"])
    for x, expected in ((data["q"], data["expected_q"]), (data["k"], data["expected_k"])):
        got = oracle.rotary(x.transpose(0, 2, 1, 3), data["cos"], data["sin"], backward=backward)
        assert got.shape == expected.shape
        assert np.abs(got - expected).max() <= 1e-6


def rope_tables(batch, length, seed):
    """cos/sin of real rotation angles, the same angle for column c and c + 16 (as rotary embeddings build them)."""
    angles = inputs.normal(seed, (batch, length, 16)).astype(np.float64) * 3.0
    cos = np.concatenate([np.cos(angles)] * 2, axis=-1).astype(np.float32)
    sin = np.concatenate([np.sin(angles)] * 2, axis=-1).astype(np.float32)
    return cos, sin


def test_rotary_closed_forms():
    x = inputs.normal(5, (2, 3, 7, 32))
    # Angle 0 is the identity, exactly.
    ones, zeros = np.ones((2, 7, 32), np.float32), np.zeros((2, 7, 32), np.float32)
    assert np.array_equal(oracle.rotary(x, ones, zeros), x.transpose(0, 2, 1, 3))
    assert np.array_equal(oracle.rotary(x, ones, zeros, backward=True), x.transpose(0, 2, 1, 3))
    # A quarter turn maps (lo, hi) to (-hi, lo), exactly.
    quarter = oracle.rotary(x, zeros, ones)
    xt = x.transpose(0, 2, 1, 3)
    assert np.array_equal(quarter[..., :16], -xt[..., 16:]) and np.array_equal(quarter[..., 16:], xt[..., :16])
    # Real rotations: pair norms are kept, and the backward undoes the forward.
    cos, sin = rope_tables(2, 7, 6)
    rotated = oracle.rotary(x, cos, sin)
    norm_in = np.hypot(xt[..., :16].astype(np.float64), xt[..., 16:])
    norm_out = np.hypot(rotated[..., :16].astype(np.float64), rotated[..., 16:])
    assert np.abs(norm_in - norm_out).max() <= 1e-5
    back = oracle.rotary(rotated.transpose(0, 2, 1, 3), cos, sin, backward=True)
    assert np.abs(back - xt).max() <= 1e-5
