"""CPU tests that pin the float64 oracle (oracle/attn_oracle.c).

The oracle restates pmkl_pytorch_ext/fused_self_attention.cpp:5-64 in float64.
It is pinned by:
  * the reference's own CPU operator, compiled from its source into oracle/_ref,
    through the committed fixtures (tests/golden, float64 runs) and, where the
    build is present, live on fresh inputs;
  * torch.nn.functional.scaled_dot_product_attention in float64 (the
    reference's Python oracle, test_fused_self_attention.py:6-7);
  * closed forms (K = 0, constant V, S = 1, row 0) and brute force on tiny
    shapes written independently of the oracle;
and the checks are shown to catch plausible mistakes (wrong scale, flipped
mask, shifted keys, transposed operands) planted in the oracle's inputs.
"""
from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"
FIXTURES = sorted(GOLDEN.glob("ref_*.npz"))


def _load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def test_fixtures_present():
    assert len(FIXTURES) >= 6


@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: p.stem)
def test_oracle_matches_reference_fp64_fixture(path):
    """float64 run of the reference operator == oracle (same algorithm in double)."""
    f = _load(path)
    B, H, S, D, causal = int(f["B"]), int(f["H"]), int(f["S"]), int(f["D"]), bool(f["causal"])
    q, k, v = (f[x].reshape(B * H, S, D) for x in "qkv")
    o, m, l = oracle.attn_fwd_rows(q, k, v, causal=causal)
    assert np.abs(o - f["o_fp64"].reshape(B * H, S, D)).max() <= 1e-13
    assert np.abs(m - f["m_fp64"].reshape(B * H, S)).max() <= 1e-13
    assert np.all(np.abs(l - f["l_fp64"].reshape(B * H, S)) <= 1e-13 * np.abs(f["l_fp64"].reshape(B * H, S)))


@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: p.stem)
def test_reference_fp32_within_tolerance_of_oracle(path):
    """The reference's own float32 run is within the fp32 tolerance of the oracle:
    the oracle is the fp32+ accumulation target the device path is held to."""
    f = _load(path)
    B, H, S, D, causal = int(f["B"]), int(f["H"]), int(f["S"]), int(f["D"]), bool(f["causal"])
    q, k, v = (f[x].reshape(B * H, S, D) for x in "qkv")
    o, m, l = oracle.attn_fwd_rows(q, k, v, causal=causal)
    assert np.abs(o - f["o_fp32"].reshape(B * H, S, D)).max() <= 1e-5
    assert np.allclose(f["m_fp32"].reshape(B * H, S), m, atol=1e-5, rtol=1e-5)
    assert np.allclose(f["l_fp32"].reshape(B * H, S), l, atol=1e-5, rtol=1e-5)


def test_oracle_live_against_reference_build():
    """Fresh inputs through the reference operator built in oracle/_ref."""
    import torch

    ref = oracle.reference_op()
    if ref is None:
        pytest.skip("oracle/_ref not built (the reference tree is absent)")
    rng = _rng(77)
    for (B, H, S, D, causal) in [(1, 3, 50, 64, True), (2, 1, 33, 32, False), (1, 1, 70, 128, True)]:
        q, k, v = (rng.standard_normal((B, H, S, D)).astype(np.float32) for _ in range(3))
        o_r, m_r, l_r = ref.fused_self_attention_fw(*(torch.from_numpy(x).double() for x in (q, k, v)), causal)
        o, m, l = oracle.attn_fwd_rows(q.reshape(-1, S, D), k.reshape(-1, S, D), v.reshape(-1, S, D), causal=causal)
        assert np.abs(o - o_r.numpy().reshape(-1, S, D)).max() <= 1e-13
        assert np.abs(m - m_r.numpy().reshape(-1, S)).max() <= 1e-13


@pytest.mark.parametrize("causal", [True, False])
def test_oracle_vs_sdpa_float64(causal):
    rng = _rng(5)
    for (BH, S, D) in [(3, 1, 32), (2, 17, 64), (1, 129, 128), (4, 64, 32)]:
        q, k, v = (rng.standard_normal((BH, S, D)).astype(np.float32) for _ in range(3))
        o, _, _ = oracle.attn_fwd_rows(q, k, v, causal=causal)
        assert np.abs(o - oracle.attn_sdpa_f64(q, k, v, causal=causal)).max() <= 1e-12


def test_oracle_closed_forms():
    rng = _rng(6)
    BH, S, D = 2, 45, 64
    q, v = (rng.standard_normal((BH, S, D)).astype(np.float32) for _ in range(2))
    kz = np.zeros_like(q)
    # K == 0: all scores 0 -> O_i = mean(V_0..V_i), m_i = 0, l_i = i + 1
    o, m, l = oracle.attn_fwd_rows(q, kz, v, causal=True)
    prefix = np.cumsum(v.astype(np.float64), axis=1) / np.arange(1, S + 1)[None, :, None]
    assert np.abs(o - prefix).max() <= 1e-12
    assert np.all(m == 0.0) and np.all(l == np.arange(1, S + 1)[None, :])
    # non-causal K == 0: O_i = mean of all V
    o, _, l = oracle.attn_fwd_rows(q, kz, v, causal=False)
    assert np.abs(o - v.astype(np.float64).mean(axis=1, keepdims=True)).max() <= 1e-12 and np.all(l == S)
    # constant V -> O == c
    k = rng.standard_normal((BH, S, D)).astype(np.float32)
    o, _, _ = oracle.attn_fwd_rows(q, k, np.full_like(v, 0.375), causal=True)
    assert np.abs(o - 0.375).max() <= 1e-14
    # row 0 of a causal problem sees only key 0: O_0 = V_0, m_0 = s_00, l_0 = 1
    o, m, l = oracle.attn_fwd_rows(q, k, v, causal=True)
    s00 = (q[:, 0].astype(np.float64) * k[:, 0]).sum(-1) * oracle.default_scale(D)
    assert np.abs(o[:, 0] - v[:, 0]).max() == 0.0
    assert np.abs(m[:, 0] - s00).max() <= 1e-13 and np.all(l[:, 0] == 1.0)
    # 1 <= l_i <= i + 1 and m_i >= every visible score
    idx = np.arange(S)[None, :]
    assert np.all(l >= 1.0 - 1e-12) and np.all(l <= idx + 1 + 1e-9)


def _brute(q, k, v, causal, scale):
    """Direct softmax attention in pure Python (independent of the oracle)."""
    BH, S, D = q.shape
    o = np.zeros((BH, S, D))
    m = np.zeros((BH, S))
    l = np.zeros((BH, S))
    for b in range(BH):
        for i in range(S):
            js = range(i + 1) if causal else range(S)
            sc = [sum(float(q[b, i, d]) * float(k[b, j, d]) for d in range(D)) * scale for j in js]
            mx = max(sc)
            w = [math.exp(s - mx) for s in sc]
            tot = sum(w)
            m[b, i], l[b, i] = mx, tot
            for d in range(D):
                o[b, i, d] = sum(wj * float(v[b, j, d]) for wj, j in zip(w, js)) / tot
    return o, m, l


@pytest.mark.parametrize("causal", [True, False])
def test_oracle_brute_force_tiny(causal):
    rng = _rng(8)
    for S in range(1, 7):
        q, k, v = (rng.standard_normal((2, S, 4)).astype(np.float32) for _ in range(3))
        sc = 0.5
        o, m, l = oracle.attn_fwd_rows(q, k, v, causal=causal, scale=sc)
        ob, mb, lb = _brute(q, k, v, causal, sc)
        assert np.abs(o - ob).max() <= 1e-12 and np.abs(m - mb).max() <= 1e-12
        assert np.abs(l - lb).max() <= 1e-12


def test_oracle_row_subset_matches_full():
    rng = _rng(9)
    q, k, v = (rng.standard_normal((3, 90, 64)).astype(np.float32) for _ in range(3))
    o, m, l = oracle.attn_fwd_rows(q, k, v)
    rows = [0, 5, 63, 64, 89]
    o2, m2, l2 = oracle.attn_fwd_rows(q, k, v, rows=rows)
    assert np.array_equal(o2, o[:, rows]) and np.array_equal(m2, m[:, rows]) and np.array_equal(l2, l[:, rows])


def test_default_scale_is_float_rounded():
    """Reference scale: 1.0f / std::sqrt((float)D), rounded to float (fused_self_attention.cpp:30)."""
    for D in (32, 64, 128, 80):
        assert oracle.default_scale(D) == float(np.float32(1.0) / np.sqrt(np.float32(D)))
    assert oracle.default_scale(128) != 1.0 / math.sqrt(128)


def test_planted_mistakes_are_caught():
    """Each plausible mistake, planted in the oracle's inputs, breaks a check above."""
    rng = _rng(10)
    BH, S, D = 2, 40, 64
    q, k, v = (rng.standard_normal((BH, S, D)).astype(np.float32) for _ in range(3))
    good = oracle.attn_sdpa_f64(q, k, v, causal=True)
    sc = oracle.default_scale(D)
    mutants = {
        "scale off by 1%": oracle.attn_fwd_rows(q, k, v, causal=True, scale=sc * 1.01)[0],
        "mask dropped": oracle.attn_fwd_rows(q, k, v, causal=False)[0],
        "keys shifted by one": oracle.attn_fwd_rows(q, np.roll(k, 1, axis=1), v, causal=True)[0],
        "q and k swapped": oracle.attn_fwd_rows(k, q, v, causal=True)[0],
        "v transposed in head_dim": oracle.attn_fwd_rows(q, k, v[:, :, ::-1].copy(), causal=True)[0],
    }
    for name, o in mutants.items():
        assert np.abs(o - good).max() > 1e-3, f"planted mistake not caught: {name}"
    # and the K == 0 closed form catches a dropped scale-independent term (l off by one)
    _, _, l = oracle.attn_fwd_rows(q, np.zeros_like(k), v, causal=True)
    assert not np.all(l == np.arange(0, S)[None, :])


def test_causal_flop_count():
    for S in (1, 2, 7, 64):
        pairs = sum(1 for i in range(S) for j in range(S) if j <= i)
        assert oracle.causal_flops(1, 1, S, 16) == 4 * 16 * pairs
    assert oracle.causal_flops(4, 32, 4096, 128) == 549_890_031_616
