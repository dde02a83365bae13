"""CPU tests that pin the float64 backward oracle (oracle_attn_bwd in
oracle/attn_oracle.c), the restatement of the reference's backward operator
pmkl_pytorch_ext/fused_self_attention.cpp:66-135 (gradients of O only, as the
reference's autograd backward, pmkl_function/__init__.py:25-32).

Pinned by:
  * the reference's own backward operator run in float64 (committed fixtures
    tests/golden/bwd_*.npz written by tests/golden/gen_golden.py from the
    build in oracle/_ref, and live where that build is present);
  * torch autograd through scaled_dot_product_attention in float64;
  * central differences of the forward oracle (d<O, dout>/dx);
  * closed forms: dv = P^T dout; with constant V, dq = dk = 0;
and plausible mistakes planted in the inputs are shown to break them.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"
BWD_FIXTURES = sorted(GOLDEN.glob("bwd_*.npz"))


def _load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def _sdpa_grads(q, k, v, dout, causal, scale=None):
    import torch

    ts = [torch.from_numpy(np.asarray(a, dtype=np.float64)).requires_grad_() for a in (q, k, v)]
    if scale is None:
        scale = oracle.default_scale(q.shape[-1])
    o = torch.nn.functional.scaled_dot_product_attention(*ts, is_causal=causal, scale=scale)
    o.backward(torch.from_numpy(np.asarray(dout, dtype=np.float64)))
    return tuple(t.grad.numpy() for t in ts)


def test_bwd_fixtures_present():
    assert len(BWD_FIXTURES) >= 4


@pytest.mark.parametrize("path", BWD_FIXTURES, ids=lambda p: p.stem)
def test_bwd_oracle_matches_reference_fp64_fixture(path):
    f = _load(path)
    B, H, S, D, causal = int(f["B"]), int(f["H"]), int(f["S"]), int(f["D"]), bool(f["causal"])
    q, k, v, do = (f[x].reshape(B * H, S, D) for x in ("q", "k", "v", "dout"))
    m, l = f["m_fp64"].reshape(B * H, S), f["l_fp64"].reshape(B * H, S)
    got = oracle.attn_bwd(q, k, v, do, m, l, causal=causal)
    for name, g in zip(("dq", "dk", "dv"), got):
        ref = f[f"{name}_fp64"].reshape(B * H, S, D)
        assert np.abs(g - ref).max() <= 1e-12 * max(1.0, np.abs(ref).max()), name


def test_bwd_oracle_live_against_reference_build():
    import torch

    ref = oracle.reference_op()
    if ref is None:
        pytest.skip("oracle/_ref not built (the reference tree is absent)")
    rng = _rng(91)
    for (B, H, S, D, causal) in [(1, 2, 23, 32, True), (1, 1, 30, 64, False)]:
        q, k, v, do = (rng.standard_normal((B, H, S, D)) for _ in range(4))
        t = [torch.from_numpy(x) for x in (q, k, v, do)]
        o, m, l = ref.fused_self_attention_fw(t[0], t[1], t[2], causal)
        dq_r, dk_r, dv_r = ref.fused_self_attention_bw(t[3], t[0], t[1], t[2], m, l, causal)
        r = lambda x: x.reshape(B * H, S, D)
        got = oracle.attn_bwd(r(q), r(k), r(v), r(do), m.numpy().reshape(B * H, S), l.numpy().reshape(B * H, S),
                              causal=causal)
        # float32 inputs to the oracle: compare at float32 input rounding
        for g, rr in zip(got, (dq_r, dk_r, dv_r)):
            assert np.abs(g - rr.numpy().reshape(B * H, S, D)).max() <= 1e-5


@pytest.mark.parametrize("causal", [True, False])
def test_bwd_oracle_vs_sdpa_autograd(causal):
    rng = _rng(31)
    for (BH, S, D) in [(2, 1, 32), (3, 19, 64), (1, 70, 128), (2, 33, 16)]:
        q, k, v, do = (rng.standard_normal((BH, S, D)).astype(np.float32) for _ in range(4))
        _, m, l = oracle.attn_fwd_rows(q, k, v, causal=causal)
        got = oracle.attn_bwd(q, k, v, do, m, l, causal=causal)
        want = _sdpa_grads(q, k, v, do, causal)
        for g, w in zip(got, want):
            assert np.abs(g - w).max() <= 1e-11


def test_bwd_oracle_central_differences():
    """d<O, dout>/dx from the forward oracle by central differences (float64
    forward on float32-exact perturbations is not possible, so the check runs
    at h = 2^-8 on inputs that are multiples of 2^-8: q + h stays exact in
    float32 and the second-order error is O(h^2))."""
    rng = _rng(4)
    BH, S, D = 1, 9, 8
    q, k, v, do = (np.round(rng.standard_normal((BH, S, D)) * 64) / 64 for _ in range(4))
    q, k, v = (x.astype(np.float32) for x in (q, k, v))
    _, m, l = oracle.attn_fwd_rows(q, k, v, causal=True)
    dq, dk, dv = oracle.attn_bwd(q, k, v, do, m, l, causal=True)
    h = 2.0 ** -8

    def loss(qq, kk, vv):
        o, _, _ = oracle.attn_fwd_rows(qq, kk, vv, causal=True)
        return float((o * do).sum())

    for (x, g, which) in ((q, dq, 0), (k, dk, 1), (v, dv, 2)):
        for idx in [(0, 0, 0), (0, 4, 3), (0, 8, 7), (0, 2, 5)]:
            xp, xm = x.copy(), x.copy()
            xp[idx] += h
            xm[idx] -= h
            args_p = [q, k, v]
            args_m = [q, k, v]
            args_p[which], args_m[which] = xp, xm
            fd = (loss(*args_p) - loss(*args_m)) / (2 * h)
            assert abs(fd - g[idx]) <= 2e-4 * max(1.0, abs(g[idx])), (which, idx, fd, g[idx])


def test_bwd_oracle_closed_forms():
    rng = _rng(8)
    BH, S, D = 2, 25, 32
    q, k, do = (rng.standard_normal((BH, S, D)).astype(np.float32) for _ in range(3))
    # constant V: O does not depend on q or k, so dq = dk = 0; dv_j = sum_i p_ij dout_i
    v = np.full((BH, S, D), 0.5, dtype=np.float32)
    _, m, l = oracle.attn_fwd_rows(q, k, v, causal=True)
    dq, dk, dv = oracle.attn_bwd(q, k, v, do, m, l, causal=True)
    assert np.abs(dq).max() <= 1e-12 and np.abs(dk).max() <= 1e-12
    # K == 0: p_ij = 1/(i+1) for j <= i, so dv_j = sum_{i>=j} dout_i / (i+1)
    kz = np.zeros_like(k)
    v2 = rng.standard_normal((BH, S, D)).astype(np.float32)
    _, m, l = oracle.attn_fwd_rows(q, kz, v2, causal=True)
    _, _, dv = oracle.attn_bwd(q, kz, v2, do, m, l, causal=True)
    w = np.zeros((S, S))
    for i in range(S):
        w[i, : i + 1] = 1.0 / (i + 1)
    want = np.einsum("ij,bid->bjd", w, do.astype(np.float64))
    assert np.abs(dv - want).max() <= 1e-12


def test_bwd_head_subset_matches_full():
    rng = _rng(12)
    BH, S, D = 4, 30, 32
    q, k, v, do = (rng.standard_normal((BH, S, D)).astype(np.float32) for _ in range(4))
    _, m, l = oracle.attn_fwd_rows(q, k, v, causal=True)
    full = oracle.attn_bwd(q, k, v, do, m, l, causal=True)
    sub = oracle.attn_bwd(q, k, v, do, m, l, causal=True, heads=[3, 1])
    for a, b in zip(full, sub):
        assert np.array_equal(a[[3, 1]], b)


def test_bwd_planted_mistakes_are_caught():
    rng = _rng(13)
    BH, S, D = 2, 24, 32
    q, k, v, do = (rng.standard_normal((BH, S, D)).astype(np.float32) for _ in range(4))
    want = _sdpa_grads(q, k, v, do, True)
    _, m, l = oracle.attn_fwd_rows(q, k, v, causal=True)
    sc = oracle.default_scale(D)
    mutants = {
        "scale off by 1%": oracle.attn_bwd(q, k, v, do, m, l, causal=True, scale=sc * 1.01),
        "mask dropped": oracle.attn_bwd(q, k, v, do, m, l, causal=False),
        "l off by 1%": oracle.attn_bwd(q, k, v, do, m, l * 1.01, causal=True),
        "q and k swapped": oracle.attn_bwd(k, q, v, do, m, l, causal=True),
        "dout shifted by one row": oracle.attn_bwd(q, k, v, np.roll(do, 1, axis=1), m, l, causal=True),
    }
    for name, got in mutants.items():
        assert max(np.abs(g - w).max() for g, w in zip(got, want)) > 1e-3, f"planted mistake not caught: {name}"
