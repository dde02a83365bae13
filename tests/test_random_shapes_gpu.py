"""Fixed-seed random sweep of the device forward and backward over shapes the
hand-picked cases do not hit: batch, heads and sequence length drawn at
random (S from 1 to 700, log-uniform, so that ragged tiles, single tiles and
multi-item workgroups all occur), every head_dim and dtype, causal or not.
Each case runs the forward against the float64 forward oracle
(tests/parity.py bounds) and then the backward, fed with that forward's m and
l, against the float64 backward oracle (bounds of test_attn_bwd_gpu.py),
without the forward's output and (S > 1) with it.
The case list is a pure function of the seed, so a failure names a case that
reruns identically.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

N_CASES = 24


def _cases(seed=20261202, n=N_CASES):
    rng = np.random.Generator(np.random.PCG64(seed))
    out = []
    for i in range(n):
        S = int(np.clip(np.round(np.exp(rng.uniform(0.0, np.log(700.0)))), 1, 700))
        out.append(dict(B=int(rng.integers(1, 3)), H=int(rng.integers(1, 4)), S=S,
                        D=int(rng.choice([32, 64, 128])), dtype=str(rng.choice(["bf16", "fp16", "fp32"])),
                        causal=bool(rng.integers(0, 2)), seed=7000 + i))
    return out


@pytest.mark.parametrize("case", _cases(), ids=lambda c: "B{B}H{H}S{S}D{D}-{dtype}-{c}".format(
    c="causal" if c["causal"] else "full", **{k: v for k, v in c.items() if k != "causal"}))
def test_random_shape_forward_and_backward(device, case):
    import torch

    import pmkl_amd
    from oracle import oracle
    from pmkl_amd.workloads import small_inputs, torch_dtype
    from tests.parity import check_outputs
    from tests.test_attn_bwd_gpu import _check, _np, _say, _term_floors

    B, H, S, D, dtype, causal = (case[k] for k in ("B", "H", "S", "D", "dtype", "causal"))
    tag = f"random B{B} H{H} S{S} D{D} {dtype} causal={causal} seed={case['seed']}"
    _say(f"case {tag}")
    q, k, v = small_inputs(B, H, S, D, dtype, seed=case["seed"])
    qd, kd, vd = (x.to("cuda:0") for x in (q, k, v))
    o, m, l = pmkl_amd.attn_fwd(qd, kd, vd, is_causal=causal)
    torch.cuda.synchronize()
    check_outputs(q, k, v, o, m, l, dtype, causal=causal, label=tag)

    rng = np.random.Generator(np.random.PCG64(case["seed"] + 17))
    do = torch.from_numpy(rng.standard_normal((B, H, S, D)).astype(np.float32)).to(torch_dtype(dtype))
    dq, dk, dv = pmkl_amd.attn_bwd(do.to("cuda:0"), qd, kd, vd, m, l, is_causal=causal)
    torch.cuda.synchronize()
    r = lambda t: _np(t).reshape(B * H, S, D)
    mn, ln = _np(m).reshape(B * H, S), _np(l).reshape(B * H, S)
    ref = oracle.attn_bwd(r(q), r(k), r(v), r(do), mn, ln, causal=causal)
    fl = _term_floors(r(q), r(k), r(v), r(do), mn, ln, causal) if dtype == "fp32" else (0.0, 0.0, 0.0)
    _say(f"  {_check([r(dq), r(dk), r(dv)], ref, dtype, tag, fl)}")
    # The autograd path's call: row terms from <dout, O> (not at S = 1, where
    # every row has one visible key and the exact dq is 0: see
    # test_attn_bwd_gpu.test_bwd_with_forward_output).
    if S > 1:
        dq, dk, dv = pmkl_amd.attn_bwd(do.to("cuda:0"), qd, kd, vd, m, l, is_causal=causal, out=o)
        torch.cuda.synchronize()
        _say(f"  with O {_check([r(dq), r(dk), r(dv)], ref, dtype, tag + ' with O', fl)}")


N_MANY = 12


def _many_head_cases(seed=20261203, n=N_MANY):
    """Many heads (B 2-8, H 16-40) at S 129-1,100: the other side of the
    small-problem kernel rules (several work items per workgroup of the 64-row
    kernel, the fp32 kernel of 128-row workgroups)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    out = []
    for i in range(n):
        S = int(np.round(np.exp(rng.uniform(np.log(129.0), np.log(1100.0)))))
        out.append(dict(B=int(rng.integers(2, 9)), H=int(rng.integers(16, 41)), S=S,
                        D=int(rng.choice([64, 128])), dtype=str(rng.choice(["bf16", "fp16", "fp32"])),
                        causal=bool(rng.integers(0, 2)), seed=7200 + i))
    return out


@pytest.mark.parametrize("case", _many_head_cases(), ids=lambda c: "B{B}H{H}S{S}D{D}-{dtype}-{c}".format(
    c="causal" if c["causal"] else "full", **{k: v for k, v in c.items() if k != "causal"}))
def test_random_shape_forward_many_heads(device, case):
    """Forward only, every head, sampled rows (first, last, tile edges and 8
    random ones) against the float64 oracle."""
    import torch

    import pmkl_amd
    from pmkl_amd.workloads import small_inputs
    from tests.parity import check_outputs
    from tests.test_attn_bwd_gpu import _say

    B, H, S, D, dtype, causal = (case[k] for k in ("B", "H", "S", "D", "dtype", "causal"))
    tag = f"random many heads B{B} H{H} S{S} D{D} {dtype} causal={causal} seed={case['seed']}"
    _say(f"case {tag}")
    q, k, v = small_inputs(B, H, S, D, dtype, seed=case["seed"])
    o, m, l = pmkl_amd.attn_fwd(q.to("cuda:0"), k.to("cuda:0"), v.to("cuda:0"), is_causal=causal)
    torch.cuda.synchronize()
    rng = np.random.Generator(np.random.PCG64(case["seed"]))
    fixed = [0, 1, 63, 64, 127, 128, 255, 256, S // 2, S - 65, S - 64, S - 1]
    rows = sorted(set(r for r in fixed + rng.choice(S, size=8, replace=False).tolist() if 0 <= r < S))
    _say(f"  {check_outputs(q, k, v, o, m, l, dtype, causal=causal, rows=rows, label=tag)}")


N_SHORT = 120


def _short_cases(seed=20261204, n=N_SHORT):
    """Short sequences (S 1-300) at head_dim 32 and 64 in the 16-bit dtypes,
    mostly causal, with float m/l on some: the 8-wave kernel's resident form
    (diagonal mask as the score MFMA's accumulator input at head_dim 32, every
    row-block pairing) and its streaming form just above it."""
    rng = np.random.Generator(np.random.PCG64(seed))
    out = []
    for i in range(n):
        out.append(dict(B=int(rng.integers(1, 4)), H=int(rng.integers(1, 7)), S=int(rng.integers(1, 301)),
                        D=int(rng.choice([32, 32, 64])), dtype=str(rng.choice(["bf16", "fp16"])),
                        causal=bool(rng.random() < 0.75), ml32=bool(rng.random() < 0.25), seed=7400 + i))
    return out


def test_random_short_sequences_forward(device):
    """Forward only, every row of every case against the float64 oracle; the
    cases run in one test (each is a few milliseconds) and each is named
    before it runs."""
    import torch

    import pmkl_amd
    from pmkl_amd.workloads import small_inputs
    from tests.parity import check_outputs
    from tests.test_attn_bwd_gpu import _say

    worst = 0.0
    for case in _short_cases():
        B, H, S, D, dtype, causal, ml32 = (case[k] for k in ("B", "H", "S", "D", "dtype", "causal", "ml32"))
        tag = f"random short B{B} H{H} S{S} D{D} {dtype} causal={causal} ml_f32={ml32} seed={case['seed']}"
        _say(f"case {tag}")
        q, k, v = small_inputs(B, H, S, D, dtype, seed=case["seed"])
        o, m, l = pmkl_amd.attn_fwd(q.to("cuda:0"), k.to("cuda:0"), v.to("cuda:0"), is_causal=causal,
                                    ml_dtype=torch.float32 if ml32 else None)
        torch.cuda.synchronize()
        if ml32:
            assert m.dtype == torch.float32 and l.dtype == torch.float32
            m, l = m.to(q.dtype), l.to(q.dtype)
        errs = check_outputs(q, k, v, o, m, l, dtype, causal=causal, label=tag, check_ml=not ml32)
        worst = max(worst, errs["worst_over_bound"])
    _say(f"{len(_short_cases())} short cases, worst O error / bound {worst:.3f}")
