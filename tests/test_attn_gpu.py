"""GPU parity tests of the gfx950 attention forward, called through the C ABI
(pmkl_attn_fwd via ctypes) and through the torch operator.

Every case compares against the float64 oracle (oracle/attn_oracle.c) on the
same seeded inputs, at the stated tolerances (tests/parity.py).  Shapes cover
the reference's own test shape (4x16x1024x64 fp32, test_causal_attention.cpp:
146-148), the sizes of test_fused_self_attention.py:10-14 (B 2-3, H 16,
S 128, D 64/128, causal and not), sequence lengths that are not multiples of
any tile (the reference rejects them in its GPU launcher but its CPU operator
accepts them), S = 1, and the five benchmark configurations (all rows where
the oracle finishes in seconds, sampled rows plus size-independent invariants
at the two large ones).
"""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch_mod(device):
    import torch

    return torch


def _run_capi(q, k, v, device, causal=True, ml_dtype=None):
    import pmkl_amd
    import torch

    qd, kd, vd = (x.to(device) for x in (q, k, v))
    o, m, l = pmkl_amd.attn_fwd(qd, kd, vd, is_causal=causal, ml_dtype=ml_dtype)
    torch.cuda.synchronize()
    return o, m, l


SMALL_SHAPES = [
    (1, 1, 1, "S=1"),
    (1, 2, 16, "S<tile"),
    (2, 1, 33, "S%32!=0"),
    (1, 3, 64, "one key tile"),
    (2, 2, 100, "ragged"),
    (1, 2, 128, "one query tile"),
    (1, 1, 129, "query tile + 1"),
    (2, 1, 300, "ragged multi-tile"),
    (1, 2, 512, "multi-tile"),
]


@pytest.mark.parametrize("dtype", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_small_shapes_vs_oracle(device, dtype, D, causal):
    from pmkl_amd.workloads import small_inputs
    from tests.parity import check_outputs

    for i, (B, H, S, label) in enumerate(SMALL_SHAPES):
        tag = f"{dtype} D={D} causal={causal} B{B} H{H} S{S} ({label})"
        _say(f"case {tag}")
        q, k, v = small_inputs(B, H, S, D, dtype, seed=100 + i)
        o, m, l = _run_capi(q, k, v, device, causal=causal)
        check_outputs(q, k, v, o, m, l, dtype, causal=causal, label=tag)


# (S, D, causal) of the float m/l cases: S 200 at head_dim 64 runs the 8-wave
# kernel in its resident form, head_dim 128 at S 300 (few work items) its
# 4-wave streaming form; head_dim 128 from S 385 and causal head_dim 64 from
# S 512 run the 64-row kernel, whose epilogue has its own float m/l store.
ML_F32_SHAPES = [(200, 64, True), (300, 128, True), (520, 128, True), (520, 128, False), (1024, 64, True),
                 # head_dim 32 causal resident form (diagonal mask as the MFMA accumulator
                 # input, zero-start first tile), and the streaming form's LDS-staged O
                 (200, 32, True), (256, 32, True), (600, 64, False)]


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("S,D,causal", ML_F32_SHAPES)
def test_ml_float32_output(device, dtype, S, D, causal):
    """ml_dtype = F32 returns m and l without rounding them to the tensor dtype.
    m is the fp32 row max (1e-5).  l is the sum of the probabilities as rounded
    to the tensor dtype for the P*V product (the weights O is normalised by),
    so it sits within the relative rounding of those probabilities of the
    exact sum: 2^-8 for bf16, 2^-11 for fp16.  O meets the usual bound."""
    import torch
    from oracle import oracle
    from pmkl_amd.workloads import small_inputs
    from tests.parity import check_outputs, to_np

    _say(f"case ml f32 {dtype} B2 H2 S{S} D{D} causal={causal}")
    q, k, v = small_inputs(2, 2, S, D, dtype, seed=7 + S + D)
    o, m, l = _run_capi(q, k, v, device, causal=causal, ml_dtype=torch.float32)
    assert m.dtype == torch.float32 and l.dtype == torch.float32
    qn, kn, vn = (to_np(x).reshape(4, S, D) for x in (q, k, v))
    _, m_ref, l_ref = oracle.attn_fwd_rows(qn, kn, vn, causal=causal)
    assert np.allclose(to_np(m).reshape(4, S), m_ref, rtol=1e-5, atol=1e-5)
    rel = {"bf16": 2.0 ** -8, "fp16": 2.0 ** -11}[dtype]
    assert np.all(np.abs(to_np(l).reshape(4, S) - l_ref) <= rel * l_ref)
    # O against the oracle; m and l checked above in float32
    check_outputs(q, k, v, o, m.to(q.dtype), l.to(q.dtype), dtype, causal=causal,
                  label=f"ml f32 S{S} D{D}", check_ml=False)


# 16-bit head_dim 128 on both sides of the host's small-problem rule (fewer
# 256-row work items than CUs at S <= 384, causal 192 < S <= 352 -> the
# 4-wave kernel, else the 64-row kernel): (B, H, S, dtype, causal).
D128_RULE_SHAPES = [
    (2, 4, 192, "bf16", True), (2, 4, 193, "fp16", True),        # causal lower edge
    (2, 4, 352, "bf16", True), (2, 4, 353, "fp16", True),        # causal upper edge
    (2, 4, 384, "fp16", False), (2, 4, 385, "bf16", False),      # non-causal upper edge
    (1, 255, 256, "bf16", True), (1, 256, 256, "bf16", True),    # 255 vs 256 work items
]


@pytest.mark.parametrize("B,H,S,dtype,causal", D128_RULE_SHAPES)
def test_head_dim128_rule_edges(device, B, H, S, dtype, causal):
    from pmkl_amd.workloads import small_inputs
    from tests.parity import check_outputs

    tag = f"{dtype} B{B} H{H} S{S} D128 causal={causal}"
    _say(f"case {tag}")
    q, k, v = small_inputs(B, H, S, 128, dtype, seed=7700 + S + H)
    o, m, l = _run_capi(q, k, v, device, causal=causal)
    rows = _sample_rows(S, 16, seed=S) if B * H > 64 else None
    errs = check_outputs(q, k, v, o, m, l, dtype, causal=causal, rows=rows, label=tag)
    _say(f"{tag}: {errs}")


# fp32 on both sides of the host's key-split rule (the 128-row fp32 kernel's
# workgroups on fewer than half the CUs and S <= 1024 -> 32-row workgroups
# whose waves split the key tiles): (B, H, S, D, causal, rows sampled).
F32_RULE_SHAPES = [
    (1, 1, 1024, 64, True, False),    # split kernel at its largest S, 32 key tiles over 4 waves
    (1, 1, 1025, 64, True, False),    # one past: the 128-row kernel
    (1, 3, 700, 128, False, False),   # split kernel, non-causal, ragged
    (4, 40, 384, 64, True, True),     # 480 workgroups of 128 rows: the 128-row kernel
    (2, 8, 200, 32, True, False),     # split kernel, head_dim 32, ragged
]


@pytest.mark.parametrize("B,H,S,D,causal,sampled", F32_RULE_SHAPES)
def test_fp32_both_kernels(device, B, H, S, D, causal, sampled):
    from pmkl_amd.workloads import small_inputs
    from tests.parity import check_outputs

    tag = f"fp32 B{B} H{H} S{S} D{D} causal={causal}"
    _say(f"case {tag}")
    q, k, v = small_inputs(B, H, S, D, "fp32", seed=7500 + S + H)
    o, m, l = _run_capi(q, k, v, device, causal=causal)
    rows = _sample_rows(S, 16, seed=S) if sampled else None
    errs = check_outputs(q, k, v, o, m, l, "fp32", causal=causal, rows=rows, label=tag)
    _say(f"{tag}: {errs}")


def test_reference_test_shape_fp32(device):
    """The reference's GPU test: {4,16,1024,64} fp32, U(-1.05,1.05), all_close 1e-5."""
    from pmkl_amd.workloads import small_inputs
    from tests.parity import check_outputs

    q, k, v = small_inputs(4, 16, 1024, 64, "fp32", seed=2024, dist="uniform")
    o, m, l = _run_capi(q, k, v, device)
    check_outputs(q, k, v, o, m, l, "fp32", label="reference shape fp32")


@pytest.mark.parametrize("name", ["C1", "C2", "C5"])
def test_config_all_rows(device, name):
    from pmkl_amd.workloads import WORKLOADS, torch_dtype, host_inputs
    from tests.parity import check_outputs
    import torch

    w = WORKLOADS[name]
    _say(f"config {name} {w.shape} {w.dtype}")
    q, k, v = (torch.from_numpy(a).to(torch_dtype(w.dtype)) for a in host_inputs(w))
    o, m, l = _run_capi(q, k, v, device)
    errs = check_outputs(q, k, v, o, m, l, w.dtype, label=name)
    _say(f"{name}: {errs}")


def _sample_rows(S, n_random, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    fixed = [0, 1, 31, 32, 63, 64, 127, 128, 129, 255, 256, S // 2, S - 129, S - 128, S - 65, S - 64, S - 2, S - 1]
    rnd = rng.choice(S, size=n_random, replace=False).tolist()
    return sorted(set(r for r in fixed + rnd if 0 <= r < S))


# Heads (flattened b * H + h) checked on every row at the full-size configs:
# the first and last head and one in the middle (C3: batch 1 head 31).
FULL_HEADS = {"C3": (0, 63, 127), "C4": (0, 15)}


def check_full_heads(q, k, v, o, m, l, dtype, heads, label):
    """Every row of the given flattened heads against the oracle, as the
    reference's GPU test checks every element (test/test_causal_attention.cpp:197-204)."""
    from tests.parity import check_outputs

    B, H, S, D = q.shape
    idx = list(heads)
    sel = lambda t, shape: t.reshape(B * H, *shape)[idx].reshape(1, len(idx), *shape)   # noqa: E731
    return check_outputs(sel(q, (S, D)), sel(k, (S, D)), sel(v, (S, D)), sel(o.cpu(), (S, D)),
                         sel(m.cpu(), (S,)), sel(l.cpu(), (S,)), dtype, label=label)


@pytest.mark.parametrize("name", ["C3", "C4"])
def test_config_sampled_rows(device, name):
    """Full-size C3 / C4: every row of three (C3) / two (C4) whole heads, and in
    every head a fixed set of rows (tile edges, first and last rows, random
    rows), against the oracle."""
    from pmkl_amd.workloads import WORKLOADS, torch_dtype, host_inputs
    from tests.parity import check_outputs
    import torch

    w = WORKLOADS[name]
    _say(f"config {name} {w.shape} {w.dtype}")
    q, k, v = (torch.from_numpy(a).to(torch_dtype(w.dtype)) for a in host_inputs(w))
    o, m, l = _run_capi(q, k, v, device)
    errs = check_full_heads(q, k, v, o, m, l, w.dtype, FULL_HEADS[name], label=f"{name} full heads")
    _say(f"{name}: all rows of heads {FULL_HEADS[name]} {errs}")
    rows = _sample_rows(w.S, 24 if name == "C3" else 12, seed=w.seed)
    errs = check_outputs(q, k, v, o, m, l, w.dtype, rows=rows, label=name)
    _say(f"{name}: rows {len(rows)} {errs}")
    # invariants over all rows: finite, l in [1, i+1], O within the V range of its prefix bound
    ln = l.float().cpu().numpy().reshape(w.B * w.H, w.S)
    idx = np.arange(w.S)[None, :]
    assert np.isfinite(ln).all()
    assert (ln >= 1.0 - 1e-2).all() and (ln <= (idx + 1) * (1 + 2.0 ** -7) + 1e-2).all()
    vmax = float(v.float().abs().max())
    assert float(o.float().abs().max()) <= vmax * (1 + 2.0 ** -7)


@pytest.mark.parametrize("B,H,S,D,dtype,causal", [
    (4, 64, 512, 128, "bf16", False),   # 512 items, XCD-grouped order
    (2, 65, 512, 128, "fp16", True),    # 260 items: last round ragged, plain order
    (1, 256, 384, 128, "bf16", True),   # 512 items, half of the last q-tile's waves idle
])
def test_many_items_per_workgroup(device, B, H, S, D, dtype, causal):
    """More work items than CUs: the 64-row kernel's workgroups each run several
    (head, query tile) items back to back, streaming the next item's first K/V
    tiles during the current one's last iterations."""
    from pmkl_amd.workloads import small_inputs
    from tests.parity import check_outputs

    tag = f"{dtype} B{B} H{H} S{S} D{D} causal={causal}"
    _say(f"case {tag}")
    q, k, v = small_inputs(B, H, S, D, dtype, seed=7000 + H)
    o, m, l = _run_capi(q, k, v, device, causal=causal)
    rows = _sample_rows(S, 16, seed=S + H)
    errs = check_outputs(q, k, v, o, m, l, dtype, causal=causal, rows=rows, label=tag)
    _say(f"{tag}: {errs}")


# (D, S): every sequence length class of the resident 8-wave form (all key
# tiles in LDS at once): 5 to 8 row blocks of 32 (the SIMD pairing of short
# and long blocks changes with each), ragged last blocks and tiles, and the
# head_dim-128 limit of two key tiles.
RESIDENT_SHAPES = [(32, 160), (32, 193), (32, 224), (32, 255), (64, 192), (64, 225), (64, 256),
                   (128, 65), (128, 127), (128, 128)]


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("causal", [True, False])
def test_resident_short_sequences(device, dtype, causal):
    """Short sequences (S <= 256, S <= 128 at head_dim 128) run the 8-wave
    kernel with every key tile resident in LDS and SIMD-balanced row blocks:
    all rows against the oracle."""
    from pmkl_amd.workloads import small_inputs
    from tests.parity import check_outputs

    for i, (D, S) in enumerate(RESIDENT_SHAPES):
        B, H = 2, 3
        tag = f"{dtype} B{B} H{H} S{S} D{D} causal={causal} (resident)"
        _say(f"case {tag}")
        q, k, v = small_inputs(B, H, S, D, dtype, seed=7300 + 10 * i)
        o, m, l = _run_capi(q, k, v, device, causal=causal)
        check_outputs(q, k, v, o, m, l, dtype, causal=causal, label=tag)


@pytest.mark.parametrize("S", [513, 1000, 2048])
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("causal", [True, False])
def test_head_dim64_four_wave_range(device, S, dtype, causal):
    """head_dim 64 at 512 < S <= 2048 runs the MFMA kernel (4-wave, 128-row
    workgroups when causal, 8-wave otherwise): sampled rows against the
    oracle."""
    from pmkl_amd.workloads import small_inputs
    from tests.parity import check_outputs

    B, H, D = 1, 3, 64
    tag = f"{dtype} B{B} H{H} S{S} D{D} causal={causal}"
    _say(f"case {tag}")
    q, k, v = small_inputs(B, H, S, D, dtype, seed=7100 + S)
    o, m, l = _run_capi(q, k, v, device, causal=causal)
    rows = _sample_rows(S, 24, seed=S)
    errs = check_outputs(q, k, v, o, m, l, dtype, causal=causal, rows=rows, label=tag)
    _say(f"{tag}: {errs}")


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("slope", [2.0, 0.4])
@pytest.mark.parametrize("causal", [True, False])
def test_running_max_grows_every_tile(device, dtype, slope, causal):
    """Scores that rise along the keys (s_ij ~ slope * j plus noise): the
    running row max grows on every key tile (slope 2: by ~128 per 64 keys,
    past the 16-bit kernels' lazy-rescale threshold each tile; slope 0.4:
    every other tile), so the O^T accumulators are rescaled over and over
    between MFMAs.  Several work items per workgroup (B H = 260 heads)."""
    import torch

    from pmkl_amd.workloads import torch_dtype
    from tests.parity import check_outputs

    B, H, S, D = 2, 130, 512, 128
    tag = f"{dtype} slope {slope} causal={causal}"
    _say(f"case {tag}")
    g = torch.Generator().manual_seed(91)
    u = torch.randn(D, generator=g)
    u = u / u.norm()
    a = (slope * D ** 0.5) ** 0.5          # |q| * |k_j| / sqrt(D) = slope * j
    j = torch.arange(S, dtype=torch.float32)
    q = a * u.expand(B, H, S, D) + 0.3 * torch.randn(B, H, S, D, generator=g)
    k = (a * j[:, None]) * u
    k = k.expand(B, H, S, D) + 0.3 * torch.randn(B, H, S, D, generator=g)
    v = torch.randn(B, H, S, D, generator=g)
    q, k, v = (x.to(torch_dtype(dtype)) for x in (q, k, v))
    o, m, l = _run_capi(q, k, v, device, causal=causal)
    rows = _sample_rows(S, 24, seed=int(slope * 10) + causal)
    errs = check_outputs(q, k, v, o, m, l, dtype, causal=causal, rows=rows, label=tag)
    _say(f"{tag}: {errs}")


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("S,D,causal", [(256, 32, True), (200, 32, True), (256, 64, True), (600, 64, False)])
def test_running_max_grows_short(device, dtype, S, D, causal):
    """Rising scores as in test_running_max_grows_every_tile (slope 2: the
    running max passes the lazy-rescale threshold on every key tile) on the
    8-wave kernel: its resident form at head_dim 32 and 64, where every tile
    after a wave's first rescales O and l, and its streaming form (S 600,
    non-causal head_dim 64), every row against the oracle."""
    import torch

    from pmkl_amd.workloads import torch_dtype
    from tests.parity import check_outputs

    B, H = 2, 3
    tag = f"{dtype} rising scores B{B} H{H} S{S} D{D} causal={causal}"
    _say(f"case {tag}")
    g = torch.Generator().manual_seed(93 + S + D)
    u = torch.randn(D, generator=g)
    u = u / u.norm()
    a = (2.0 * D ** 0.5) ** 0.5
    j = torch.arange(S, dtype=torch.float32)
    q = a * u.expand(B, H, S, D) + 0.3 * torch.randn(B, H, S, D, generator=g)
    k = (a * j[:, None]) * u
    k = k.expand(B, H, S, D) + 0.3 * torch.randn(B, H, S, D, generator=g)
    v = torch.randn(B, H, S, D, generator=g)
    q, k, v = (x.to(torch_dtype(dtype)) for x in (q, k, v))
    o, m, l = _run_capi(q, k, v, device, causal=causal)
    errs = check_outputs(q, k, v, o, m, l, dtype, causal=causal, label=tag)
    _say(f"{tag}: {errs}")


@pytest.mark.parametrize("dtype", ["bf16", "fp16", "fp32"])
def test_closed_forms(device, dtype):
    """K == 0: O_i = mean(V_0..V_i), m_i = 0, l_i = i + 1 (every tile, diagonal included).
    V == c: O == c.  Row 0: O_0 = V_0."""
    import torch
    from pmkl_amd.workloads import small_inputs, torch_dtype

    B, H, S, D = 1, 2, 300, 64
    q, k, v = small_inputs(B, H, S, D, dtype, seed=11)
    kz = torch.zeros_like(k)
    o, m, l = _run_capi(q, kz, v, device)
    vf = v.double()
    prefix_mean = vf.cumsum(2) / torch.arange(1, S + 1, dtype=torch.float64).view(1, 1, S, 1)
    tol = {"fp32": 1e-5, "fp16": 2e-3, "bf16": 1e-2}[dtype]
    assert (o.double().cpu() - prefix_mean).abs().max().item() <= tol
    assert m.double().abs().max().item() == 0.0
    lref = torch.arange(1, S + 1, dtype=torch.float64).view(1, 1, S).expand(B, H, S)
    rel = {"fp32": 1e-5, "fp16": 2.0 ** -10, "bf16": 2.0 ** -7}[dtype]
    assert ((l.double().cpu() - lref).abs() <= rel * lref).all()
    c = torch.full_like(v, 0.71875)
    o2, _, _ = _run_capi(q, k, c, device)
    assert (o2.double().cpu() - 0.71875).abs().max().item() <= tol
    o3, _, _ = _run_capi(q, k, v, device)
    assert (o3[:, :, 0].double().cpu() - v[:, :, 0].double()).abs().max().item() <= tol


def test_head_permutation_and_prefix(device):
    """Heads are independent (permuting heads permutes outputs bit-exactly) and
    causal rows < S' of a length-S problem equal the length-S' problem (m
    bit-exactly, O and l to one bf16 rounding step)."""
    import torch
    from pmkl_amd.workloads import small_inputs

    q, k, v = small_inputs(2, 3, 384, 128, "bf16", seed=5)
    o, m, l = _run_capi(q, k, v, device)
    perm = torch.tensor([4, 0, 5, 2, 1, 3])
    qp, kp, vp = (x.reshape(6, 384, 128)[perm].reshape(2, 3, 384, 128) for x in (q, k, v))
    op, mp, lp = _run_capi(qp, kp, vp, device)
    assert torch.equal(op.reshape(6, 384, 128), o.reshape(6, 384, 128)[perm.to(o.device)])
    assert torch.equal(mp.reshape(6, 384), m.reshape(6, 384)[perm.to(m.device)])
    # Prefix: the row max is exact in both problems; O and l may differ by
    # rounding because the exponential offset is refreshed per wave of rows.
    Sp = 200
    o2, m2, l2 = _run_capi(q[:, :, :Sp].contiguous(), k[:, :, :Sp].contiguous(), v[:, :, :Sp].contiguous(), device)
    assert torch.equal(m2, m[:, :, :Sp])
    assert (o2.float() - o[:, :, :Sp].float()).abs().max().item() <= 2 ** -7
    assert ((l2.float() - l[:, :, :Sp].float()).abs() <= 2 ** -7 * l[:, :, :Sp].float()).all()


def test_deterministic(device):
    import torch
    from pmkl_amd.workloads import small_inputs

    q, k, v = small_inputs(2, 4, 1000, 128, "bf16", seed=9)
    a = _run_capi(q, k, v, device)
    b = _run_capi(q, k, v, device)
    assert all(torch.equal(x, y) for x, y in zip(a, b))


def test_strided_bshd_inputs(device):
    """q/k/v given as [B, S, H, D] memory viewed as [B, H, S, D] (strided) give
    the same bits as contiguous inputs; outputs are written with o strides."""
    import torch
    import pmkl_amd
    from pmkl_amd.workloads import small_inputs

    B, H, S, D = 2, 4, 257, 64
    q, k, v = small_inputs(B, H, S, D, "fp16", seed=12)
    ref = _run_capi(q, k, v, device)
    qs, ks, vs = (x.transpose(1, 2).contiguous().to(device).transpose(1, 2) for x in (q, k, v))
    assert not qs.is_contiguous()
    out = _run_capi(qs, ks, vs, device)
    assert all(torch.equal(x, y) for x, y in zip(ref, out))
    # strided output buffer ([B, S, H, D] memory)
    ob = torch.empty((B, S, H, D), dtype=q.dtype, device=device).transpose(1, 2)
    o, m, l = pmkl_amd.attn_fwd(q.to(device), k.to(device), v.to(device), out=ob)
    torch.cuda.synchronize()
    assert torch.equal(o, ref[0])


@pytest.mark.parametrize("B,H,S,D", [(1, 3, 200, 64), (2, 2, 131, 128)])
def test_strided_bshd_fp32_against_oracle(device, B, H, S, D):
    """fp32 (the key-split kernel at these sizes): q/k/v as [B, S, H, D]
    memory viewed as [B, H, S, D], and the output written through a strided
    [B, S, H, D] view, against the oracle; equal bit for bit to the
    contiguous call."""
    import torch
    import pmkl_amd
    from pmkl_amd.workloads import small_inputs
    from tests.parity import check_outputs

    tag = f"fp32 strided B{B} H{H} S{S} D{D}"
    _say(f"case {tag}")
    q, k, v = small_inputs(B, H, S, D, "fp32", seed=7600 + S)
    qs, ks, vs = (x.transpose(1, 2).contiguous().to(device).transpose(1, 2) for x in (q, k, v))
    assert not qs.is_contiguous()
    ob = torch.empty((B, S, H, D), dtype=q.dtype, device=device).transpose(1, 2)
    o, m, l = pmkl_amd.attn_fwd(qs, ks, vs, is_causal=True, out=ob)
    torch.cuda.synchronize()
    check_outputs(q, k, v, o, m, l, "fp32", causal=True, label=tag)
    ref = _run_capi(q, k, v, device)
    assert all(torch.equal(x, y) for x, y in zip(ref, (o, m, l)))


def test_output_canaries(device):
    """Nothing is written outside O, m, l: guard regions before and after stay
    intact, and poisoned (NaN) outputs are fully overwritten."""
    import torch
    import pmkl_amd
    from pmkl_amd.workloads import small_inputs

    B, H, S, D = 1, 3, 333, 128
    q, k, v = (x.to(device) for x in small_inputs(B, H, S, D, "bf16", seed=13))
    n, nr, pad = B * H * S * D, B * H * S, 4096
    ob = torch.full((n + 2 * pad,), float("nan"), dtype=torch.bfloat16, device=device)
    mb = torch.full((nr + 2 * pad,), float("nan"), dtype=torch.bfloat16, device=device)
    lb = torch.full((nr + 2 * pad,), float("nan"), dtype=torch.bfloat16, device=device)
    o = ob[pad:pad + n].view(B, H, S, D)
    m = mb[pad:pad + nr].view(B, H, S)
    l = lb[pad:pad + nr].view(B, H, S)
    pmkl_amd.attn_fwd(q, k, v, out=o, out_m=m, out_l=l)
    torch.cuda.synchronize()
    for buf, inner in ((ob, n), (mb, nr), (lb, nr)):
        assert torch.isnan(buf[:pad]).all() and torch.isnan(buf[pad + inner:]).all()
        assert torch.isfinite(buf[pad:pad + inner]).all()


def test_torch_operator_device_branch(device):
    """pmkl_pytorch_ext.fused_self_attention_fw on ROCm tensors = the C ABI result."""
    import torch
    from pmkl_amd import pmkl_pytorch_ext
    from pmkl_amd.pmkl_function import fused_self_attention
    from pmkl_amd.workloads import small_inputs

    q, k, v = small_inputs(3, 16, 128, 128, "bf16", seed=21)
    qd, kd, vd = (x.to(device) for x in (q, k, v))
    for causal in (True, False):
        ref = _run_capi(q, k, v, device, causal=causal)
        out = pmkl_pytorch_ext.fused_self_attention_fw(qd, kd, vd, causal)
        torch.cuda.synchronize()
        assert all(torch.equal(x, y) for x, y in zip(ref, out))
        out2 = fused_self_attention(qd, kd, vd, causal)
        torch.cuda.synchronize()
        assert all(torch.equal(x, y) for x, y in zip(ref, out2))
        assert out[0].is_contiguous() and out[1].shape == (3, 16, 128)


def test_torch_operator_errors(device):
    import torch
    from pmkl_amd import pmkl_pytorch_ext

    q = torch.randn(1, 2, 64, 80, device=device, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="head_dim 80"):
        pmkl_pytorch_ext.fused_self_attention_fw(q, q, q, True)
    q64 = torch.randn(1, 2, 64, 64, device=device, dtype=torch.float64)
    with pytest.raises(RuntimeError, match="float32, float16 and bfloat16"):
        pmkl_pytorch_ext.fused_self_attention_fw(q64, q64, q64, True)


def test_cpp_drop_in_header(device):
    """The C++ test binary (pmkl::nlp::causal_attention_forward) passes."""
    exe = ROOT / "tests" / "cpp" / "_bin" / "test_causal_attention"
    assert exe.exists(), "C++ test not built (run __graft_entry__.build())"
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=110)
    _say(res.stdout[-2000:])
    assert res.returncode == 0, res.stdout + res.stderr
