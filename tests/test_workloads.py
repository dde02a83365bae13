"""CPU tests of the seeded benchmark inputs (pmkl_amd/workloads.py)."""
from __future__ import annotations

import numpy as np

from pmkl_amd.workloads import WORKLOADS, host_inputs, small_inputs


def test_configs_match_the_benchmark_table():
    shapes = {n: (w.dtype, w.B, w.H, w.S, w.D, w.seed) for n, w in WORKLOADS.items()}
    assert shapes == {
        "C1": ("fp32", 1, 4, 128, 64, 1001),
        "C2": ("fp16", 8, 16, 1024, 64, 1002),
        "C3": ("bf16", 4, 32, 4096, 128, 1003),
        "C4": ("bf16", 1, 16, 16384, 128, 1004),
        "C5": ("fp16", 64, 8, 256, 32, 1005),
    }


def test_inputs_are_deterministic():
    a = host_inputs(WORKLOADS["C1"])
    b = host_inputs(WORKLOADS["C1"])
    assert all(np.array_equal(x, y) for x, y in zip(a, b))
    assert all(x.dtype == np.float32 and x.shape == (1, 4, 128, 64) for x in a)


def test_c5_outlier_rows():
    w = WORKLOADS["C5"]
    q, k, v = host_inputs(w)
    rows = q.reshape(-1, w.D)
    norms = np.linalg.norm(rows, axis=1)
    # round(0.01 * B*H*S) rows scaled by 8: their norms sit far above sqrt(D)
    assert int(round(0.01 * w.B * w.H * w.S)) == 1311
    assert (norms > 4 * np.sqrt(w.D)).sum() == 1311


def test_small_inputs_dtype_and_seed():
    import torch

    a = small_inputs(1, 2, 5, 32, "bf16", seed=1)
    b = small_inputs(1, 2, 5, 32, "bf16", seed=1)
    c = small_inputs(1, 2, 5, 32, "bf16", seed=2)
    assert all(torch.equal(x, y) for x, y in zip(a, b))
    assert not torch.equal(a[0], c[0])
    assert a[0].dtype == torch.bfloat16


def test_causal_flops_counts_visible_pairs():
    from pmkl_amd.workloads import causal_flops

    for S in (1, 2, 7, 64):
        pairs = sum(1 for i in range(S) for j in range(S) if j <= i)
        assert causal_flops(1, 1, S, 16) == 4 * 16 * pairs
    assert causal_flops(4, 32, 4096, 128) == 549_890_031_616
