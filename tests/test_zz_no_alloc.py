"""GPU test of pmkl_attn_bwd_noalloc, the backward entry point that allocates
nothing (its per-row workspace lives in a fixed device array of the
library).  Called through the C ABI, it must give exactly the results of
pmkl_attn_bwd (same kernels, same arithmetic) on two calls in a row, the
second with a smaller input than the first; sizes past its maximum are
rejected with PMKL_EINVAL before anything is launched.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _both(B, H, S, D, dtype, causal, seed, with_o):
    """Runs pmkl_attn_bwd (torch-allocated workspace) and then
    pmkl_attn_bwd_noalloc on the same inputs; returns both (dq, dk, dv)."""
    import torch

    import pmkl_amd
    from pmkl_amd import capi
    from pmkl_amd.workloads import small_inputs, torch_dtype

    dev = torch.device("cuda:0")
    q, k, v = (x.to(dev) for x in small_inputs(B, H, S, D, dtype, seed=seed))
    rng = np.random.Generator(np.random.PCG64(seed + 1))
    do = torch.from_numpy(rng.standard_normal((B, H, S, D)).astype(np.float32)).to(torch_dtype(dtype)).to(dev)
    o, m, l = pmkl_amd.attn_fwd(q, k, v, is_causal=causal)
    ref = pmkl_amd.attn_bwd(do, q, k, v, m, l, is_causal=causal, out=o if with_o else None)
    got = tuple(torch.full_like(x, float("nan")) for x in ref)
    a = capi.make_bwd_args(do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr() if with_o else 0,
                           m.data_ptr(), l.data_ptr(), got[0].data_ptr(), got[1].data_ptr(), got[2].data_ptr(), 0, 0,
                           dtype=pmkl_amd.torch_dtype_to_pmkl(q.dtype), ml_dtype=pmkl_amd.torch_dtype_to_pmkl(m.dtype),
                           batch=B, heads=H, seq_len=S, head_dim=D, is_causal=causal)
    rc = capi.attn_bwd_noalloc_raw(a, torch.cuda.current_stream(dev).cuda_stream)
    assert rc == capi.PMKL_OK, capi.last_error()
    torch.cuda.synchronize()
    return ref, got


@pytest.mark.parametrize("dtype", ["bf16", "fp16", "fp32"])
def test_noalloc_backward_matches_workspace_backward(device, dtype):
    import torch

    # Two calls in a row, the second smaller: the second reuses the array the
    # first filled, and must not see anything of it.
    cases = [(2, 4, 700, 128, True, False), (1, 3, 257, 64, True, True), (1, 2, 100, 32, False, False)]
    for i, (B, H, S, D, causal, with_o) in enumerate(cases):
        tag = f"noalloc {dtype} B{B} H{H} S{S} D{D} causal={causal} with_o={with_o}"
        _say(f"case {tag}")
        ref, got = _both(B, H, S, D, dtype, causal, seed=1200 + 10 * i, with_o=with_o)
        for name, r, g in zip(("dq", "dk", "dv"), ref, got):
            assert torch.equal(r, g), f"{tag}: {name} differs from pmkl_attn_bwd"


def test_noalloc_backward_rejects_oversize(device):
    import torch

    import pmkl_amd
    from pmkl_amd import capi

    B, H, S, D = 1, 1, capi.PMKL_ATTN_BWD_NOALLOC_MAX_ROWS + 1, 64
    dev = torch.device("cuda:0")
    t = torch.zeros(16, dtype=torch.bfloat16, device=dev)   # never read: the call is rejected first
    p = t.data_ptr()
    a = capi.make_bwd_args(p, p, p, p, 0, p, p, p, p, p, 0, 0, dtype=capi.PMKL_DTYPE_BF16,
                           ml_dtype=capi.PMKL_DTYPE_BF16, batch=B, heads=H, seq_len=S, head_dim=D, is_causal=True)
    rc = capi.attn_bwd_noalloc_raw(a, torch.cuda.current_stream(dev).cuda_stream)
    assert rc == capi.PMKL_EINVAL
    assert "at most 1048576 query rows" in capi.last_error()
    del pmkl_amd
