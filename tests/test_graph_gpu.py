"""The forward and the allocation-free backward inside a captured HIP graph.

Serving loops capture their launches once and replay them.  pmkl_attn_fwd
and pmkl_attn_bwd_noalloc launch only kernels on the caller's stream (no
allocation, no memset, no host synchronisation), so both can be recorded by
torch's graph capture.  Each graph is replayed several times with eager work
in between (new inputs copied into the captured buffers, eager calls of the
same entry points, synchronisations), and every replay must equal the eager
result on the same inputs bit for bit.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _inputs(B, H, S, D, dtype, seed):
    import torch

    from pmkl_amd.workloads import small_inputs, torch_dtype

    q, k, v = small_inputs(B, H, S, D, dtype, seed=seed)
    rng = np.random.Generator(np.random.PCG64(seed + 1))
    do = torch.from_numpy(rng.standard_normal((B, H, S, D)).astype(np.float32)).to(torch_dtype(dtype))
    return [x.to("cuda:0") for x in (q, k, v, do)]


@pytest.mark.parametrize("dtype,D,S", [("bf16", 128, 1000), ("fp16", 64, 520), ("bf16", 32, 300)])
def test_forward_replays_match_eager(device, dtype, D, S):
    import torch

    import pmkl_amd

    B, H = 2, 3
    _say(f"case graph forward {dtype} D={D} S={S}")
    q, k, v, _ = _inputs(B, H, S, D, dtype, seed=900 + D)
    out = torch.empty_like(q)
    m = torch.empty((B, H, S), dtype=q.dtype, device=q.device)
    l = torch.empty_like(m)
    pmkl_amd.attn_fwd(q, k, v, is_causal=True, out=out, out_m=m, out_l=l)   # warm-up, outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        pmkl_amd.attn_fwd(q, k, v, is_causal=True, out=out, out_m=m, out_l=l)
    for rep in range(4):
        nq, nk, nv, _ = _inputs(B, H, S, D, dtype, seed=1000 + 10 * rep + D)
        q.copy_(nq)
        k.copy_(nk)
        v.copy_(nv)
        want = pmkl_amd.attn_fwd(nq, nk, nv, is_causal=True)   # eager, other buffers
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("o", "m", "l"), (out, m, l), want):
            assert torch.equal(a, b), f"replay {rep}: {name} differs from the eager call"
    _say("  4 replays equal the eager calls")


@pytest.mark.parametrize("dtype,D,S", [("bf16", 128, 700), ("fp16", 64, 300)])
def test_noalloc_backward_replays_match_eager(device, dtype, D, S):
    import torch

    import pmkl_amd
    from pmkl_amd import capi

    B, H = 1, 2
    _say(f"case graph backward (noalloc) {dtype} D={D} S={S}")
    q, k, v, do = _inputs(B, H, S, D, dtype, seed=1100 + D)
    o, m, l = pmkl_amd.attn_fwd(q, k, v, is_causal=True)
    grads = [torch.empty_like(q) for _ in range(3)]
    a = capi.make_bwd_args(do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), m.data_ptr(),
                           l.data_ptr(), grads[0].data_ptr(), grads[1].data_ptr(), grads[2].data_ptr(), 0, 0,
                           dtype=pmkl_amd.torch_dtype_to_pmkl(q.dtype), batch=B, heads=H, seq_len=S, head_dim=D,
                           is_causal=True)
    # first call on the device outside the capture (it looks up the array's address)
    assert capi.attn_bwd_noalloc_raw(a, torch.cuda.current_stream().cuda_stream) == capi.PMKL_OK, capi.last_error()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = capi.attn_bwd_noalloc_raw(a, torch.cuda.current_stream().cuda_stream)
    assert rc == capi.PMKL_OK, capi.last_error()
    for rep in range(4):
        nq, nk, nv, ndo = _inputs(B, H, S, D, dtype, seed=1200 + 10 * rep + D)
        no, nm, nl = pmkl_amd.attn_fwd(nq, nk, nv, is_causal=True)
        for dst, src in zip((q, k, v, do, o, m, l), (nq, nk, nv, ndo, no, nm, nl)):
            dst.copy_(src)
        want = pmkl_amd.attn_bwd(ndo, nq, nk, nv, nm, nl, is_causal=True, out=no)   # eager, own workspace
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for name, x, y in zip(("dq", "dk", "dv"), grads, want):
            assert torch.equal(x, y), f"replay {rep}: {name} differs from the eager call"
    _say("  4 replays equal the eager calls")
