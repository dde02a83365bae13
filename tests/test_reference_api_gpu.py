"""GPU parity through the reference's own API surface, against the oracles.

The reference's callers reach this path as
  * ``pmkl_pytorch_ext.fused_self_attention_fw(q, k, v, is_causal)``
    (pmkl_pytorch_ext/fused_self_attention.cpp:139-173), and
  * ``pmkl_function.fused_self_attention(q, k, v, is_casual, debug=False)``
    (pmkl_pytorch_ext/pmkl_function/__init__.py:12-33), whose backward is
    ``fused_self_attention_bw`` (fused_self_attention.cpp:175-215),
imported by those top-level names as the reference's harness does
(pmkl_pytorch_ext/test/test_fused_self_attention.py:3).  Here both run on
ROCm tensors and every output is compared with the float64 oracles
(oracle/attn_oracle.c): the forward at the benchmark configurations C1, C2, C5
(all rows) and C3 (every head, sampled rows); the harness's own grid
(test_fused_self_attention.py:10-41: B 2-3, H 16, S 128, D 64/128, causal and
not, forward then out.sum().backward()) in fp32 (the harness's dtype) and the
16-bit dtypes, gradients included; strided [B, S, H, D] inputs and outputs;
and m, l kept in float32 at head_dim 128, fed on to the backward.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from oracle import oracle

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _config_inputs(name):
    import torch

    from pmkl_amd.workloads import WORKLOADS, host_inputs, torch_dtype

    w = WORKLOADS[name]
    q, k, v = (torch.from_numpy(a).to(torch_dtype(w.dtype)) for a in host_inputs(w))
    return w, q, k, v


def _sample_rows(S, n_random, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    fixed = [0, 1, 31, 32, 63, 64, 127, 128, 129, 255, 256, S // 2, S - 129, S - 128, S - 65, S - 64, S - 2, S - 1]
    rnd = rng.choice(S, size=n_random, replace=False).tolist()
    return sorted(set(r for r in fixed + rnd if 0 <= r < S))


@pytest.mark.parametrize("name", ["C1", "C2", "C5", "C3"])
def test_torch_op_and_autograd_forward_vs_oracle(device, name):
    """fused_self_attention_fw and fused_self_attention (device branch) at a
    benchmark configuration: all rows (C3: every row of heads 0, 63 and 127,
    and sampled rows of every head)."""
    import torch
    import pmkl_pytorch_ext
    from pmkl_function import fused_self_attention
    from tests.parity import check_outputs
    from tests.test_attn_gpu import FULL_HEADS, check_full_heads

    w, q, k, v = _config_inputs(name)
    rows = _sample_rows(w.S, 24, seed=w.seed) if name == "C3" else None
    qd, kd, vd = (x.to(device) for x in (q, k, v))
    _say(f"config {name} {w.shape} {w.dtype}: fused_self_attention_fw")
    o, m, l = pmkl_pytorch_ext.fused_self_attention_fw(qd, kd, vd, True)
    torch.cuda.synchronize()
    assert o.dtype == m.dtype == l.dtype == q.dtype and o.is_contiguous()
    errs = check_outputs(q, k, v, o, m, l, w.dtype, rows=rows, label=f"{name} fused_self_attention_fw")
    _say(f"PARITY {name} fused_self_attention_fw {errs}")
    if name == "C3":
        errs = check_full_heads(q, k, v, o, m, l, w.dtype, FULL_HEADS[name],
                                label=f"{name} fused_self_attention_fw full heads")
        _say(f"PARITY {name} fused_self_attention_fw all rows of heads {FULL_HEADS[name]} {errs}")
    del o, m, l
    _say(f"config {name}: pmkl_function.fused_self_attention")
    o, m, l = fused_self_attention(qd, kd, vd, True)
    torch.cuda.synchronize()
    errs = check_outputs(q, k, v, o, m, l, w.dtype, rows=rows, label=f"{name} fused_self_attention")
    _say(f"PARITY {name} fused_self_attention {errs}")
    if name == "C3":
        errs = check_full_heads(q, k, v, o, m, l, w.dtype, FULL_HEADS[name],
                                label=f"{name} fused_self_attention full heads")
        _say(f"PARITY {name} fused_self_attention all rows of heads {FULL_HEADS[name]} {errs}")


@pytest.mark.parametrize("dtype", ["fp32", "bf16", "fp16"])
def test_reference_harness_grid_device_autograd(device, dtype):
    """test_fused_self_attention.py:10-41 on the device: forward through the
    autograd entry, then out.sum().backward(); O, m, l against the forward
    oracle and dq, dk, dv against the backward oracle (on the m, l the
    forward returned, as the reference's autograd saves them)."""
    import torch
    from pmkl_function import fused_self_attention
    from pmkl_amd.workloads import small_inputs
    from tests.parity import check_outputs
    from tests.test_attn_bwd_gpu import _check, _np, _term_floors

    for bi, B in enumerate((2, 3)):
        H, S = 16, 128
        for D in (64, 128):
            for is_causal in (False, True):
                tag = f"harness {dtype} B{B} H{H} S{S} D{D} causal={is_causal}"
                _say(f"case {tag}")
                q, k, v = small_inputs(B, H, S, D, dtype, seed=800 + 10 * bi + D + int(is_causal))
                qg, kg, vg = (x.to(device).requires_grad_(True) for x in (q, k, v))
                out, m, l = fused_self_attention(qg, kg, vg, is_causal)
                loss = out.sum()
                loss.backward()
                torch.cuda.synchronize()
                check_outputs(q, k, v, out, m, l, dtype, causal=is_causal, label=tag)
                r = lambda t: _np(t).reshape(B * H, S, D)
                mn, ln = _np(m).reshape(B * H, S), _np(l).reshape(B * H, S)
                do = np.ones((B * H, S, D))
                ref = oracle.attn_bwd(r(q), r(k), r(v), do, mn, ln, causal=is_causal)
                fl = _term_floors(r(q), r(k), r(v), do, mn, ln, is_causal) if dtype == "fp32" else (0.0, 0.0, 0.0)
                errs = _check([r(qg.grad), r(kg.grad), r(vg.grad)], ref, dtype, tag, fl)
                _say(f"  grads (max rel err, worst/bound): {errs}")


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_strided_bshd_vs_oracle(device, dtype):
    """q, k, v held as [B, S, H, D] memory and viewed as [B, H, S, D]: the C ABI
    reads them in place (and writes a strided output); the torch operator
    passes them without copies.  Both against the oracle."""
    import torch
    import pmkl_amd
    import pmkl_pytorch_ext
    from pmkl_amd.workloads import small_inputs
    from tests.parity import check_outputs

    for (B, H, S, D) in [(2, 4, 257, 64), (1, 3, 520, 128), (2, 2, 190, 32)]:
        tag = f"strided {dtype} B{B} H{H} S{S} D{D}"
        _say(f"case {tag}")
        q, k, v = small_inputs(B, H, S, D, dtype, seed=900 + S)
        qs, ks, vs = (x.transpose(1, 2).contiguous().to(device).transpose(1, 2) for x in (q, k, v))
        assert not qs.is_contiguous()
        ob = torch.empty((B, S, H, D), dtype=qs.dtype, device=device).transpose(1, 2)
        o, m, l = pmkl_amd.attn_fwd(qs, ks, vs, is_causal=True, out=ob)
        torch.cuda.synchronize()
        assert o.data_ptr() == ob.data_ptr()
        check_outputs(q, k, v, o, m, l, dtype, label=tag + " C ABI")
        o2, m2, l2 = pmkl_pytorch_ext.fused_self_attention_fw(qs, ks, vs, False)
        torch.cuda.synchronize()
        check_outputs(q, k, v, o2, m2, l2, dtype, causal=False, label=tag + " torch op, non-causal")


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_ml_float32_head_dim128_into_backward(device, dtype):
    """m, l stored as float32 by the 64-row head_dim-128 kernel (S > 384):
    m to 1e-5 of the oracle's, l within the relative rounding of the
    probabilities it sums (2^-8 bf16, 2^-11 fp16); then the backward from
    those float32 m, l against the backward oracle."""
    import torch
    import pmkl_amd
    from pmkl_amd.workloads import small_inputs, torch_dtype
    from tests.parity import check_outputs, to_np
    from tests.test_attn_bwd_gpu import _check

    B, H, S, D = 1, 4, 520, 128
    q, k, v = small_inputs(B, H, S, D, dtype, seed=950)
    qd, kd, vd = (x.to(device) for x in (q, k, v))
    o, m, l = pmkl_amd.attn_fwd(qd, kd, vd, is_causal=True, ml_dtype=torch.float32)
    torch.cuda.synchronize()
    assert m.dtype == torch.float32 and l.dtype == torch.float32
    qn, kn, vn = (to_np(x).reshape(B * H, S, D) for x in (q, k, v))
    o_ref, m_ref, l_ref = oracle.attn_fwd_rows(qn, kn, vn)
    assert np.allclose(to_np(m).reshape(B * H, S), m_ref, rtol=1e-5, atol=1e-5)
    rel = {"bf16": 2.0 ** -8, "fp16": 2.0 ** -11}[dtype]
    assert np.all(np.abs(to_np(l).reshape(B * H, S) - l_ref) <= rel * l_ref)
    # O itself to the usual bound (m, l in the dtype, from a second call)
    o2, m2, l2 = pmkl_amd.attn_fwd(qd, kd, vd, is_causal=True)
    torch.cuda.synchronize()
    assert torch.equal(o, o2)
    check_outputs(q, k, v, o2, m2, l2, dtype, label=f"ml f32 D128 {dtype}")
    rng = np.random.Generator(np.random.PCG64(951))
    do = torch.from_numpy(rng.standard_normal((B, H, S, D)).astype(np.float32)).to(torch_dtype(dtype))
    dq, dk, dv = pmkl_amd.attn_bwd(do.to(device), qd, kd, vd, m, l, is_causal=True)
    torch.cuda.synchronize()
    r = lambda t: to_np(t).reshape(B * H, S, D)
    ref = oracle.attn_bwd(qn, kn, vn, r(do), to_np(m).reshape(B * H, S), to_np(l).reshape(B * H, S), causal=True)
    _check([r(dq), r(dk), r(dv)], ref, dtype, f"bwd from f32 m, l {dtype}")
