"""GPU parity tests of the gfx950 attention backward (pmkl_attn_bwd through the
C ABI), against the float64 backward oracle (oracle_attn_bwd, the restatement
of pmkl_pytorch_ext/fused_self_attention.cpp:66-135).

The device forward runs first and its m, l (in the tensor dtype, as the
reference's autograd saves them) feed both the device backward and the
oracle, so both use the same probabilities P = exp(s - m) / l.

Tolerance: the 16-bit kernels round P and dS to the tensor dtype for the
MFMA products and round dq, dk, dv on output; accumulation is fp32.  Each
gradient tensor is held to max|g - g_ref| <= TOL * max|g_ref| (+ the half-ulp
output rounding of each element), TOL = 1.5e-2 for bf16 and 3e-3 for fp16.
The fp32 kernels keep every product and sum in fp32: TOL = 1e-5, relative
to the larger of max|g_ref| and the magnitude of the summed terms (for dq:
scale * max over (i, d) of sum_j P_ij (|dP_ij| + |D_i|) |k_jd|; dk alike with
q; dv: max of sum_i P_ij |dout_id|), because dP - D cancels: at S = 1 the
exact dq is 0 and both sides return rounding noise of that magnitude.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from oracle import oracle

pytestmark = pytest.mark.gpu

TOL = {"bf16": 1.5e-2, "fp16": 3e-3, "fp32": 1e-5}
MANT = {"bf16": 7, "fp16": 10, "fp32": 23}


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _np(t):
    import torch

    return t.detach().to("cpu", torch.float32).numpy().astype(np.float64)


def _run(B, H, S, D, dtype, causal, seed, with_o=False, dist="normal", heads=None, ml_dtype=None):
    import torch

    import pmkl_amd
    from pmkl_amd.workloads import small_inputs, torch_dtype

    q, k, v = small_inputs(B, H, S, D, dtype, seed=seed, dist=dist)
    rng = np.random.Generator(np.random.PCG64(seed + 17))
    do = torch.from_numpy(rng.standard_normal((B, H, S, D)).astype(np.float32)).to(torch_dtype(dtype))
    qd, kd, vd, dod = (x.to("cuda:0") for x in (q, k, v, do))
    o, m, l = pmkl_amd.attn_fwd(qd, kd, vd, is_causal=causal, ml_dtype=ml_dtype)
    dq, dk, dv = pmkl_amd.attn_bwd(dod, qd, kd, vd, m, l, is_causal=causal, out=o if with_o else None)
    torch.cuda.synchronize()
    r = lambda t: _np(t).reshape(B * H, S, D)
    ref = oracle.attn_bwd(r(q), r(k), r(v), r(do), _np(m).reshape(B * H, S), _np(l).reshape(B * H, S),
                          causal=causal, heads=heads)
    got = [r(x) if heads is None else r(x)[list(heads)] for x in (dq, dk, dv)]
    if dtype == "fp32":
        hs = list(range(B * H)) if heads is None else list(heads)
        fl = _term_floors(r(q)[hs], r(k)[hs], r(v)[hs], r(do)[hs], _np(m).reshape(B * H, S)[hs],
                          _np(l).reshape(B * H, S)[hs], causal)
        return got, ref, fl
    return got, ref, (0.0, 0.0, 0.0)


def _term_floors(q, k, v, do, m, l, causal):
    """Magnitudes of the summed terms of dq, dk, dv (float64, [BH, S, D]
    inputs, default scale): the error scale of an fp32 sum with cancellation."""
    sc = 1.0 / np.sqrt(q.shape[-1])
    fl = np.zeros(3)
    for h in range(q.shape[0]):
        s = sc * q[h] @ k[h].T
        if causal:
            s = np.where(np.tril(np.ones(s.shape, dtype=bool)), s, -np.inf)
        p = np.exp(s - m[h][:, None]) / l[h][:, None]
        dp = do[h] @ v[h].T
        dr = (p * dp).sum(axis=1, keepdims=True)
        a = p * (np.abs(dp) + np.abs(dr))
        fl = np.maximum(fl, [sc * (a @ np.abs(k[h])).max(), sc * (a.T @ np.abs(q[h])).max(),
                             (p.T @ np.abs(do[h])).max()])
    return fl


def _check(got, ref, dtype, label, floors=(0.0, 0.0, 0.0)):
    errs = {}
    for name, g, w, fl in zip(("dq", "dk", "dv"), got, ref, floors):
        assert np.isfinite(g).all(), f"{label}: {name} not finite"
        scale = max(float(np.abs(w).max()), fl, 1e-30)
        bound = TOL[dtype] * scale + oracle.ulp(w, MANT[dtype]) / 2
        err = np.abs(g - w)
        worst = float((err / bound).max())
        errs[name] = (float(err.max()) / scale, worst)
        assert worst <= 1.0, f"{label}: {name} beyond bound (max rel err {err.max() / scale:.3g}, worst {worst:.3f})"
    return errs


SHAPES = [
    (1, 1, 1, "S=1"),
    (1, 2, 33, "ragged"),
    (2, 1, 64, "one tile"),
    (1, 2, 100, "ragged multi"),
    (1, 1, 256, "one workgroup"),
    (2, 2, 300, "two workgroups, ragged"),
]


@pytest.mark.parametrize("dtype", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_bwd_small_shapes_vs_oracle(device, dtype, D, causal):
    for i, (B, H, S, label) in enumerate(SHAPES):
        tag = f"bwd {dtype} D={D} causal={causal} B{B} H{H} S{S} ({label})"
        _say(f"case {tag}")
        got, ref, fl = _run(B, H, S, D, dtype, causal, seed=300 + i)
        errs = _check(got, ref, dtype, tag, fl)
        _say(f"  {errs}")


@pytest.mark.parametrize("dtype", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("D", [64, 128])
def test_bwd_with_forward_output(device, dtype, D):
    """Row terms from <dout, O> instead of the extra pass over the keys
    (head_dim 128: the pipelined dQ loop with DMA staging runs its second
    pass only).  Not at S = 1: with one visible key per row the true dq is 0;
    the oracle, following the reference's formula over the stored bf16 m and
    l, gets P = 1 + O(2^-9) and so dq = P dP (1 - P) k / sqrt(D), small but
    not 0, while <dout, O> cancels dP to fp32 rounding: a 100% difference of
    a tiny scale, which a bound relative to the oracle's own maximum fails."""
    for causal in (True, False):
        for S in ((300,) if D == 64 else (63, 300)):
            tag = f"bwd with O {dtype} D={D} S={S} causal={causal}"
            _say(f"case {tag}")
            got, ref, fl = _run(2, 2, S, D, dtype, causal, seed=400 + S, with_o=True)
            _check(got, ref, dtype, tag, fl)


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("causal", [True, False])
def test_bwd_float_ml_from_64_row_kernel(device, dtype, causal):
    """m and l in float32 from the 64-row forward kernel (head_dim 128,
    S > 384) feed the backward, which reads them as float32."""
    tag = f"bwd {dtype} float m/l D=128 causal={causal} B1 H2 S520"
    _say(f"case {tag}")
    got, ref, fl = _run(1, 2, 520, 128, dtype, causal, seed=450, ml_dtype=__import__("torch").float32)
    _check(got, ref, dtype, tag, fl)


def test_bwd_larger_heads_sampled(device):
    """S = 1024, head_dim 128, bf16: two heads against the oracle."""
    tag = "bwd bf16 B1 H4 S1024 D128"
    _say(f"case {tag}")
    got, ref, fl = _run(1, 4, 1024, 128, "bf16", True, seed=500, heads=[0, 3])
    _check(got, ref, "bf16", tag, fl)


def test_bwd_closed_form_constant_v(device):
    """Constant V: O does not depend on q, k, so dq = dk = 0.  With m, l in
    float32 the probabilities of a row sum to 1 within float32 rounding, so
    dS = P (dP - sum P dP) vanishes up to that (with m, l rounded to bf16 the
    row sums are off by up to 2^-9 and dq, dk are small but not zero, in the
    reference's algorithm as well)."""
    import torch

    import pmkl_amd
    from pmkl_amd.workloads import small_inputs

    q, k, _ = small_inputs(1, 2, 200, 64, "bf16", seed=9)
    v = torch.full_like(q, 0.5)
    do = torch.ones_like(q)
    qd, kd, vd, dod = (x.to("cuda:0") for x in (q, k, v, do))
    o, m, l = pmkl_amd.attn_fwd(qd, kd, vd, is_causal=True, ml_dtype=torch.float32)
    dq, dk, dv = pmkl_amd.attn_bwd(dod, qd, kd, vd, m, l, is_causal=True)
    torch.cuda.synchronize()
    assert float(dq.abs().max()) <= 1e-2 and float(dk.abs().max()) <= 1e-2
    # dv_j = sum_{i >= j} P_ij: the column sums of P; the total over j is S per head
    tot = dv.float().sum(dim=2)[..., 0]
    assert torch.allclose(tot.cpu(), torch.full_like(tot.cpu(), 200.0), rtol=2e-2)


def test_bwd_error_paths(device):
    import torch

    import pmkl_amd

    q = torch.zeros((1, 1, 64, 64), dtype=torch.float64, device="cuda:0")
    m = torch.zeros((1, 1, 64), dtype=torch.float64, device="cuda:0")
    with pytest.raises(Exception, match="dtype"):
        pmkl_amd.attn_bwd(q, q, q, q, m, m)


@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
def test_bwd_torch_operator_and_autograd_device(device, dtype):
    """fused_self_attention_bw on ROCm tensors runs the device backward (same
    result as the C ABI call); the autograd entry's device branch, which hands
    the saved forward output to the kernel, is within the bound of the oracle."""
    import torch

    import pmkl_amd
    from pmkl_amd import pmkl_pytorch_ext
    from pmkl_amd.pmkl_function import fused_self_attention
    from pmkl_amd.workloads import small_inputs, torch_dtype

    B, H, S, D = 1, 2, 300, 64
    q, k, v = small_inputs(B, H, S, D, dtype, seed=600)
    do = torch.randn(B, H, S, D, generator=torch.Generator().manual_seed(601)).to(torch_dtype(dtype))
    qd, kd, vd, dod = (x.to("cuda:0") for x in (q, k, v, do))
    o, m, l = pmkl_pytorch_ext.fused_self_attention_fw(qd, kd, vd, True)
    a = pmkl_pytorch_ext.fused_self_attention_bw(dod, qd, kd, vd, m, l, True)
    b = pmkl_amd.attn_bwd(dod, qd, kd, vd, m, l, is_causal=True)
    torch.cuda.synchronize()
    assert all(torch.equal(x, y) for x, y in zip(a, b))

    qg, kg, vg = (x.clone().requires_grad_(True) for x in (qd, kd, vd))
    out, mm, ll = fused_self_attention(qg, kg, vg, True)
    out.backward(dod)
    torch.cuda.synchronize()
    r = lambda t: _np(t).reshape(B * H, S, D)
    mn, ln = _np(mm).reshape(B * H, S), _np(ll).reshape(B * H, S)
    ref = oracle.attn_bwd(r(q), r(k), r(v), r(do), mn, ln, causal=True)
    fl = _term_floors(r(q), r(k), r(v), r(do), mn, ln, True) if dtype == "fp32" else (0.0, 0.0, 0.0)
    _check([r(qg.grad), r(kg.grad), r(vg.grad)], ref, dtype, f"autograd device {dtype}", fl)


@pytest.mark.parametrize("dtype", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("D", [32, 64, 128])
def test_bwd_strided_views_without_copies(device, dtype, D):
    """Strided inputs and outputs of the backward, as the forward takes them:
    q and k are views into one packed [B, S, 3, H, D] buffer, v, dout and o
    are BSHD views (so K and V have different row strides), and dq, dk, dv are
    written into BSHD buffers through the C ABI.  The kernels do the same
    arithmetic whatever the strides, so every gradient equals the contiguous
    call's bit for bit; the contiguous call is held to the oracle.  The torch
    operator and the autograd entry take the same views (no copies on their
    way to the kernels) and give the same bits."""
    import torch

    import pmkl_amd
    from pmkl_amd import capi, pmkl_pytorch_ext
    from pmkl_amd.pmkl_function import fused_self_attention
    from pmkl_amd.workloads import small_inputs, torch_dtype

    B, H, S, causal = 2, 3, 190, True
    tag = f"bwd strided {dtype} D={D} B{B} H{H} S{S}"
    _say(f"case {tag}")
    q, k, v = small_inputs(B, H, S, D, dtype, seed=700 + D)
    rng = np.random.Generator(np.random.PCG64(701 + D))
    do = torch.from_numpy(rng.standard_normal((B, H, S, D)).astype(np.float32)).to(torch_dtype(dtype))
    dev = torch.device("cuda:0")
    tdt = torch_dtype(dtype)
    qkv = torch.zeros((B, S, 3, H, D), dtype=tdt, device=dev)
    qkv[:, :, 0] = q.transpose(1, 2).to(dev)
    qkv[:, :, 1] = k.transpose(1, 2).to(dev)
    qs, ks = qkv[:, :, 0].transpose(1, 2), qkv[:, :, 1].transpose(1, 2)
    bshd = lambda t: t.transpose(1, 2).contiguous().to(dev).transpose(1, 2)
    vs, dos = bshd(v), bshd(do)
    assert qs.stride(2) == 3 * H * D and vs.stride(2) == H * D and not qs.is_contiguous()
    obuf = torch.empty((B, S, H, D), dtype=tdt, device=dev)
    os_ = obuf.transpose(1, 2)
    o, m, l = pmkl_amd.attn_fwd(qs, ks, vs, is_causal=causal, out=os_)

    qc, kc, vc, doc, oc = (x.contiguous() for x in (qs, ks, vs, dos, os_))
    want = pmkl_amd.attn_bwd(doc, qc, kc, vc, m, l, is_causal=causal, out=oc)

    # C ABI with strided inputs and outputs
    gb = [torch.full((B, S, H, D), float("nan"), dtype=tdt, device=dev) for _ in range(3)]
    gv = [g.transpose(1, 2) for g in gb]
    ws_bytes = int(capi.load().pmkl_attn_bwd_workspace_size(B, H, S))
    ws = torch.empty((ws_bytes + 3) // 4, dtype=torch.float32, device=dev)
    st = lambda t: tuple(t.stride()[:3])
    a = capi.make_bwd_args(dos.data_ptr(), qs.data_ptr(), ks.data_ptr(), vs.data_ptr(), os_.data_ptr(),
                           m.data_ptr(), l.data_ptr(), gv[0].data_ptr(), gv[1].data_ptr(), gv[2].data_ptr(),
                           ws.data_ptr(), ws.numel() * 4, dtype=pmkl_amd.torch_dtype_to_pmkl(tdt),
                           batch=B, heads=H, seq_len=S, head_dim=D, is_causal=causal,
                           strides={"dout": st(dos), "q": st(qs), "k": st(ks), "v": st(vs), "o": st(os_),
                                    "dq": st(gv[0]), "dk": st(gv[1]), "dv": st(gv[2])})
    assert capi.attn_bwd_raw(a, torch.cuda.current_stream().cuda_stream) == capi.PMKL_OK, capi.last_error()
    # the Python wrapper with strided inputs (contiguous outputs)
    got_py = pmkl_amd.attn_bwd(dos, qs, ks, vs, m, l, is_causal=causal, out=os_)
    # the torch operator (no O: its own row-term pass) against the contiguous call without O
    want_no_o = pmkl_amd.attn_bwd(doc, qc, kc, vc, m, l, is_causal=causal)
    got_op = pmkl_pytorch_ext.fused_self_attention_bw(dos, qs, ks, vs, m, l, causal)
    # autograd through strided leaves
    qb, kb2, vb = (x.transpose(1, 2).detach().clone().requires_grad_(True) for x in (qs, ks, vs))
    out, _, _ = fused_self_attention(qb.transpose(1, 2), kb2.transpose(1, 2), vb.transpose(1, 2), causal)
    out.backward(dos)
    torch.cuda.synchronize()
    for name, w, g1, g2, g3, w0, g4 in zip(("dq", "dk", "dv"), want, gv, got_py, got_op, want_no_o,
                                           (qb.grad, kb2.grad, vb.grad)):
        assert torch.equal(g1, w), f"{tag}: C ABI strided {name} differs from the contiguous call"
        assert torch.equal(g2, w), f"{tag}: attn_bwd strided {name} differs"
        assert torch.equal(g3, w0), f"{tag}: torch op strided {name} differs"
        assert torch.equal(g4.transpose(1, 2), w), f"{tag}: autograd strided {name} differs"
    r = lambda t: _np(t).reshape(B * H, S, D)
    ref = oracle.attn_bwd(r(q), r(k), r(v), r(do), _np(m).reshape(B * H, S), _np(l).reshape(B * H, S),
                          causal=causal)
    fl = _term_floors(r(q), r(k), r(v), r(do), _np(m).reshape(B * H, S), _np(l).reshape(B * H, S), causal) \
        if dtype == "fp32" else (0.0, 0.0, 0.0)
    _say(f"  {_check([r(x) for x in want], ref, dtype, tag, fl)}")
