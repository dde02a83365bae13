"""CPU tests of the torch operator and the autograd entry (no GPU).

pmkl_amd.pmkl_pytorch_ext.fused_self_attention_fw keeps the reference's CPU
body for CPU tensors (pmkl_pytorch_ext/fused_self_attention.cpp:5-64,139-173):
its results must equal the reference operator's bit for bit, in every dtype the
reference dispatches (float, double, half, bfloat16).  This is checked against
the committed fixtures (outputs of the reference operator built from its
source) and, where oracle/_ref is built, live on fresh inputs.  The
pmkl_function wrapper keeps the reference's API and CPU/debug behaviour
(pmkl_function/__init__.py:12-33).  fused_self_attention_bw's CPU body is held
to the reference's backward operator (fused_self_attention.cpp:66-135) the
same way, through tests/golden/bwd_*.npz.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle
from pmkl_amd import pmkl_pytorch_ext
from pmkl_amd.pmkl_function import fused_self_attention

GOLDEN = Path(__file__).resolve().parent / "golden"
FIXTURES = sorted(GOLDEN.glob("ref_*.npz"))
TORCH = {"fp64": torch.float64, "fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}


def _stored(arr, dt):
    t = torch.from_numpy(np.ascontiguousarray(arr))
    return t.view(torch.bfloat16) if dt == "bf16" else t


@pytest.mark.parametrize("dt", list(TORCH))
@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: p.stem)
def test_cpu_branch_bit_exact_vs_reference_fixture(path, dt):
    with np.load(path, allow_pickle=False) as z:
        f = {k: z[k] for k in z.files}
    B, H, S, D, causal = int(f["B"]), int(f["H"]), int(f["S"]), int(f["D"]), bool(f["causal"])
    q, k, v = (torch.from_numpy(f[x]).reshape(B, H, S, D).to(TORCH[dt]) for x in "qkv")
    o, m, l = pmkl_pytorch_ext.fused_self_attention_fw(q, k, v, causal)
    assert o.shape == (B, H, S, D) and m.shape == (B, H, S) and l.shape == (B, H, S)
    assert o.dtype == m.dtype == l.dtype == TORCH[dt]
    assert torch.equal(o, _stored(f[f"o_{dt}"], dt).reshape(B, H, S, D))
    assert torch.equal(m, _stored(f[f"m_{dt}"], dt).reshape(B, H, S))
    assert torch.equal(l, _stored(f[f"l_{dt}"], dt).reshape(B, H, S))


def test_cpu_branch_bit_exact_vs_reference_build_live():
    ref = oracle.reference_op()
    if ref is None:
        pytest.skip("oracle/_ref not built (the reference tree is absent)")
    g = torch.Generator().manual_seed(3)
    for dt in TORCH.values():
        for (B, H, S, D, causal) in [(2, 3, 45, 64, True), (1, 2, 70, 32, False), (1, 1, 33, 128, True)]:
            q, k, v = (torch.randn(B, H, S, D, generator=g).to(dt) for _ in range(3))
            a = pmkl_pytorch_ext.fused_self_attention_fw(q, k, v, causal)
            b = ref.fused_self_attention_fw(q, k, v, causal)
            assert all(torch.equal(x, y) for x, y in zip(a, b)), (dt, B, H, S, D, causal)


def test_noncontiguous_inputs_and_contiguous_output():
    """Strided inputs give the contiguous-input result; the output is contiguous
    (the reference's empty_like(v) would keep a strided v's layout)."""
    g = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn(2, 40, 3, 64, generator=g) for _ in range(3))
    qs, ks, vs = (x.transpose(1, 2) for x in (q, k, v))
    a = pmkl_pytorch_ext.fused_self_attention_fw(qs, ks, vs, True)
    b = pmkl_pytorch_ext.fused_self_attention_fw(qs.contiguous(), ks.contiguous(), vs.contiguous(), True)
    assert all(torch.equal(x, y) for x, y in zip(a, b))
    assert a[0].is_contiguous()


def test_shape_checks_match_reference_messages():
    x = torch.randn(2, 3, 8, 64)
    with pytest.raises(RuntimeError, match="Input tensor shapes must match"):
        pmkl_pytorch_ext.fused_self_attention_fw(x[0], x[0], x[0], True)
    with pytest.raises(RuntimeError, match="Input tensor shapes must match"):
        pmkl_pytorch_ext.fused_self_attention_fw(x, x[:, :, :4], x, True)
    with pytest.raises(RuntimeError, match="dtypes must match"):
        pmkl_pytorch_ext.fused_self_attention_fw(x, x.double(), x, True)


def test_empty_sequence():
    x = torch.randn(2, 3, 0, 64)
    o, m, l = pmkl_pytorch_ext.fused_self_attention_fw(x, x, x, True)
    assert o.shape == (2, 3, 0, 64) and m.shape == (2, 3, 0)


def test_pmkl_function_cpu_debug_and_errors():
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(1, 2, 16, 32, generator=g) for _ in range(3))
    out = fused_self_attention(q, k, v, True, True)
    ref = pmkl_pytorch_ext.fused_self_attention_fw(q, k, v, True)
    assert all(torch.equal(a, b) for a, b in zip(out, ref))
    with pytest.raises(NotImplementedError):
        fused_self_attention(q, k, v, True)          # CPU without debug, as in the reference
    # backward on the CPU with debug: the operator's CPU body, as in the reference
    qg, kg, vg = (x.clone().requires_grad_(True) for x in (q, k, v))
    o, m, l = fused_self_attention(qg, kg, vg, True, True)
    gout = torch.randn(o.shape, generator=g)
    o.backward(gout)
    want = pmkl_pytorch_ext.fused_self_attention_bw(gout, q, k, v, m.detach(), l.detach(), True)
    for got, w in zip((qg.grad, kg.grad, vg.grad), want):
        assert torch.equal(got, w)


BWD_FIXTURES = sorted(GOLDEN.glob("bwd_*.npz"))


@pytest.mark.parametrize("dt", list(TORCH))
@pytest.mark.parametrize("path", BWD_FIXTURES, ids=lambda p: p.stem)
def test_cpu_backward_bit_exact_vs_reference_fixture(path, dt):
    """fused_self_attention_bw's CPU body == the reference operator's, bit for bit
    (fused_self_attention.cpp:66-135,175-215), on the m, l its forward returned."""
    with np.load(path, allow_pickle=False) as z:
        f = {k: z[k] for k in z.files}
    B, H, S, D, causal = int(f["B"]), int(f["H"]), int(f["S"]), int(f["D"]), bool(f["causal"])
    q, k, v, do = (torch.from_numpy(f[x]).reshape(B, H, S, D).to(TORCH[dt]) for x in ("q", "k", "v", "dout"))
    m = _stored(f[f"m_{dt}"], dt).reshape(B, H, S)
    l = _stored(f[f"l_{dt}"], dt).reshape(B, H, S)
    dq, dk, dv = pmkl_pytorch_ext.fused_self_attention_bw(do, q, k, v, m, l, causal)
    for name, got in (("dq", dq), ("dk", dk), ("dv", dv)):
        assert got.dtype == TORCH[dt]
        assert torch.equal(got, _stored(f[f"{name}_{dt}"], dt).reshape(B, H, S, D)), (name, dt)


def test_cpu_backward_bit_exact_vs_reference_build_live():
    ref = oracle.reference_op()
    if ref is None:
        pytest.skip("oracle/_ref not built (the reference tree is absent)")
    g = torch.Generator().manual_seed(6)
    for dt in TORCH.values():
        for (B, H, S, D, causal) in [(1, 2, 19, 32, True), (1, 1, 24, 64, False)]:
            q, k, v, do = (torch.randn(B, H, S, D, generator=g).to(dt) for _ in range(4))
            _, m, l = ref.fused_self_attention_fw(q, k, v, causal)
            a = pmkl_pytorch_ext.fused_self_attention_bw(do, q, k, v, m, l, causal)
            b = ref.fused_self_attention_bw(do, q, k, v, m, l, causal)
            assert all(torch.equal(x, y) for x, y in zip(a, b)), (dt, B, H, S, D, causal)


def test_backward_checks_match_reference_messages():
    x = torch.randn(1, 2, 8, 32)
    m = torch.randn(1, 2, 8)
    with pytest.raises(RuntimeError, match="Input tensor must be contiguous"):
        pmkl_pytorch_ext.fused_self_attention_bw(x, x.transpose(2, 3), x, x, m, m, True)
    with pytest.raises(RuntimeError, match="Input tensor shapes must match"):
        pmkl_pytorch_ext.fused_self_attention_bw(x, x, x[:, :1].contiguous(), x, m, m, True)


def test_backward_rejects_tensors_on_another_device():
    """Every tensor must sit on q's device: checked before any dispatch, so a
    host pointer never reaches a kernel (and no device pointer the CPU body).
    The meta device stands in for "another device" here (no GPU needed)."""
    x = torch.randn(1, 2, 8, 32)
    m = torch.randn(1, 2, 8)
    xm = torch.empty_like(x, device="meta")
    mm = torch.empty_like(m, device="meta")
    for args in ((xm, x, x, x, m, m), (x, x, xm, x, m, m), (x, x, x, xm, m, m),
                 (x, x, x, x, mm, m), (x, x, x, x, m, mm)):
        with pytest.raises(RuntimeError, match="on one device"):
            pmkl_pytorch_ext.fused_self_attention_bw(*args, True)
