"""CPU tests of the torch operator and the autograd entry (no GPU).

pmkl_amd.pmkl_pytorch_ext.fused_self_attention_fw keeps the reference's CPU
body for CPU tensors (pmkl_pytorch_ext/fused_self_attention.cpp:5-64,139-173):
its results must equal the reference operator's bit for bit, in every dtype the
reference dispatches (float, double, half, bfloat16).  This is checked against
the committed fixtures (outputs of the reference operator built from its
source) and, where oracle/_ref is built, live on fresh inputs.  The
pmkl_function wrapper keeps the reference's API and CPU/debug behaviour
(pmkl_function/__init__.py:12-33).
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
    qg = q.clone().requires_grad_(True)
    o, _, _ = fused_self_attention(qg, k, v, True, True)
    with pytest.raises(NotImplementedError):
        o.sum().backward()
