"""The reference's callers import the operators by top-level names:
``import pmkl_pytorch_ext`` (pmkl_pytorch_ext/pmkl_function/__init__.py:4) and
``from pmkl_function import fused_self_attention``
(pmkl_pytorch_ext/test/test_fused_self_attention.py:3).  Both resolve with the
repository root on sys.path, to this build's operators, and run the
reference harness's calls unchanged (CPU tensors with debug=True here; the
device branch is covered by the GPU tests)."""
from __future__ import annotations

import torch


def test_top_level_names_resolve_to_this_build():
    import pmkl_pytorch_ext
    from pmkl_function import fused_self_attention

    import pmkl_amd.pmkl_function
    from pmkl_amd import pmkl_pytorch_ext as ext

    assert pmkl_pytorch_ext.fused_self_attention_fw is ext.fused_self_attention_fw
    assert pmkl_pytorch_ext.fused_self_attention_bw is ext.fused_self_attention_bw
    assert fused_self_attention is pmkl_amd.pmkl_function.fused_self_attention


def test_reference_harness_calls_run_unchanged():
    """The calls of test_fused_self_attention.py:16-36, at a reduced size
    (B 1, H 2; the CPU backward is O(S^3 D)): forward with debug=True,
    out.sum().backward(), compared with SDPA and its autograd in float64.
    The reference's scale is the float 1.0f/sqrtf(D) (fused_self_attention.cpp:
    30), which differs from SDPA's double 1/sqrt(D) by up to 2^-24 relative,
    hence the 1e-6 bounds."""
    import torch.nn.functional as F
    from pmkl_function import fused_self_attention

    g = torch.Generator().manual_seed(31)
    for D in (64, 128):
        for is_causal in (False, True):
            q_ref, k_ref, v_ref = (torch.randn(1, 2, 32, D, generator=g, dtype=torch.float64).requires_grad_(True)
                                   for _ in range(3))
            out_ref = F.scaled_dot_product_attention(q_ref, k_ref, v_ref, attn_mask=None, dropout_p=0.0,
                                                     is_causal=is_causal)
            out_ref.sum().backward()
            q, k, v = (x.detach().clone().requires_grad_(True) for x in (q_ref, k_ref, v_ref))
            out, _, _ = fused_self_attention(q, k, v, is_causal, True)
            out.sum().backward()
            assert (out - out_ref).abs().max().item() < 1e-6
            for a, b in ((q.grad, q_ref.grad), (k.grad, k_ref.grad), (v.grad, v_ref.grad)):
                assert (a - b).abs().max().item() < 1e-6 * max(1.0, b.abs().max().item())
