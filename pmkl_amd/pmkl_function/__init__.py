"""Autograd entry of the fused self-attention.

Same API as the reference pmkl_pytorch_ext/pmkl_function/__init__.py:1-33:
``fused_self_attention(q, k, v, is_casual, debug=False)`` returning
``(out, out_m, out_l)`` (the parameter really is spelled ``is_casual``).

Dispatch:
  * ROCm device tensors -> the gfx950 kernels (new: the reference raises
    NotImplementedError for anything that is not a CPU tensor with debug=True,
    __init__.py:15-18);
  * CPU tensors with debug=True -> the operator's CPU body, as in the
    reference;
  * anything else -> NotImplementedError, as in the reference.
Backward (gradients of out only; those of out_m, out_l are ignored, as in the
reference, __init__.py:25-32): CPU with debug=True -> fused_self_attention_bw's
CPU body, as the reference; ROCm float32 / float16 / bfloat16 tensors ->
pmkl_attn_bwd (the gfx950 backward: vector-ALU kernels for float32, MFMA for
the 16-bit types), given the saved forward output so its row terms come from
<dout, out>; anything else -> NotImplementedError.
"""
import torch
from torch.autograd import Function

from .. import pmkl_pytorch_ext

__all__ = [
    'fused_self_attention',
]


class fused_self_attention_(Function):
    @staticmethod
    def forward(q, k, v, is_casual, debug=False):
        if q.is_cuda:
            return pmkl_pytorch_ext.fused_self_attention_fw(q, k, v, is_casual)
        if q.is_cpu and debug:
            return pmkl_pytorch_ext.fused_self_attention_fw(q, k, v, is_casual)
        raise NotImplementedError()

    @staticmethod
    def setup_context(ctx, inputs, output):
        q, k, v, is_casual, debug = inputs
        out, out_m, out_l = output
        ctx.save_for_backward(q, k, v, out, out_m, out_l)
        ctx.is_casual = bool(is_casual)
        ctx.debug = bool(debug)

    @staticmethod
    def backward(ctx, grad_output, grad_m, grad_l):
        q, k, v, out, out_m, out_l = ctx.saved_tensors
        if q.is_cuda:
            if q.dtype not in (torch.float32, torch.float16, torch.bfloat16):
                raise NotImplementedError(f"the device backward supports float32, float16 and bfloat16, got {q.dtype}")
            from .. import attn_bwd, kernel_view

            # Strided inputs (BSHD views, a packed QKV) go to the kernels as
            # they are; only what they cannot address (an expanded gradient,
            # say) is made contiguous.
            dq, dk, dv = attn_bwd(kernel_view(grad_output), kernel_view(q), kernel_view(k), kernel_view(v),
                                  out_m, out_l, is_causal=ctx.is_casual, out=kernel_view(out))
        elif q.is_cpu and ctx.debug:
            dq, dk, dv = pmkl_pytorch_ext.fused_self_attention_bw(grad_output, q, k, v, out_m, out_l, ctx.is_casual)
        else:
            raise NotImplementedError()
        return dq, dk, dv, None, None


fused_self_attention = fused_self_attention_.apply
