"""Autograd entry of the fused self-attention forward.

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
Backward: the reference computes it only on the CPU with debug=True through
fused_self_attention_bw (fused_self_attention.cpp:175-215); that operator is
not part of this forward path, so backward raises NotImplementedError.
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
        ctx.save_for_backward(q, k, v, out_m, out_l)
        ctx.is_casual = bool(is_casual)
        ctx.debug = bool(debug)

    @staticmethod
    def backward(ctx, grad_output, grad_m, grad_l):
        raise NotImplementedError("fused_self_attention backward is not implemented by pmkl_amd")


fused_self_attention = fused_self_attention_.apply
