"""Top-level import name of the torch operators.

The reference installs its extension as the top-level module
``pmkl_pytorch_ext`` (pmkl_pytorch_ext/setup.py:5-12) and its callers import it
by that name (pmkl_pytorch_ext/pmkl_function/__init__.py:4).  With this
repository's root on ``sys.path`` the same ``import pmkl_pytorch_ext`` resolves
here, to the operators built into ``pmkl_amd/pmkl_pytorch_ext*.so`` (ROCm
device tensors go to the gfx950 kernels, CPU tensors to the reference's CPU
algorithm).  Importing fails loudly when that extension has not been built.
"""
from pmkl_amd.pmkl_pytorch_ext import fused_self_attention_bw, fused_self_attention_fw

__all__ = ["fused_self_attention_fw", "fused_self_attention_bw"]
