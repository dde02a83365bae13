"""Top-level import name of the autograd entry.

The reference ships ``pmkl_function`` as a top-level package
(pmkl_pytorch_ext/setup.py:14, ``packages=['pmkl_function']``) and its harness
imports ``from pmkl_function import fused_self_attention``
(pmkl_pytorch_ext/test/test_fused_self_attention.py:3).  With this repository's
root on ``sys.path`` that import resolves here, to the autograd Function in
``pmkl_amd.pmkl_function`` (same signature, ``is_casual`` spelling kept).
"""
from pmkl_amd.pmkl_function import fused_self_attention, fused_self_attention_

__all__ = ["fused_self_attention"]
