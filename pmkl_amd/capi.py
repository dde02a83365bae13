"""ctypes view of the C ABI in include/pmkl_attn.h and include/pmkl_softmax.h
(libpmkl_attn.so).

This is the thin Python handle on the drop-in boundary: it passes device
pointers, sizes and a HIP stream, nothing else.  Loading fails loudly when the
library has not been built; there is no fallback path.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

_LIB_PATH = Path(__file__).resolve().parent / "libpmkl_attn.so"

PMKL_DTYPE_F32 = 0
PMKL_DTYPE_F16 = 1
PMKL_DTYPE_BF16 = 2

PMKL_OK = 0
PMKL_EINVAL = 1
PMKL_EUNSUPPORTED = 2
PMKL_EHIP = 3

PMKL_SOFTMAX_MAX_ELEMENTS = 1024
PMKL_ATTN_BWD_NOALLOC_MAX_ROWS = 1048576   # include/pmkl_attn.h

# Every symbol include/pmkl_attn.h and include/pmkl_softmax.h declare.
EXPORTED_SYMBOLS = (
    "pmkl_attn_fwd",
    "pmkl_attn_fwd_kernel_name",
    "pmkl_causal_attention_forward",
    "pmkl_attn_fwd_supported",
    "pmkl_attn_bwd_workspace_size",
    "pmkl_attn_bwd",
    "pmkl_attn_bwd_supported",
    "pmkl_attn_bwd_noalloc",
    "pmkl_last_error",
    "pmkl_abi_version",
    "pmkl_softmax_fwd",
    "pmkl_warp_softmax_forward",
)


class AttnFwdArgs(ctypes.Structure):
    """Mirror of pmkl_attn_fwd_args."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("m", ctypes.c_void_p),
        ("l", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("ml_dtype", ctypes.c_int32),
        ("batch", ctypes.c_int64),
        ("heads", ctypes.c_int64),
        ("seq_len", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("q_strides", ctypes.c_int64 * 3),
        ("k_strides", ctypes.c_int64 * 3),
        ("v_strides", ctypes.c_int64 * 3),
        ("o_strides", ctypes.c_int64 * 3),
        ("scale", ctypes.c_float),
        ("is_causal", ctypes.c_int32),
    ]


class AttnBwdArgs(ctypes.Structure):
    """Mirror of pmkl_attn_bwd_args."""

    _fields_ = [
        ("dout", ctypes.c_void_p),
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("m", ctypes.c_void_p),
        ("l", ctypes.c_void_p),
        ("dq", ctypes.c_void_p),
        ("dk", ctypes.c_void_p),
        ("dv", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_uint64),
        ("dtype", ctypes.c_int32),
        ("ml_dtype", ctypes.c_int32),
        ("batch", ctypes.c_int64),
        ("heads", ctypes.c_int64),
        ("seq_len", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("scale", ctypes.c_float),
        ("is_causal", ctypes.c_int32),
        ("dout_strides", ctypes.c_int64 * 3),
        ("q_strides", ctypes.c_int64 * 3),
        ("k_strides", ctypes.c_int64 * 3),
        ("v_strides", ctypes.c_int64 * 3),
        ("o_strides", ctypes.c_int64 * 3),
        ("dq_strides", ctypes.c_int64 * 3),
        ("dk_strides", ctypes.c_int64 * 3),
        ("dv_strides", ctypes.c_int64 * 3),
    ]


BWD_STRIDE_FIELDS = ("dout", "q", "k", "v", "o", "dq", "dk", "dv")


class SoftmaxArgs(ctypes.Structure):
    """Mirror of pmkl_softmax_args."""

    _fields_ = [
        ("dst", ctypes.c_void_p),
        ("src", ctypes.c_void_p),
        ("out_dtype", ctypes.c_int32),
        ("in_dtype", ctypes.c_int32),
        ("elements", ctypes.c_int64),
        ("stride", ctypes.c_int64),
        ("batch", ctypes.c_int64),
        ("is_log", ctypes.c_int32),
    ]


class PmklError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"pmkl error {code}: {msg}")
        self.code = code


_lib = None


def load() -> ctypes.CDLL:
    """Load libpmkl_attn.so (raises if it is missing)."""
    global _lib
    if _lib is not None:
        return _lib
    if not _LIB_PATH.exists():
        raise ImportError(f"{_LIB_PATH} is not built; run __graft_entry__.build() or python -m pmkl_amd._build")
    lib = ctypes.CDLL(str(_LIB_PATH))
    lib.pmkl_attn_fwd.argtypes = [ctypes.POINTER(AttnFwdArgs), ctypes.c_void_p]
    lib.pmkl_attn_fwd.restype = ctypes.c_int
    lib.pmkl_causal_attention_forward.argtypes = [
        ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
        ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
    ]
    lib.pmkl_causal_attention_forward.restype = ctypes.c_int
    lib.pmkl_attn_fwd_kernel_name.argtypes = [ctypes.POINTER(AttnFwdArgs)]
    lib.pmkl_attn_fwd_kernel_name.restype = ctypes.c_char_p
    lib.pmkl_attn_fwd_supported.argtypes = [ctypes.c_int32, ctypes.c_int64]
    lib.pmkl_attn_fwd_supported.restype = ctypes.c_int
    lib.pmkl_last_error.argtypes = []
    lib.pmkl_last_error.restype = ctypes.c_char_p
    lib.pmkl_abi_version.argtypes = []
    lib.pmkl_abi_version.restype = ctypes.c_int
    lib.pmkl_attn_bwd_workspace_size.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64]
    lib.pmkl_attn_bwd_workspace_size.restype = ctypes.c_uint64
    lib.pmkl_attn_bwd.argtypes = [ctypes.POINTER(AttnBwdArgs), ctypes.c_void_p]
    lib.pmkl_attn_bwd.restype = ctypes.c_int
    lib.pmkl_attn_bwd_noalloc.argtypes = [ctypes.POINTER(AttnBwdArgs), ctypes.c_void_p]
    lib.pmkl_attn_bwd_noalloc.restype = ctypes.c_int
    lib.pmkl_attn_bwd_supported.argtypes = [ctypes.c_int32, ctypes.c_int64]
    lib.pmkl_attn_bwd_supported.restype = ctypes.c_int
    lib.pmkl_softmax_fwd.argtypes = [ctypes.POINTER(SoftmaxArgs), ctypes.c_void_p]
    lib.pmkl_softmax_fwd.restype = ctypes.c_int
    lib.pmkl_warp_softmax_forward.argtypes = [
        ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p,
        ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
    ]
    lib.pmkl_warp_softmax_forward.restype = ctypes.c_int
    _lib = lib
    return lib


def library_path() -> Path:
    return _LIB_PATH


def last_error() -> str:
    return load().pmkl_last_error().decode()


def attn_fwd_raw(args: AttnFwdArgs, stream: int | None = None) -> int:
    """Call pmkl_attn_fwd; returns the status code."""
    return load().pmkl_attn_fwd(ctypes.byref(args), ctypes.c_void_p(stream or 0))


def attn_fwd_kernel_name(args: AttnFwdArgs) -> str | None:
    """The kernel (and launch shape) pmkl_attn_fwd would launch for args, as
    the library's dispatcher chooses it; None where the call would fail
    (last_error() says why)."""
    name = load().pmkl_attn_fwd_kernel_name(ctypes.byref(args))
    return None if name is None else name.decode()


def make_args(q, k, v, o, m, l, *, dtype: int, ml_dtype: int | None = None, batch: int, heads: int,
              seq_len: int, head_dim: int, is_causal: bool = True, scale: float = 0.0,
              q_strides=(0, 0, 0), k_strides=(0, 0, 0), v_strides=(0, 0, 0), o_strides=(0, 0, 0)) -> AttnFwdArgs:
    """Build an AttnFwdArgs from raw integer pointers."""
    a = AttnFwdArgs()
    a.q, a.k, a.v, a.o, a.m, a.l = q, k, v, o, m, l
    a.dtype = dtype
    a.ml_dtype = dtype if ml_dtype is None else ml_dtype
    a.batch, a.heads, a.seq_len, a.head_dim = batch, heads, seq_len, head_dim
    a.q_strides[:] = list(q_strides)
    a.k_strides[:] = list(k_strides)
    a.v_strides[:] = list(v_strides)
    a.o_strides[:] = list(o_strides)
    a.scale = scale
    a.is_causal = 1 if is_causal else 0
    return a


def attn_bwd_raw(args: AttnBwdArgs, stream: int | None = None) -> int:
    """Call pmkl_attn_bwd; returns the status code."""
    return load().pmkl_attn_bwd(ctypes.byref(args), ctypes.c_void_p(stream or 0))


def attn_bwd_noalloc_raw(args: AttnBwdArgs, stream: int | None = None) -> int:
    """Call pmkl_attn_bwd_noalloc (the workspace fields of args are ignored);
    returns the status code."""
    return load().pmkl_attn_bwd_noalloc(ctypes.byref(args), ctypes.c_void_p(stream or 0))


def make_bwd_args(dout, q, k, v, o, m, l, dq, dk, dv, workspace, workspace_bytes, *, dtype: int,
                  ml_dtype: int | None = None, batch: int, heads: int, seq_len: int, head_dim: int,
                  is_causal: bool = True, scale: float = 0.0, strides: dict | None = None) -> AttnBwdArgs:
    """Build an AttnBwdArgs from raw integer pointers (o may be 0).  strides:
    {name: (batch, head, seq)} element strides for any of dout, q, k, v, o, dq,
    dk, dv; absent ones are contiguous."""
    a = AttnBwdArgs()
    for name, st in (strides or {}).items():
        if name not in BWD_STRIDE_FIELDS:
            raise ValueError(f"no stride field for {name!r}")
        getattr(a, f"{name}_strides")[:] = [int(x) for x in st]
    a.dout, a.q, a.k, a.v, a.o, a.m, a.l = dout, q, k, v, o, m, l
    a.dq, a.dk, a.dv = dq, dk, dv
    a.workspace, a.workspace_bytes = workspace, workspace_bytes
    a.dtype = dtype
    a.ml_dtype = dtype if ml_dtype is None else ml_dtype
    a.batch, a.heads, a.seq_len, a.head_dim = batch, heads, seq_len, head_dim
    a.scale = scale
    a.is_causal = 1 if is_causal else 0
    return a


def softmax_raw(args: SoftmaxArgs, stream: int | None = None) -> int:
    """Call pmkl_softmax_fwd; returns the status code."""
    return load().pmkl_softmax_fwd(ctypes.byref(args), ctypes.c_void_p(stream or 0))


def make_softmax_args(dst, src, *, out_dtype: int, in_dtype: int, elements: int, stride: int, batch: int,
                      is_log: bool = False) -> SoftmaxArgs:
    """Build a SoftmaxArgs from raw integer pointers."""
    a = SoftmaxArgs()
    a.dst, a.src = dst, src
    a.out_dtype, a.in_dtype = out_dtype, in_dtype
    a.elements, a.stride, a.batch = elements, stride, batch
    a.is_log = 1 if is_log else 0
    return a
