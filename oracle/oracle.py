"""TEST INFRASTRUCTURE ONLY - Python handle on the parity oracle.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker.  The product (pmkl_amd/,
include/) never imports it.

* ``attn_fwd_rows`` - ctypes call of oracle/liboracle.so, the float64
  restatement of the reference CPU operator
  (pmkl_pytorch_ext/fused_self_attention.cpp:5-64); see attn_oracle.c.
* ``attn_bwd`` - the float64 restatement of the reference's backward
  operator (fused_self_attention.cpp:66-135), gradients of O only.
* ``softmax_f64`` - the float64 restatement of the reference row softmax /
  log-softmax (pmkl/norm/warp_softmax.h:74-201); see softmax_oracle.c.
* ``softmax_host_f32`` - the reference's CPU check of that softmax
  (test/test_softmax.cpp:10-28) op for op in float: the benchmark's CPU
  baseline.
* ``reference_op`` - the reference's own CPU operator compiled from its source
  into oracle/_ref (oracle/Makefile), or None when that build is absent.
* ``attn_sdpa_f64`` - torch.nn.functional.scaled_dot_product_attention in
  float64 on the CPU, the reference's own Python oracle
  (pmkl_pytorch_ext/test/test_fused_self_attention.py:6-7); used to pin the
  restatement, not as the oracle itself.
"""
from __future__ import annotations

import ctypes
import importlib.util
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
_LIB = None
_REF = None


def _lib():
    global _LIB
    if _LIB is None:
        path = _DIR / "liboracle.so"
        if not path.exists():
            raise ImportError(f"{path} is not built (make -C oracle)")
        lib = ctypes.CDLL(str(path))
        lib.oracle_default_scale.argtypes = [ctypes.c_int64]
        lib.oracle_default_scale.restype = ctypes.c_double
        dp = ctypes.POINTER(ctypes.c_double)
        fp = ctypes.POINTER(ctypes.c_float)
        lib.oracle_attn_fwd_rows.argtypes = [fp, fp, fp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                             ctypes.c_int, ctypes.c_double, ctypes.POINTER(ctypes.c_int64),
                                             ctypes.c_int64, dp, dp, dp]
        lib.oracle_attn_fwd_rows.restype = ctypes.c_int
        lib.oracle_attn_bwd.argtypes = [fp, fp, fp, fp, dp, dp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                        ctypes.c_int, ctypes.c_double, ctypes.POINTER(ctypes.c_int64),
                                        ctypes.c_int64, dp, dp, dp]
        lib.oracle_attn_bwd.restype = ctypes.c_int
        lib.oracle_softmax_f64.argtypes = [dp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, dp]
        lib.oracle_softmax_f64.restype = ctypes.c_int
        lib.oracle_softmax_host_f32.argtypes = [fp, fp, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.oracle_softmax_host_f32.restype = None
        _LIB = lib
    return _LIB


def default_scale(D: int) -> float:
    """1.0f / sqrtf((float)D) as a double (fused_self_attention.cpp:30)."""
    return _lib().oracle_default_scale(D)


def attn_fwd_rows(q: np.ndarray, k: np.ndarray, v: np.ndarray, causal: bool = True,
                  scale: float | None = None, rows=None):
    """Float64 oracle.  q, k, v: [BH, S, D] (any float dtype; converted to
    float32 exactly for fp16/bf16/fp32 sources).  rows: None for all rows, or
    an int sequence of row indices evaluated in every head.
    Returns (o [BH, R, D], m [BH, R], l [BH, R]) as float64."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    assert q.ndim == 3 and q.shape == k.shape == v.shape
    BH, S, D = q.shape
    if scale is None:
        scale = default_scale(D)
    if rows is None:
        R = S
        rows_p = None
    else:
        rows_arr = np.ascontiguousarray(np.asarray(rows, dtype=np.int64))
        R = rows_arr.size
        rows_p = rows_arr.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))
    o = np.empty((BH, R, D), dtype=np.float64)
    m = np.empty((BH, R), dtype=np.float64)
    l = np.empty((BH, R), dtype=np.float64)
    fp = ctypes.POINTER(ctypes.c_float)
    dp = ctypes.POINTER(ctypes.c_double)
    rc = _lib().oracle_attn_fwd_rows(q.ctypes.data_as(fp), k.ctypes.data_as(fp), v.ctypes.data_as(fp),
                                     BH, S, D, 1 if causal else 0, float(scale), rows_p, R,
                                     o.ctypes.data_as(dp), m.ctypes.data_as(dp), l.ctypes.data_as(dp))
    if rc != 0:
        raise RuntimeError("oracle_attn_fwd_rows failed")
    return o, m, l


def attn_bwd(q: np.ndarray, k: np.ndarray, v: np.ndarray, dout: np.ndarray, m: np.ndarray, l: np.ndarray,
             causal: bool = True, scale: float | None = None, heads=None):
    """Float64 backward oracle (gradients of O; fused_self_attention.cpp:66-135).
    q, k, v, dout: [BH, S, D]; m, l: [BH, S] as the forward returned them.
    heads: None for every head, or the head indices to evaluate.
    Returns (dq, dk, dv), each [nheads, S, D] float64."""
    q, k, v, dout = (np.ascontiguousarray(x, dtype=np.float32) for x in (q, k, v, dout))
    m = np.ascontiguousarray(m, dtype=np.float64)
    l = np.ascontiguousarray(l, dtype=np.float64)
    assert q.ndim == 3 and q.shape == k.shape == v.shape == dout.shape and m.shape == l.shape == q.shape[:2]
    BH, S, D = q.shape
    if scale is None:
        scale = default_scale(D)
    if heads is None:
        NH, heads_p = BH, None
    else:
        heads_arr = np.ascontiguousarray(np.asarray(heads, dtype=np.int64))
        NH = heads_arr.size
        heads_p = heads_arr.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))
    out = [np.empty((NH, S, D), dtype=np.float64) for _ in range(3)]
    fp = ctypes.POINTER(ctypes.c_float)
    dp = ctypes.POINTER(ctypes.c_double)
    rc = _lib().oracle_attn_bwd(q.ctypes.data_as(fp), k.ctypes.data_as(fp), v.ctypes.data_as(fp),
                                dout.ctypes.data_as(fp), m.ctypes.data_as(dp), l.ctypes.data_as(dp),
                                BH, S, D, 1 if causal else 0, float(scale), heads_p, NH,
                                *(x.ctypes.data_as(dp) for x in out))
    if rc != 0:
        raise RuntimeError("oracle_attn_bwd failed")
    return tuple(out)


def softmax_f64(x: np.ndarray, n: int | None = None, is_log: bool = False) -> np.ndarray:
    """Float64 row softmax oracle.  x: [batch, stride] (any float dtype, taken
    exactly as float64); the first n columns of each row (default: all) are
    the row.  Returns [batch, n] float64."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float64))
    if x.ndim == 1:
        x = x[None, :]
    assert x.ndim == 2
    batch, stride = x.shape
    n = stride if n is None else n
    y = np.full((batch, stride), np.nan, dtype=np.float64)
    dp = ctypes.POINTER(ctypes.c_double)
    if _lib().oracle_softmax_f64(x.ctypes.data_as(dp), n, stride, batch, 1 if is_log else 0, y.ctypes.data_as(dp)):
        raise RuntimeError("oracle_softmax_f64 failed")
    return y[:, :n]


def softmax_host_f32(x: np.ndarray, n: int | None = None) -> np.ndarray:
    """The reference's CPU softmax check (test/test_softmax.cpp:10-28) in float.
    x: float32 [batch, stride]; returns [batch, n] float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    batch, stride = x.shape
    n = stride if n is None else n
    y = np.zeros_like(x)
    fp = ctypes.POINTER(ctypes.c_float)
    _lib().oracle_softmax_host_f32(y.ctypes.data_as(fp), x.ctypes.data_as(fp), n, stride, batch)
    return y[:, :n]


def reference_op():
    """The reference operator module built into oracle/_ref, or None."""
    global _REF
    if _REF is not None:
        return _REF
    import sysconfig

    path = _DIR / "_ref" / ("pmkl_pytorch_ext" + sysconfig.get_config_var("EXT_SUFFIX"))
    if not path.exists():
        return None
    import torch  # noqa: F401  (the extension needs libtorch's Python bindings)

    spec = importlib.util.spec_from_file_location("pmkl_pytorch_ext", str(path))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    _REF = mod
    return _REF


def attn_sdpa_f64(q, k, v, causal: bool = True, scale: float | None = None):
    """torch SDPA in float64 on the CPU; returns o as float64 numpy [BH, S, D]."""
    import torch
    import torch.nn.functional as F

    qt = torch.from_numpy(np.asarray(q, dtype=np.float64))
    kt = torch.from_numpy(np.asarray(k, dtype=np.float64))
    vt = torch.from_numpy(np.asarray(v, dtype=np.float64))
    if scale is None:
        scale = default_scale(q.shape[-1])
    o = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=None, dropout_p=0.0, is_causal=causal, scale=scale)
    return o.numpy()


def causal_flops(B: int, H: int, S: int, D: int, causal: bool = True) -> int:
    """Algorithmic FLOPs: 4*D per visible (i, j) pair (QK^T and PV multiply-adds)."""
    pairs = S * (S + 1) // 2 if causal else S * S
    return 4 * D * pairs * B * H


def ulp(x: np.ndarray, mant_bits: int) -> np.ndarray:
    """ulp of |x| in a binary format with `mant_bits` explicit mantissa bits."""
    x = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.where(x > 0, x, 1.0)))
    return np.ldexp(1.0, (e - mant_bits).astype(np.int64))


__all__ = ["attn_fwd_rows", "attn_bwd", "softmax_f64", "softmax_host_f32", "default_scale", "reference_op", "attn_sdpa_f64", "causal_flops", "ulp"]
