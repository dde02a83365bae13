"""Shared parity checks: device outputs against the float64 oracle.

Tolerances are the path's stated ones (max abs error of O against an fp32+
accumulation reference): fp32 1e-5, fp16 2e-3, bf16 1e-2.  m and l are
stored in the tensor dtype (as fused_self_attention.cpp:149-150 does), so for
16-bit dtypes they are held to 1 ulp of that dtype; for fp32 they are held to
the reference test's all_close(atol=1e-5, rtol=1e-5)
(test/test_causal_attention.cpp:197-201, pmkl/core/utils/measure.h:11-12).

Rounding floor.  Storing O in bf16 / fp16 costs up to half an ulp of the
output dtype on its own: for bf16 that is 0.0078 at |O| in [2, 4) and 0.0156
at [4, 8), so no bf16 output can meet 1e-2 at |O| >= 4.  The element-wise
bound is therefore

    |O - O_ref| <= tol                     where ulp(O_ref) / 2 <  tol
    |O - O_ref| <= ulp(O_ref) / 2 + tol/2  where ulp(O_ref) / 2 >= tol

i.e. the plain tolerance wherever the dtype can represent the answer within
it (bf16 |O| < 4, fp16 |O| < 8: every fp16 output of these workloads, all of
fp32), and only where half an ulp alone exceeds it (bf16 |O| >= 4) at most
tol/2 of the kernel's own error on top of the unavoidable output rounding.
check_outputs also reports the plain max |O - O_ref|, the same over the
elements where the plain tolerance applies, and the floor
max |round(O_ref) - O_ref|, so they can be read side by side.
"""
from __future__ import annotations

import numpy as np

from oracle import oracle

TOL_O = {"fp32": 1e-5, "fp16": 2e-3, "bf16": 1e-2}
MANT_BITS = {"fp32": 23, "fp16": 10, "bf16": 7}


def to_np(t):
    import torch

    return t.detach().to("cpu", torch.float32).numpy().astype(np.float64)


def check_outputs(q, k, v, o, m, l, dtype: str, causal: bool = True, rows=None, scale=None, label="",
                  check_ml: bool = True):
    """q, k, v: CPU torch tensors [B, H, S, D] (in `dtype`); o, m, l: device or
    CPU outputs.  rows: None (all rows) or the row indices to compare.
    check_ml=False reports m and l but asserts only O (for callers that hold
    m and l to a bound of their own).
    Returns a dict of the errors; raises AssertionError beyond tolerance."""
    B, H, S, D = q.shape
    qn, kn, vn = (to_np(x).reshape(B * H, S, D) for x in (q, k, v))
    o_ref, m_ref, l_ref = oracle.attn_fwd_rows(qn, kn, vn, causal=causal, scale=scale, rows=rows)
    on = to_np(o).reshape(B * H, S, D)
    mn = to_np(m).reshape(B * H, S)
    ln = to_np(l).reshape(B * H, S)
    if rows is not None:
        idx = np.asarray(rows, dtype=np.int64)
        on, mn, ln = on[:, idx], mn[:, idx], ln[:, idx]
    assert np.isfinite(on).all() and np.isfinite(mn).all() and np.isfinite(ln).all(), f"{label}: non-finite output"
    tol = TOL_O[dtype]
    diff = np.abs(on - o_ref)
    err_o = float(diff.max()) if on.size else 0.0
    half_ulp = oracle.ulp(o_ref, MANT_BITS[dtype]) / 2
    bound = np.where(half_ulp < tol, tol, half_ulp + tol / 2)
    floor = float(np.max(np.abs(round_to(o_ref, dtype) - o_ref))) if on.size else 0.0
    err_m = np.abs(mn - m_ref)
    err_l = np.abs(ln - l_ref)
    worst = float(np.max(diff / bound)) if on.size else 0.0
    plain = half_ulp < tol
    err_plain = float(diff[plain].max()) if plain.any() else 0.0
    if dtype == "fp32":
        ulps_m = ulps_l = None
    else:
        um = oracle.ulp(m_ref, MANT_BITS[dtype])
        ul = oracle.ulp(l_ref, MANT_BITS[dtype])
        ulps_m = float((err_m / um).max()) if err_m.size else 0.0
        ulps_l = float((err_l / ul).max()) if err_l.size else 0.0
    report = {"err_o": err_o, "err_o_where_representable": err_plain, "floor_o": floor,
              "worst_over_bound": worst,
              "err_m": float(err_m.max()) if err_m.size else 0.0,
              "err_l": float(err_l.max()) if err_l.size else 0.0,
              "ulps_m": ulps_m, "ulps_l": ulps_l}
    _log(label, dtype, (B, H, S, D), causal, rows, report)
    assert worst <= 1.0, (f"{label}: O beyond bound: max|dO| {err_o:.3g} (tol {tol}, floor {floor:.3g}, "
                          f"worst error/bound {worst:.3f})")
    if not check_ml:
        return report
    if dtype == "fp32":
        assert np.all(err_m <= 1e-5 + 1e-5 * np.abs(m_ref)), f"{label}: m beyond all_close, max {err_m.max():.3g}"
        assert np.all(err_l <= 1e-5 + 1e-5 * np.abs(l_ref)), f"{label}: l beyond all_close, max {err_l.max():.3g}"
    else:
        assert np.all(err_m <= um), f"{label}: m beyond 1 ulp ({ulps_m:.2f} ulp)"
        assert np.all(err_l <= ul), f"{label}: l beyond 1 ulp ({ulps_l:.2f} ulp)"
    return report


def _log(label, dtype, shape, causal, rows, report):
    """Append one JSON line per check to the file PMKL_PARITY_LOG names (if
    set): the per-configuration error table is built from these records."""
    import json
    import os

    path = os.environ.get("PMKL_PARITY_LOG")
    if not path:
        return
    rec = {"label": label, "dtype": dtype, "shape": list(shape), "causal": bool(causal),
           "rows": None if rows is None else len(rows), **report}
    with open(path, "a") as f:
        f.write(json.dumps(rec) + "\n")


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float64 values to the dtype (RNE), back as float64."""
    import torch

    tdt = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}[dtype]
    return torch.from_numpy(np.asarray(x, dtype=np.float64)).to(tdt).double().numpy()
