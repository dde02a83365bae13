"""Pins the row softmax oracle (oracle/softmax_oracle.c) on the CPU.

The reference holds no golden vectors for pmkl::norm::warp_softmax_forward
(its test, test/test_softmax.cpp:30-60, draws rand() inputs and compares with
a CPU copy at all_close 1e-5), and its kernel cannot be built here (CUDA/SYCL
launcher).  The float64 restatement is therefore pinned by:
  * library routines: scipy.special.softmax / log_softmax and torch.softmax /
    log_softmax in float64;
  * closed forms: a constant row gives 1/n (log: -log n); two elements give
    the logistic function; one dominant element gives a one-hot row without
    overflow at |x| ~ 1e4 (which a missing max subtraction cannot reach);
  * invariants: shift invariance, rows summing to 1, logsumexp of a
    log-softmax row = 0, log(softmax) = log-softmax;
  * special values as the reference kernel produces them (NaN rows, -inf
    elements, all -inf rows);
  * the row placement r * stride of the reference's CPU check;
  * the reference's CPU check itself (softmax_host_f32, a restatement of
    test_softmax.cpp:10-28 in float) against the float64 oracle at the
    reference test's own all_close criterion.
Each check is shown to reject a planted mistake (a mutated copy of the
oracle), so it can fail.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle

RNG = np.random.Generator(np.random.PCG64(77))


def _rows(batch, n, lo=-10.0, hi=10.0):
    return RNG.uniform(lo, hi, size=(batch, n))


@pytest.mark.parametrize("n", [1, 2, 3, 31, 32, 33, 100, 128, 1000, 1024])
def test_matches_scipy_and_torch(n):
    import scipy.special as sp
    import torch

    x = _rows(7, n)
    y = oracle.softmax_f64(x)
    ly = oracle.softmax_f64(x, is_log=True)
    assert np.allclose(y, sp.softmax(x, axis=1), rtol=1e-14, atol=0)
    assert np.allclose(ly, sp.log_softmax(x, axis=1), rtol=1e-13, atol=1e-14)
    xt = torch.from_numpy(x)
    assert np.allclose(y, torch.softmax(xt, dim=1).numpy(), rtol=1e-14, atol=0)
    assert np.allclose(ly, torch.log_softmax(xt, dim=1).numpy(), rtol=1e-13, atol=1e-14)


def _closed_form_checks(softmax):
    """Closed forms and invariants; returns the list of failed check names."""
    failed = []
    for n in (1, 5, 1024):
        c = np.full((2, n), 3.25)
        if not np.allclose(softmax(c, False), 1.0 / n, rtol=1e-15, atol=0):
            failed.append(f"constant softmax n={n}")
        if not np.allclose(softmax(c, True), -np.log(n), rtol=1e-15, atol=1e-15):
            failed.append(f"constant log-softmax n={n}")
    a, b = 1.5, -0.75
    two = softmax(np.array([[a, b]]), False)[0]
    if not np.allclose(two, [1 / (1 + np.exp(b - a)), 1 / (1 + np.exp(a - b))], rtol=1e-15, atol=0):
        failed.append("two-element logistic")
    big = np.array([[1.0e4, 0.0, -1.0e4, 9.99e3]])
    yb = softmax(big, False)[0]
    if not (np.all(np.isfinite(yb)) and np.allclose(yb, [1 / (1 + np.exp(-10)), 0, 0, np.exp(-10) / (1 + np.exp(-10))],
                                                    rtol=1e-14, atol=1e-300)):
        failed.append("dominant element without overflow")
    x = _rows(5, 300)
    y = softmax(x, False)
    if not np.allclose(softmax(x + 123.0, False), y, rtol=1e-12, atol=0):
        failed.append("shift invariance")
    if not np.allclose(y.sum(axis=1), 1.0, rtol=1e-14, atol=0):
        failed.append("rows sum to 1")
    ly = softmax(x, True)
    mx = ly.max(axis=1, keepdims=True)
    if not np.allclose(mx[:, 0] + np.log(np.exp(ly - mx).sum(axis=1)), 0.0, atol=1e-13):
        failed.append("logsumexp of log-softmax")
    if not np.allclose(np.log(y), ly, rtol=1e-12, atol=1e-13):
        failed.append("log(softmax) == log-softmax")
    return failed


def _oracle_fn(x, is_log):
    return oracle.softmax_f64(x, is_log=is_log)


def test_closed_forms_and_invariants():
    assert _closed_form_checks(_oracle_fn) == []


def _mutant_no_max(x, is_log):     # exp(x) / sum exp(x): overflows at |x| ~ 1e4
    with np.errstate(over="ignore", invalid="ignore"):
        e = np.exp(x)
        s = e.sum(axis=1, keepdims=True)
        return np.log(e / s) if is_log else e / s


def _mutant_log_sign(x, is_log):    # (x - m) + log(s)
    m = x.max(axis=1, keepdims=True)
    s = np.exp(x - m).sum(axis=1, keepdims=True)
    return (x - m) + np.log(s) if is_log else np.exp(x - m) / s


def _mutant_off_by_one(x, is_log):  # the sum misses the last element
    m = x.max(axis=1, keepdims=True)
    e = np.exp(x - m)
    s = e[:, :-1].sum(axis=1, keepdims=True) if x.shape[1] > 1 else e.sum(axis=1, keepdims=True)
    return (x - m) - np.log(s) if is_log else e / s


def _mutant_no_log(x, is_log):      # log-softmax returns x - m - s
    m = x.max(axis=1, keepdims=True)
    s = np.exp(x - m).sum(axis=1, keepdims=True)
    return (x - m) - s if is_log else np.exp(x - m) / s


@pytest.mark.parametrize("mutant", [_mutant_no_max, _mutant_log_sign, _mutant_off_by_one, _mutant_no_log])
def test_checks_reject_planted_mistakes(mutant):
    assert _closed_form_checks(mutant) != []


def test_special_values():
    x = np.array([[0.0, 1.0, np.nan, 2.0],
                  [0.0, -np.inf, 1.0, -np.inf],
                  [-np.inf, -np.inf, -np.inf, -np.inf],
                  [np.inf, 0.0, 1.0, 2.0]])
    y = oracle.softmax_f64(x)
    ly = oracle.softmax_f64(x, is_log=True)
    assert np.isnan(y[0]).all() and np.isnan(ly[0]).all()          # a NaN poisons its row
    assert y[1, 1] == 0.0 and y[1, 3] == 0.0 and np.isclose(y[1, 0] + y[1, 2], 1.0)
    assert ly[1, 1] == -np.inf and ly[1, 3] == -np.inf
    assert np.isnan(y[2]).all() and np.isnan(ly[2]).all()          # -inf - (-inf) = NaN
    assert np.isnan(y[3]).all()                                    # inf - inf = NaN in the sum


def test_row_placement_strided():
    x = _rows(6, 40)
    y = oracle.softmax_f64(x, n=33)
    for r in range(6):
        assert np.allclose(y[r], oracle.softmax_f64(x[r:r + 1, :33])[0], rtol=0, atol=0)


def test_reference_host_check_vs_oracle():
    """The reference's own test: 12 x 1024 fp32, U(-10, 10), all_close 1e-5."""
    x = RNG.uniform(-10, 10, size=(12, 1024)).astype(np.float32)
    host = oracle.softmax_host_f32(x).astype(np.float64)
    ref = oracle.softmax_f64(x)
    assert np.all(np.abs(host - ref) <= 1e-5 + 1e-5 * np.abs(ref))
    # and the float copy is a faithful float computation: its error is the
    # rounding of x - max (|x - max| ulps, amplified by exp) plus a few dozen
    # ulps of the sequential float sum over 1024 terms
    d = np.abs(x.astype(np.float64) - x.max(axis=1, keepdims=True))
    assert np.all(np.abs(host - ref) <= (64.0 + d) * 2.0 ** -24 * ref)


def test_host_check_strided():
    x = _rows(4, 20).astype(np.float32)
    h = oracle.softmax_host_f32(x, n=17)
    assert h.shape == (4, 17)
    assert np.allclose(h, oracle.softmax_f64(x, n=17), rtol=2e-6, atol=0)
