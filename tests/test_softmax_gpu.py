"""GPU parity tests of the gfx950 row softmax / log-softmax (pmkl_softmax_fwd
through the C ABI) against the float64 oracle (oracle/softmax_oracle.c, the
restatement of pmkl/norm/warp_softmax.h:74-201).

Tolerance (per element, y the device result, w the oracle value, d = |x - max|):
  fp32 softmax:      |y - w| <= (16 + d) * 2^-24 * |w| + 2^-126
  fp32 log-softmax:  |y - w| <= (d + |w| + 16) * 2^-23
  16-bit outputs:    the fp32 bound + 1 ulp of w in the output type (at least
                     its subnormal spacing) + 2^-126.
The d term is the rounding of x - max in fp32 (exp turns an absolute error in
its argument into a relative one); any fp32 implementation, the reference's
included, carries it.  16 ulps cover the exponential, the reciprocal and the
sum.  NaN and +-inf must match the oracle exactly.  The reference's own case
(12 x 1024 fp32, U(-10, 10)) is also held to its own criterion, all_close
atol = rtol = 1e-5 against its CPU check (test/test_softmax.cpp:53-56).

The padding of each source row (stride > elements) is filled with NaN, so a
read past the row would poison it; the padding of each destination row is
filled with a sentinel that must survive.
"""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
MANT = {"fp32": 23, "fp16": 10, "bf16": 7}
MIN_EXP = {"fp32": -149, "fp16": -24, "bf16": -133}
SENTINEL = -7.0


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _tdt(name):
    import torch

    return {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}[name]


def _bound(w, d, out_dt, is_log):
    w = np.abs(w)
    if is_log:
        b = np.ldexp(d + w + 16.0, -23)
    else:
        b = (16.0 + d) * w * 2.0 ** -24 + 2.0 ** -126
    if out_dt != "fp32":
        e = np.floor(np.log2(np.where(w > 0, w, 1e-30))) - MANT[out_dt]
        b = b + np.ldexp(1.0, np.maximum(e, MIN_EXP[out_dt]).astype(np.int64)) + 2.0 ** -126
    return b


def _check(y, x, n, out_dt, is_log, label):
    """y: device result [batch, n] as float64; x: the inputs [batch, >= n] as float64."""
    w = oracle.softmax_f64(x, n=n, is_log=is_log)
    xr = x[:, :n]
    with np.errstate(invalid="ignore"):
        d = np.abs(xr - np.nanmax(np.where(np.isnan(xr), -np.inf, xr), axis=1, keepdims=True))
    special = ~np.isfinite(w)
    assert np.array_equal(np.isnan(y), np.isnan(w)), f"{label}: NaN pattern differs"
    assert np.array_equal(y[special & ~np.isnan(w)], w[special & ~np.isnan(w)]), f"{label}: inf differs"
    fin = ~special
    err = np.abs(y[fin] - w[fin])
    bound = _bound(w[fin], np.where(np.isfinite(d), d, 0.0)[fin], out_dt, is_log)
    worst = float((err / bound).max()) if err.size else 0.0
    assert worst <= 1.0, f"{label}: beyond bound (worst err/bound {worst:.3f}, max err {err.max():.3g})"
    return worst


def _host_inputs(batch, n, stride, in_dt, seed, lo=-10.0, hi=10.0):
    """[batch, stride] float64 host copy of the inputs rounded to in_dt; the
    padding columns hold NaN."""
    import torch

    rng = np.random.Generator(np.random.PCG64(seed))
    x = np.full((batch, stride), np.nan)
    x[:, :n] = rng.uniform(lo, hi, size=(batch, n))
    xt = torch.from_numpy(x.astype(np.float32)).to(_tdt(in_dt))
    return xt, xt.to(torch.float64).numpy()


def _run(batch, n, stride, in_dt, out_dt, is_log, seed, lo=-10.0, hi=10.0, offset=0, in_place=False,
         xt=None):
    import torch

    import pmkl_amd

    if xt is None:
        xt, x64 = _host_inputs(batch, n, stride, in_dt, seed, lo, hi)
    else:
        x64 = xt.to(torch.float64).numpy()
    total = batch * stride
    src_buf = torch.empty(total + 16, dtype=_tdt(in_dt), device="cuda:0")
    src = src_buf[offset:offset + total]
    src.copy_(xt.reshape(-1).to("cuda:0"))
    if in_place:
        dst = src
    else:
        dst_buf = torch.full((total + 16,), SENTINEL, dtype=_tdt(out_dt), device="cuda:0")
        dst = dst_buf[offset:offset + total]
    pmkl_amd.warp_softmax_forward(dst, src, n, stride, batch, is_log_softmax=is_log)
    torch.cuda.synchronize()
    y = dst.reshape(batch, stride).to("cpu", torch.float64).numpy()
    if not in_place and stride > n:
        assert (y[:, n:] == SENTINEL).all(), "destination padding was written"
    return y[:, :n], x64


NS = [1, 2, 3, 4, 5, 7, 8, 9, 15, 16, 17, 31, 32, 33, 63, 64, 65, 100, 127, 128, 129, 255, 256, 257,
      500, 511, 512, 513, 768, 1000, 1023, 1024]


@pytest.mark.parametrize("dt", ["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("is_log", [False, True])
def test_row_lengths_sweep(device, dt, is_log):
    worst = 0.0
    for i, n in enumerate(NS):
        label = f"softmax {dt} log={is_log} batch 37 n={n}"
        _say(f"case {label}")
        y, x = _run(37, n, n, dt, dt, is_log, seed=1000 + i)
        worst = max(worst, _check(y, x, n, dt, is_log, label))
    _say(f"  worst err/bound {worst:.3f}")


@pytest.mark.parametrize("in_dt,out_dt", [("fp16", "fp32"), ("bf16", "fp32"), ("fp32", "fp16"), ("fp32", "bf16"),
                                          ("fp16", "bf16")])
def test_mixed_types(device, in_dt, out_dt):
    for n in (64, 77, 1024):
        for is_log in (False, True):
            label = f"softmax {in_dt}->{out_dt} log={is_log} n={n}"
            _say(f"case {label}")
            y, x = _run(50, n, n, in_dt, out_dt, is_log, seed=n + 7)
            _check(y, x, n, out_dt, is_log, label)


@pytest.mark.parametrize("dt,n,stride", [("fp32", 100, 128), ("bf16", 100, 104), ("fp32", 33, 40),
                                         ("fp16", 1024, 1032), ("bf16", 7, 9), ("fp32", 1, 3)])
def test_strided_rows(device, dt, n, stride):
    for is_log in (False, True):
        label = f"softmax {dt} n={n} stride={stride} log={is_log}"
        _say(f"case {label}")
        y, x = _run(45, n, stride, dt, dt, is_log, seed=stride)
        _check(y, x, n, dt, is_log, label)


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
def test_unaligned_pointers(device, dt):
    """Bases off 16-byte alignment take the element-wise path."""
    for n in (256, 1024, 40):
        label = f"softmax {dt} n={n} base offset 1 element"
        _say(f"case {label}")
        y, x = _run(20, n, n, dt, dt, False, seed=n, offset=1)
        _check(y, x, n, dt, False, label)


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
def test_in_place(device, dt):
    for n in (512, 33):
        label = f"softmax {dt} n={n} in place"
        _say(f"case {label}")
        y, x = _run(64, n, n, dt, dt, True, seed=5, in_place=True)
        _check(y, x, n, dt, True, label)


def test_special_values(device):
    import torch

    rows = [
        [0.0, 1.0, float("nan"), 2.0] + [0.5] * 60,
        [0.0, -float("inf"), 1.0, -float("inf")] + [-3.0] * 60,
        [-float("inf")] * 64,
        [float("inf"), 0.0, 1.0, 2.0] + [0.0] * 60,
        [1.0e4, 0.0, -1.0e4, 9.99e3] + [-2.0e4] * 60,
        [-1.0e30, -1.0e30 + 1e24] + [-3.0e38] * 62,
        [1e-30] * 64,
    ]
    for dt in ("fp32", "bf16"):
        xt = torch.tensor(rows, dtype=torch.float32).to(_tdt(dt))
        for is_log in (False, True):
            label = f"special values {dt} log={is_log}"
            _say(f"case {label}")
            y, x = _run(len(rows), 64, 64, dt, dt, is_log, seed=0, xt=xt)
            _check(y, x, 64, dt, is_log, label)
    xt = torch.tensor([r[:64] for r in rows[:4]], dtype=torch.float32).to(torch.float16)
    y, x = _run(4, 64, 64, "fp16", "fp16", False, seed=0, xt=xt)
    _check(y, x, 64, "fp16", False, "special values fp16")


def test_single_element_rows_are_exactly_one(device):
    y, _ = _run(1000, 1, 1, "fp32", "fp32", False, seed=3)
    assert (y == 1.0).all()
    y, _ = _run(1000, 1, 1, "bf16", "bf16", True, seed=3)
    assert (y == 0.0).all()


def test_reference_case_and_criterion(device):
    """test/test_softmax.cpp:30-60: 12 x 1024 fp32 in U(-10, 10), all_close
    atol = rtol = 1e-5 against its CPU check host_softmax_forward."""
    import torch

    rng = np.random.Generator(np.random.PCG64(2024))
    x = rng.uniform(-10.0, 10.0, size=(12, 1024)).astype(np.float32)
    y, _ = _run(12, 1024, 1024, "fp32", "fp32", False, seed=0, xt=torch.from_numpy(x))
    host = oracle.softmax_host_f32(x).astype(np.float64)
    assert not np.isnan(y).any()
    assert np.all(np.abs(y - host) <= 1e-5 + 1e-5 * np.abs(host))
    _check(y, x.astype(np.float64), 1024, "fp32", False, "reference case vs float64 oracle")


def test_full_size_properties(device):
    """The benchmark workload, 131,072 rows x 1,024 fp32 (and bf16): every row
    sums to 1 (log: logsumexp 0) within the element bound, and sampled rows
    match the oracle."""
    import torch

    import pmkl_amd

    rows, n = 131072, 1024
    g = torch.Generator(device="cuda:0").manual_seed(99)
    for dt in ("fp32", "bf16"):
        x = (torch.rand((rows, n), generator=g, device="cuda:0") * 20.0 - 10.0).to(_tdt(dt))
        for is_log in (False, True):
            label = f"full size {dt} log={is_log}"
            _say(f"case {label}")
            y = pmkl_amd.softmax(x, is_log=is_log)
            torch.cuda.synchronize()
            y64 = y.to(torch.float64)
            if is_log:
                lse = torch.logsumexp(y64, dim=1)
                tol = 2.0 ** -16 if dt == "fp32" else 2.0 ** -5
                assert float(lse.abs().max()) <= tol, f"{label}: logsumexp {float(lse.abs().max())}"
            else:
                tot = y64.sum(dim=1)
                tol = 2.0 ** -18 if dt == "fp32" else 2.0 ** -8
                assert float((tot - 1.0).abs().max()) <= tol, f"{label}: row sums off by {float((tot - 1).abs().max())}"
            pick = torch.randint(0, rows, (64,), generator=g, device="cuda:0")
            xs = x[pick].to("cpu", torch.float64).numpy()
            ys = y64[pick].cpu().numpy()
            _check(ys, xs, n, dt, is_log, label + " sampled rows")
            del y, y64


def test_softmax_wrapper_shapes(device):
    """pmkl_amd.softmax over the last dim of 3-D and strided (sliced) tensors."""
    import torch

    import pmkl_amd

    x = torch.randn(3, 5, 200, device="cuda:0")
    y = pmkl_amd.softmax(x)
    assert y.shape == x.shape
    assert torch.allclose(y, torch.softmax(x.double(), dim=-1).float(), rtol=1e-5, atol=1e-7)
    base = torch.randn(40, 136, device="cuda:0", dtype=torch.bfloat16)
    xs = base[:, :128]
    ys = pmkl_amd.softmax(xs, is_log=True, out_dtype=torch.float32)
    assert ys.shape == xs.shape and ys.dtype == torch.float32
    ref = torch.log_softmax(xs.double(), dim=-1)
    assert torch.allclose(ys.double(), ref, rtol=0, atol=1e-5)


def test_cpp_drop_in_header(device):
    """The C++ test binary (pmkl::norm::warp_softmax_forward) passes."""
    exe = ROOT / "tests" / "cpp" / "_bin" / "test_softmax"
    assert exe.exists(), "C++ test not built (run __graft_entry__.build())"
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=110)
    _say(res.stdout[-2000:])
    assert res.returncode == 0, res.stdout + res.stderr
