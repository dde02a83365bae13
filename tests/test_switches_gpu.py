"""The kernel-choice switches of the C ABI (PMKL_ATTN_W32, PMKL_ATTN_W64,
PMKL_ATTN_WAVES, PMKL_ATTN_NOXCD, PMKL_ATTN_RESIDENT, PMKL_ATTN_SPLIT, PMKL_ATTN_F32SPLIT) change which kernel runs, never the
results' definition: each setting runs tests/switch_check.py in a child
process (the library reads the switches once per process), which compares a
few shapes with the float64 oracle and reports the kernel the library chose
for each (pmkl_attn_fwd_kernel_name).  The kernels are checked against what
the setting promises, and against the default setting's choice, so a switch
that stopped changing the dispatch fails here."""
from __future__ import annotations

import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent

SETTINGS = [
    {"PMKL_ATTN_W32": "0"},                          # head_dim 128: one 64-row wave per SIMD
    {"PMKL_ATTN_W64": "0"},                          # every 16-bit call on the 4/8-wave MFMA kernel
    {"PMKL_ATTN_W64": "1"},                          # the slot-scheduled kernel at head_dim 32 and 64 too
    {"PMKL_ATTN_W64": "0", "PMKL_ATTN_WAVES": "4"},  # the 4-wave MFMA kernel everywhere
    {"PMKL_ATTN_NOXCD": "1"},                        # plain (head, tile) work order
    {"PMKL_ATTN_RESIDENT": "0"},                     # short sequences on the streaming 8-wave kernel
    {"PMKL_ATTN_SPLIT": "0"},                        # small causal head_dim-64 problems on 256-row workgroups
    {"PMKL_ATTN_F32SPLIT": "0"},                     # small fp32 problems on the 128-row fp32 kernel
]


def _run(setting):
    """Runs switch_check.py under `setting`; returns its shapes and kernel names."""
    env = {k: v for k, v in os.environ.items() if not k.startswith("PMKL_ATTN")}
    env.update(setting)
    res = subprocess.run([sys.executable, str(ROOT / "tests" / "switch_check.py")], env=env, cwd=str(ROOT),
                         capture_output=True, text=True, timeout=240)
    print(res.stdout[-3000:], flush=True)
    assert res.returncode == 0, res.stdout[-3000:] + res.stderr[-3000:]
    rec = json.loads(res.stdout.strip().splitlines()[-1])
    assert all(rec["kernels"]), rec
    return [tuple(s) for s in rec["shapes"]], rec["kernels"]


_DEFAULT = {}


def _default():
    if not _DEFAULT:
        _DEFAULT["shapes"], _DEFAULT["kernels"] = _run({})
    return _DEFAULT["shapes"], _DEFAULT["kernels"]


def _expect_kernels(setting, shapes, names, base):
    """What each setting promises about the kernel of each shape (shape:
    B, H, S, D, dtype, causal), and that it changes some choice."""
    sixteen = [(s, n) for s, n in zip(shapes, names) if s[4] != "fp32"]
    key = tuple(sorted(setting.items()))
    if key == (("PMKL_ATTN_W32", "0"),):
        for s, n, b in zip(shapes, names, base):
            if b.startswith("attn_fwd_w64_kernel") and ", 1, 8>" in b:
                assert n.startswith("attn_fwd_w64_kernel") and ", 2, 4>" in n, (s, n, b)
    elif key == (("PMKL_ATTN_W64", "0"),):
        assert not any(n.startswith("attn_fwd_w64_kernel") for _, n in sixteen), names
    elif key == (("PMKL_ATTN_W64", "1"),):
        for s, n in sixteen:
            assert n.startswith("attn_fwd_w64_kernel") == (s[2] > 128), (s, n)
    elif key == (("PMKL_ATTN_W64", "0"), ("PMKL_ATTN_WAVES", "4")):
        for s, n in sixteen:
            assert n.startswith("attn_fwd_mfma16_kernel") and ", 4, 0>" in n, (s, n)
    elif key == (("PMKL_ATTN_NOXCD", "1"),):
        assert not any("xcd order" in n for n in names), names
        assert any("xcd order" in b for b in base), base
    elif key == (("PMKL_ATTN_RESIDENT", "0"),):
        assert not any(n.startswith("attn_fwd_mfma16_kernel") and not n.split(">")[0].endswith(", 0")
                       for n in names), names
    elif key == (("PMKL_ATTN_SPLIT", "0"),):
        assert not any(", 64, causal, 1, 4>" in n for n in names), names
    elif key == (("PMKL_ATTN_F32SPLIT", "0"),):
        assert not any(n.startswith("attn_fwd_f32_split_kernel") for n in names), names
    else:
        raise AssertionError(f"no expectation for {setting}")
    changed = [(s, b, n) for s, b, n in zip(shapes, base, names) if b != n]
    assert changed, f"{setting} changed no kernel choice"


@pytest.mark.parametrize("setting", SETTINGS, ids=lambda s: ",".join(f"{k}={v}" for k, v in s.items()))
def test_switch_setting_vs_oracle(device, setting):
    shapes, base = _default()
    shapes_s, names = _run(setting)
    assert shapes_s == shapes
    _expect_kernels(setting, shapes, names, base)
