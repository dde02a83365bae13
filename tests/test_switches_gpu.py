"""The kernel-choice switches of the C ABI (PMKL_ATTN_W32, PMKL_ATTN_W64,
PMKL_ATTN_WAVES, PMKL_ATTN_NOXCD, PMKL_ATTN_RESIDENT, PMKL_ATTN_SPLIT, PMKL_ATTN_F32SPLIT) change which kernel runs, never the
results' definition: each setting runs tests/switch_check.py in a child
process (the library reads the switches once per process), which compares a
few shapes with the float64 oracle."""
from __future__ import annotations

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


@pytest.mark.parametrize("setting", SETTINGS, ids=lambda s: ",".join(f"{k}={v}" for k, v in s.items()))
def test_switch_setting_vs_oracle(device, setting):
    env = {k: v for k, v in os.environ.items() if not k.startswith("PMKL_ATTN")}
    env.update(setting)
    res = subprocess.run([sys.executable, str(ROOT / "tests" / "switch_check.py")], env=env, cwd=str(ROOT),
                         capture_output=True, text=True, timeout=240)
    print(res.stdout[-3000:], flush=True)
    assert res.returncode == 0, res.stdout[-3000:] + res.stderr[-3000:]
