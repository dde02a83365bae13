"""Builds tests/cpp/_bin/test_causal_attention, the C++ drop-in test.

It includes include/pmkl/nlp/causal_attention.h as a reference caller would,
links libpmkl_attn.so, and checks its results against the float64 oracle
(oracle/liboracle.so, built by `make -C oracle`).  Test infrastructure only.
"""
from __future__ import annotations

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
SRC = ROOT / "tests" / "cpp" / "test_causal_attention.cpp"
BIN = ROOT / "tests" / "cpp" / "_bin" / "test_causal_attention"


def build() -> Path:
    if str(ROOT) not in sys.path:
        sys.path.insert(0, str(ROOT))
    from pmkl_amd import _build

    BIN.parent.mkdir(parents=True, exist_ok=True)
    _build._run([_build.HIPCC, *_build.HIP_FLAGS, "-I", str(_build.INCLUDE), str(SRC),
                 f"-L{_build.PKG}", "-lpmkl_attn", f"-L{ROOT / 'oracle'}", "-loracle",
                 "-Wl,-rpath,$ORIGIN/../../../pmkl_amd", "-Wl,-rpath,$ORIGIN/../../../oracle",
                 "-o", str(BIN)])
    return BIN


if __name__ == "__main__":
    print(build())
