"""Builds tests/cpp/_bin/test_causal_attention and test_softmax, the C++
drop-in tests.

They include include/pmkl/nlp/causal_attention.h and
include/pmkl/norm/warp_softmax.h as a reference caller would, link
libpmkl_attn.so, and check their results against the oracle
(oracle/liboracle.so, built by `make -C oracle`).  Test infrastructure only.
"""
from __future__ import annotations

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
HERE = ROOT / "tests" / "cpp"
TESTS = ("test_causal_attention", "test_softmax")
BIN = HERE / "_bin" / "test_causal_attention"


def build() -> Path:
    if str(ROOT) not in sys.path:
        sys.path.insert(0, str(ROOT))
    from pmkl_amd import _build

    BIN.parent.mkdir(parents=True, exist_ok=True)
    for name in TESTS:
        _build._run([_build.HIPCC, *_build.HIP_FLAGS, "-I", str(_build.INCLUDE), str(HERE / (name + ".cpp")),
                     f"-L{_build.PKG}", "-lpmkl_attn", f"-L{ROOT / 'oracle'}", "-loracle",
                     "-Wl,-rpath,$ORIGIN/../../../pmkl_amd", "-Wl,-rpath,$ORIGIN/../../../oracle",
                     "-o", str(HERE / "_bin" / name)])
    return BIN.parent


if __name__ == "__main__":
    print(build())
