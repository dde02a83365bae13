"""Child-process check of the kernel-choice switches (run by
tests/test_switches_gpu.py with the environment set; the C ABI reads each
switch once per process).  Runs a few 16-bit shapes that the switch affects
through pmkl_attn_fwd and compares them with the float64 oracle; exits 0 when
all are within the stated tolerances, prints the failure and exits 1
otherwise."""
from __future__ import annotations

import os
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))


def main() -> int:
    import torch

    import pmkl_amd
    from pmkl_amd.workloads import small_inputs
    from tests.parity import check_outputs

    dev = torch.device("cuda:0")
    shapes = [(1, 3, 300, 128, "bf16", True), (2, 2, 257, 128, "fp16", False), (1, 2, 520, 64, "bf16", True),
              (2, 2, 200, 32, "fp16", True), (1, 5, 1000, 128, "bf16", True), (3, 2, 256, 64, "fp16", True),
              (2, 2, 128, 128, "bf16", False), (1, 2, 129, 128, "fp16", True), (2, 1, 384, 128, "bf16", False),
              (1, 4, 128, 64, "fp32", True), (2, 1, 300, 128, "fp32", False), (1, 2, 33, 32, "fp32", True)]
    env = {k: v for k, v in os.environ.items() if k.startswith("PMKL_ATTN")}
    for i, (B, H, S, D, dt, causal) in enumerate(shapes):
        tag = f"{env} {dt} B{B} H{H} S{S} D{D} causal={causal}"
        print(f"case {tag}", flush=True)
        q, k, v = small_inputs(B, H, S, D, dt, seed=4000 + i)
        o, m, l = pmkl_amd.attn_fwd(q.to(dev), k.to(dev), v.to(dev), is_causal=causal)
        torch.cuda.synchronize()
        errs = check_outputs(q, k, v, o, m, l, dt, causal=causal, label=tag)
        print(f"  {errs}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
