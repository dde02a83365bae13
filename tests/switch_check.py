"""Child-process check of the kernel-choice switches (run by
tests/test_switches_gpu.py with the environment set; the C ABI reads each
switch once per process).  Runs a few shapes that the switches affect
through pmkl_attn_fwd and compares them with the float64 oracle; the last
line printed is a JSON list of the kernel the library chose for each shape
(pmkl_attn_fwd_kernel_name), which the parent checks against the setting.
Exits 0 when all are within the stated tolerances, prints the failure and
exits 1 otherwise."""
from __future__ import annotations

import json
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
              (1, 4, 128, 64, "fp32", True), (2, 1, 300, 128, "fp32", False), (1, 2, 33, 32, "fp32", True),
              (2, 8, 300, 64, "bf16", True)]
    env = {k: v for k, v in os.environ.items() if k.startswith("PMKL_ATTN")}
    names = []
    for i, (B, H, S, D, dt, causal) in enumerate(shapes):
        tag = f"{env} {dt} B{B} H{H} S{S} D{D} causal={causal}"
        print(f"case {tag}", flush=True)
        q, k, v = small_inputs(B, H, S, D, dt, seed=4000 + i)
        qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
        o, m, l = pmkl_amd.attn_fwd(qd, kd, vd, is_causal=causal)
        torch.cuda.synchronize()
        args = pmkl_amd.capi.make_args(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), o.data_ptr(), m.data_ptr(),
                                       l.data_ptr(), dtype=pmkl_amd.torch_dtype_to_pmkl(qd.dtype), batch=B,
                                       heads=H, seq_len=S, head_dim=D, is_causal=causal)
        names.append(pmkl_amd.capi.attn_fwd_kernel_name(args))
        print(f"  kernel {names[-1]}", flush=True)
        errs = check_outputs(q, k, v, o, m, l, dt, causal=causal, label=tag)
        print(f"  {errs}", flush=True)
    print(json.dumps({"shapes": [list(s) for s in shapes], "kernels": names}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
