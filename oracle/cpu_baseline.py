"""TEST INFRASTRUCTURE ONLY - worker of bench.py's CPU-baseline leg.

Times the reference's own CPU operator (oracle/_ref, compiled from
pmkl_pytorch_ext/fused_self_attention.cpp; its body :5-64 walks the heads
one after the other on one thread) on one head of a workload.  bench.py runs
one such worker alone (the single-core figure, the reference as written) and
then one per core at once, each on its own head (the all-cores figure: the
heads are independent, so a static partition of heads over processes is the
faithful parallelisation).

Protocol (stdin/stdout, one line each): the worker loads its head from the
.npz the parent wrote, runs the operator once on a tiny input (to page in
its code), prints "ready", waits for any line on stdin ("go"), times one
call of fused_self_attention_fw on its head with torch's intra-op threads
set to 1, and prints a JSON line {"head": h, "seconds": t}.  It never touches
a GPU.

Usage: python -m oracle.cpu_baseline <inputs.npz> <head index>
"""
from __future__ import annotations

import json
import sys
import time


def main(argv) -> int:
    import numpy as np
    import torch

    from oracle import oracle

    path, head = argv[0], int(argv[1])
    torch.set_num_threads(1)
    ref = oracle.reference_op()
    if ref is None:
        print(json.dumps({"error": "oracle/_ref is not built"}), flush=True)
        return 1
    with np.load(path, allow_pickle=False) as z:
        dtype = str(z["dtype"])
        causal = bool(z["causal"])
        q, k, v = (np.ascontiguousarray(z[name][head]) for name in ("q", "k", "v"))
    dt = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}[dtype]
    S, D = q.shape
    qt, kt, vt = (torch.from_numpy(a).to(dt).reshape(1, 1, S, D) for a in (q, k, v))
    tiny = qt[:, :, :8].contiguous()
    ref.fused_self_attention_fw(tiny, tiny, tiny, causal)
    print("ready", flush=True)
    sys.stdin.readline()
    t0 = time.perf_counter()
    ref.fused_self_attention_fw(qt, kt, vt, causal)
    dt_s = time.perf_counter() - t0
    print(json.dumps({"head": head, "seconds": dt_s}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
