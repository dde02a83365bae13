"""Writes the golden fixtures of the attention path (tests/golden/*.npz).

The expected outputs come from the reference's own CPU operator,
pmkl_pytorch_ext.fused_self_attention_fw (pmkl_pytorch_ext/fused_self_attention.cpp:
139-173), compiled from its source into oracle/_ref by oracle/Makefile:

  * in float64, where the reference computes the exact algorithm in double
    (the parity oracle must match it to rounding: these pin oracle/attn_oracle.c);
  * in float32, float16 and bfloat16, where it rounds after every operation
    as written (these pin the CPU branch of the torch operator bit for bit).

Each float64 case is cross-checked here against
torch.nn.functional.scaled_dot_product_attention in float64, the reference's
own Python oracle (test_fused_self_attention.py:6-7), before it is written.
Inputs are seeded (numpy PCG64) and stored once in float32; a rounded run
takes them rounded to its dtype (torch.Tensor.to, round-to-nearest-even).
bfloat16 outputs are stored as their uint16 bit patterns (numpy has no
bfloat16).

Backward fixtures (bwd_*.npz) come the same way from the reference's
pmkl_pytorch_ext.fused_self_attention_bw (fused_self_attention.cpp:175-215),
run per dtype on the m, l its own forward returned in that dtype (as the
reference's autograd backward does, pmkl_function/__init__.py:25-32), with a
seeded dout; the float64 case is cross-checked against torch autograd through
scaled_dot_product_attention in float64 before it is written.

Run from the repository root in a container that holds /root/reference:
    make -C oracle && python tests/golden/gen_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import torch  # noqa: E402

from oracle import oracle  # noqa: E402

OUT = Path(__file__).resolve().parent

# (name, B, H, S, D, causal, seed, distribution)
CASES = [
    ("s1_d32", 1, 1, 1, 32, True, 11, "normal"),
    ("s37_d64_causal", 1, 2, 37, 64, True, 12, "normal"),
    ("s37_d64_full", 1, 1, 37, 64, False, 13, "normal"),
    ("s48_d128_causal", 1, 1, 48, 128, True, 14, "uniform"),
    ("s130_d32_causal", 1, 1, 130, 32, True, 15, "normal"),
    ("s96_d64_outlier", 1, 1, 96, 64, True, 16, "outlier"),
]

TORCH = {"fp64": torch.float64, "fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}


def inputs(B, H, S, D, seed, dist):
    rng = np.random.Generator(np.random.PCG64(seed))
    shape = (B, H, S, D)
    if dist == "uniform":
        arrs = [rng.uniform(-1.05, 1.05, size=shape) for _ in range(3)]
    else:
        arrs = [rng.standard_normal(size=shape) for _ in range(3)]
    if dist == "outlier":   # a few query rows x8: near one-hot softmax rows
        arrs[0][:, :, ::13] *= 8.0
    return [a.astype(np.float32) for a in arrs]


# (name, B, H, S, D, causal, seed) of the backward fixtures (the reference's
# backward is O(S^3 D), so they stay small)
BWD_CASES = [
    ("s37_d64_causal", 1, 2, 37, 64, True, 21),
    ("s37_d64_full", 1, 1, 37, 64, False, 22),
    ("s48_d128_causal", 1, 1, 48, 128, True, 23),
    ("s20_d32_causal", 2, 1, 20, 32, True, 24),
]


def as_store(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def main():
    ref = oracle.reference_op()
    if ref is None:
        raise SystemExit("oracle/_ref is not built (make -C oracle in a container with the reference tree)")
    for name, B, H, S, D, causal, seed, dist in CASES:
        q, k, v = inputs(B, H, S, D, seed, dist)
        rec = {"B": B, "H": H, "S": S, "D": D, "causal": int(causal), "seed": seed,
               "q": q, "k": k, "v": v}
        for dt, tdt in TORCH.items():
            qt, kt, vt = (torch.from_numpy(a).to(tdt) for a in (q, k, v))
            o, m, l = ref.fused_self_attention_fw(qt, kt, vt, causal)
            if dt == "fp64":
                sd = oracle.attn_sdpa_f64(q.astype(np.float64).reshape(B * H, S, D),
                                          k.astype(np.float64).reshape(B * H, S, D),
                                          v.astype(np.float64).reshape(B * H, S, D), causal=causal)
                err = np.abs(o.numpy().reshape(B * H, S, D) - sd).max()
                assert err < 1e-12, f"{name}: reference fp64 vs SDPA float64 differ by {err}"
            rec[f"o_{dt}"] = as_store(o)
            rec[f"m_{dt}"] = as_store(m)
            rec[f"l_{dt}"] = as_store(l)
        path = OUT / f"ref_{name}.npz"
        np.savez_compressed(path, **rec)
        print(f"wrote {path.relative_to(ROOT)} ({path.stat().st_size} bytes)")
    for name, B, H, S, D, causal, seed in BWD_CASES:
        q, k, v = inputs(B, H, S, D, seed, "normal")
        dout = np.random.Generator(np.random.PCG64(seed + 1000)).standard_normal((B, H, S, D)).astype(np.float32)
        rec = {"B": B, "H": H, "S": S, "D": D, "causal": int(causal), "seed": seed,
               "q": q, "k": k, "v": v, "dout": dout}
        for dt, tdt in TORCH.items():
            qt, kt, vt, dot = (torch.from_numpy(a).to(tdt) for a in (q, k, v, dout))
            o, m, l = ref.fused_self_attention_fw(qt, kt, vt, causal)
            dq, dk, dv = ref.fused_self_attention_bw(dot, qt, kt, vt, m, l, causal)
            if dt == "fp64":
                ts = [torch.from_numpy(a.astype(np.float64)).requires_grad_() for a in (q, k, v)]
                ot = torch.nn.functional.scaled_dot_product_attention(
                    *ts, is_causal=causal, scale=oracle.default_scale(D))
                ot.backward(torch.from_numpy(dout.astype(np.float64)))
                for g, t in zip((dq, dk, dv), ts):
                    err = (g - t.grad).abs().max().item()
                    assert err < 1e-11, f"{name}: reference fp64 backward vs SDPA autograd differ by {err}"
            rec[f"m_{dt}"] = as_store(m)
            rec[f"l_{dt}"] = as_store(l)
            rec[f"dq_{dt}"] = as_store(dq)
            rec[f"dk_{dt}"] = as_store(dk)
            rec[f"dv_{dt}"] = as_store(dv)
        path = OUT / f"bwd_{name}.npz"
        np.savez_compressed(path, **rec)
        print(f"wrote {path.relative_to(ROOT)} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
