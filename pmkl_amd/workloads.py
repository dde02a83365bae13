"""Seeded synthetic inputs of the benchmark configurations.

Five configurations of the causal self-attention forward (scale 1/sqrt(D),
lower-triangular mask j <= i).  Inputs are drawn on the host with numpy's
PCG64 generator from a fixed seed, in float64, in the order q, k, v, then
cast to float32 and rounded to the compute dtype (round-to-nearest-even, the
rule torch.Tensor.to uses), so the same seed gives the same tensors on every
machine with this image.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class Workload:
    name: str
    dtype: str        # "fp32" | "fp16" | "bf16"
    B: int
    H: int
    S: int
    D: int
    seed: int
    note: str

    @property
    def shape(self):
        return (self.B, self.H, self.S, self.D)


WORKLOADS = {
    "C1": Workload("C1", "fp32", 1, 4, 128, 64, 1001, "Q/K/V ~ N(0,1); reference CPU-runnable case"),
    "C2": Workload("C2", "fp16", 8, 16, 1024, 64, 1002, "Q/K/V ~ N(0,1)"),
    "C3": Workload("C3", "bf16", 4, 32, 4096, 128, 1003, "Q/K/V ~ N(0,1); headline shape"),
    "C4": Workload("C4", "bf16", 1, 16, 16384, 128, 1004, "Q,K ~ N(0,0.5^2), V ~ U(-1,1); long sequence"),
    "C5": Workload("C5", "fp16", 64, 8, 256, 32, 1005, "Q/K/V ~ N(0,1), 1% of Q rows x8; many small heads"),
}


def causal_flops(B: int, H: int, S: int, D: int) -> int:
    """Multiply-add FLOPs of QK^T and PV over the visible (j <= i) pairs:
    4*D per pair, S*(S+1)/2 pairs per head (softmax not counted)."""
    return 2 * B * H * D * S * (S + 1)


def torch_dtype(name: str):
    import torch

    return {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}[name]


def host_inputs(w: Workload):
    """float32 numpy arrays q, k, v of shape [B, H, S, D] before dtype rounding."""
    rng = np.random.Generator(np.random.PCG64(w.seed))
    shape = w.shape
    if w.name == "C4":
        q = rng.normal(0.0, 0.5, size=shape)
        k = rng.normal(0.0, 0.5, size=shape)
        v = rng.uniform(-1.0, 1.0, size=shape)
    else:
        q = rng.standard_normal(size=shape)
        k = rng.standard_normal(size=shape)
        v = rng.standard_normal(size=shape)
    if w.name == "C5":
        n_rows = w.B * w.H * w.S
        n_out = int(round(0.01 * n_rows))
        rows = rng.choice(n_rows, size=n_out, replace=False)
        q.reshape(n_rows, w.D)[rows] *= 8.0
    return q.astype(np.float32), k.astype(np.float32), v.astype(np.float32)


def torch_inputs(w: Workload, device="cuda"):
    """q, k, v as torch tensors of the workload dtype on `device`."""
    import torch

    dt = torch_dtype(w.dtype)
    return tuple(torch.from_numpy(a).to(dt).to(device) for a in host_inputs(w))


def small_inputs(B, H, S, D, dtype: str, seed: int, dist: str = "normal"):
    """Seeded q, k, v (torch, CPU, in `dtype`) for parity tests at small sizes."""
    import torch

    rng = np.random.Generator(np.random.PCG64(seed))
    shape = (B, H, S, D)
    if dist == "uniform":
        arrs = [rng.uniform(-1.05, 1.05, size=shape) for _ in range(3)]
    else:
        arrs = [rng.standard_normal(size=shape) for _ in range(3)]
    dt = torch_dtype(dtype)
    return tuple(torch.from_numpy(a.astype(np.float32)).to(dt) for a in arrs)
