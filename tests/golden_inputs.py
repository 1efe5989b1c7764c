"""Load the golden fixtures under tests/golden/ and regenerate their seeded inputs."""

from __future__ import annotations

import json
from functools import lru_cache
from pathlib import Path
from typing import Dict, List, Tuple

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"
DTYPES = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16, "float64": torch.float64}


@lru_cache(maxsize=None)
def load(name: str) -> Dict[str, np.ndarray]:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def make_inputs(shape, dtype, steps, seed, grad_std=1.0, param_std=1.0, spike=False):
    """Same recipe as tests/golden/make_golden.py:make_inputs (torch CPU generator)."""
    gen = torch.Generator().manual_seed(seed)
    p0 = (param_std * torch.randn(shape, generator=gen, dtype=torch.float32)).to(dtype)
    grads = []
    for _ in range(steps):
        g = grad_std * torch.randn(shape, generator=gen, dtype=torch.float32)
        if spike:
            mask = torch.rand(shape, generator=gen) < 0.01
            g = torch.where(mask, g * 50.0, g)
        grads.append(g.to(dtype))
    return p0, grads


def _same(a: float, b: float) -> bool:
    # torch's CPU fp64 sum order differs between hosts: compare to ~1e-12
    return abs(a - b) <= 1e-12 * max(1.0, abs(a), abs(b))


def trajectory_names(file: str = "trajectories") -> List[str]:
    z = load(file)
    return sorted({k.split("/")[0] for k in z})


def trajectory(name: str, file: str = "trajectories"):
    """-> (meta, p0, grads, per-step expected dict) with inputs checked against stored sums."""
    z = load(file)
    pre = name + "/"
    sub = {k[len(pre):]: v for k, v in z.items() if k.startswith(pre)}
    meta = json.loads(str(sub["meta"]))
    dtype = DTYPES[meta["dtype"]]
    shape = tuple(meta["shape"])
    if "param0" in sub:
        p0 = torch.from_numpy(sub["param0"]).to(dtype)
        grads = [torch.from_numpy(sub[f"grad{k}"]).to(dtype) for k in range(meta["steps"])]
    else:
        p0, grads = make_inputs(shape, dtype, meta["steps"], meta["seed"], meta["grad_std"],
                                meta["param_std"], meta["spike"])
    assert _same(float(p0.double().sum()), float(sub["param0_sum"])), "regenerated param0 differs from fixture"
    for k, g in enumerate(grads):
        assert _same(float(g.double().sum()), float(sub[f"grad{k}_sum"])), "regenerated grad differs from fixture"
    steps = []
    for k in range(meta["steps"]):
        pk = f"step{k}/"
        d = {kk[len(pk):]: v for kk, v in sub.items() if kk.startswith(pk)}
        steps.append(d)
    return meta, p0, grads, steps, sub["sample_index"]
