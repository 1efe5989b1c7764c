"""Write the oracle's trajectories at the BASELINE configs' full sizes (TEST INFRASTRUCTURE).

    python tests/oracle_full/make_vectors.py [c2_bench c3_840 c4_shapes c5]

The CPU oracle (oracle/cresso_oracle.py, itself pinned to the reference's own
golden vectors by tests/test_oracle_golden.py) takes seconds to minutes per
step at these sizes, too slow to run inside a GPU test, so its results are
stored here and the GPU tests (tests/test_gpu_full_configs.py) regenerate the
same seeded inputs with bench.py's recipes and compare against them.

Each <name>.npz holds, per step k and tensor i: every state tensor
(``s{k}/t{i}/<key>``), the param at fixed sampled indices (``s{k}/t{i}/sample``,
indices in ``t{i}/index``), the fp64 sum and sum of squares of the whole
param and of its update dp = p_after - p_before (``dsum``, ``dsumsq``), and,
for fp32 params outside C3, the fp64 marginal sums of dp along every axis
(``dm{a}``: for each coordinate of axis a, the sum of dp over the other axes;
rows and columns of a matrix);
``t{i}/p0_sum`` and ``s{k}/t{i}/grad_sum`` are checksums of the
regenerated inputs.  Entries of one shape across all tensors are stored
stacked (``pack``).  Hash bin sums are accumulated in fp64 (the oracle's
``hash_accum="fp64"``): with 10^5 or more elements per bin the reference's
sequential fp32 scatter_add carries ~1e-5 relative error of its own.
"""

from __future__ import annotations

import json
import os
import sys
import time
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402  (input recipes)
from oracle.cresso_oracle import OracleCRESSO5  # noqa: E402

CASES = {
    "c1_fp64": ("c1", dict(pool=10), 10, 10, 4096),
    # name: (recipe, recipe kwargs, steps, grad pool, samples per tensor)
    "c2_bench": ("c2", dict(pool=4), 25, 4, 2048),
    "c3_840": ("c3", dict(pool=4), 4, 4, 256),
    "c4_shapes": ("c4", dict(pool=2, shapes=bench.C4_SHAPES), 2, 2, 4096),
    "c5": ("c5", dict(pool=2), 2, 2, 4096),
}


def make(recipe, **kw):
    cpu = torch.device("cpu")
    if recipe == "c1":
        return bench.make_c1(cpu, **kw)
    if recipe == "c2":
        return bench.make_c2(cpu, **kw)
    if recipe == "c3":
        return bench.make_c3(cpu, **kw)
    if recipe == "c4":
        return bench.make_c4(cpu, **kw)
    return bench.make_c5(cpu, **kw)


def sample_index(n: int, count: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    count = min(count, n)
    idx = rng.choice(n, size=count, replace=False) if n > count else np.arange(n)
    idx[:1] = 0
    idx[-1:] = n - 1
    return np.unique(idx).astype(np.int64)


def pack(out: dict, ntensors: int) -> dict:
    """Entries ``<pre>t{i}/<key>`` present for every tensor with one shape and
    dtype are stored once, stacked over the tensors, as ``<pre>stack/<key>``
    (tests/test_gpu_full_configs.py unpacks them)."""
    import re
    groups = {}
    for k, v in out.items():
        m = re.fullmatch(r"(.*?)t(\d+)/(.+)", k)
        if m:
            groups.setdefault((m.group(1), m.group(3)), {})[int(m.group(2))] = v
    packed = {k: v for k, v in out.items() if not re.fullmatch(r"(.*?)t(\d+)/(.+)", k)}
    for (pre, key), per in groups.items():
        arrs = [np.asarray(per.get(i)) for i in range(ntensors)]
        if len(per) == ntensors and len({(a.shape, a.dtype.str) for a in arrs}) == 1:
            packed[f"{pre}stack/{key}"] = np.stack(arrs)
        else:
            for i, a in per.items():
                packed[f"{pre}t{i}/{key}"] = a
    return packed


def run(name: str) -> None:
    recipe, rkw, steps, pool, ns = CASES[name]
    torch.set_num_threads(os.cpu_count() or 1)
    params, grads, kwargs, shapes, _ = make(recipe, **rkw)
    ps = [p.detach().clone() for p in params]
    out = {"meta": json.dumps(dict(recipe=recipe, recipe_kwargs={k: (v if k != "shapes" else [list(s) for s in v])
                                                                   for k, v in rkw.items()},
                                   steps=steps, pool=pool, kwargs=kwargs, hash_accum="fp64",
                                   shapes=[list(s) for s in shapes], dtypes=[str(p.dtype) for p in ps]))}
    idx = []
    for i, p in enumerate(ps):
        ix = sample_index(p.numel(), ns, 1000 + i)
        idx.append(torch.from_numpy(ix))
        out[f"t{i}/index"] = ix
        out[f"t{i}/p0_sum"] = np.float64(p.double().sum())
        out[f"t{i}/p0_sample"] = p.reshape(-1)[idx[i]].float().numpy()
    opt = OracleCRESSO5(ps, hash_accum="fp64", **kwargs)
    t0 = time.time()
    for k in range(steps):
        gs = grads[k % pool]
        before = [p.double().reshape(-1) for p in ps]
        opt.step(gs)
        for i, p in enumerate(ps):
            pre = f"s{k}/t{i}/"
            if k < pool:
                out[pre + "grad_sum"] = np.float64(gs[i].double().sum())
            flat = p.reshape(-1)
            out[pre + "sample"] = flat[idx[i]].float().numpy()
            out[pre + "sum"] = np.float64(flat.double().sum())
            out[pre + "sumsq"] = np.float64((flat.double() ** 2).sum())
            dp = flat.double() - before[i]
            out[pre + "dsum"] = np.float64(dp.sum())
            out[pre + "dsumsq"] = np.float64((dp * dp).sum())
            if recipe != "c3" and p.dtype == torch.float32:
                full = dp.view(tuple(p.shape))
                for a in range(p.ndim):
                    others = tuple(d for d in range(p.ndim) if d != a)
                    out[pre + f"dm{a}"] = (full.sum(dim=others) if others else full).numpy().copy()
            for key, v in opt.state[i].items():
                # copies: the oracle updates its state tensors in place
                out[pre + key] = v.numpy().copy() if torch.is_tensor(v) else np.int64(v)
        print(f"[{name}] step {k + 1}/{steps} done at {time.time() - t0:.1f} s", flush=True)
    np.savez_compressed(HERE / f"{name}.npz", **pack(out, len(ps)))
    print(f"[{name}] wrote {HERE / (name + '.npz')}", flush=True)


if __name__ == "__main__":
    for nm in (sys.argv[1:] or list(CASES)):
        run(nm)
