"""GPU parity at the BASELINE configs' full sizes.

* C1: the reference's own 10-step (2048, 2048) output (tests/golden/c1_2048.npz,
  written by running cresso_v5.py with cuda_ops="off").
* C2 over the benchmark's 25 steps, C3 with all 840 tensors through the
  steady-state path, one tensor of each C4 shape, and C5 (bf16 8192^2 and the
  fp32 conv / 3-D tensors at rank 16, T = 4, B = 256): against the CPU
  oracle's trajectories on bench.py's seeded inputs (tests/oracle_full/,
  written by tests/oracle_full/make_vectors.py; the oracle is pinned to the
  reference's golden vectors by tests/test_oracle_golden.py).

At every step: every state tensor (fp32 tolerance), the param at sampled
indices (fp32: rtol 1e-5 / atol 1e-6; bf16: within one ulp; 256 per tensor at
C3), the update dp = p_after - p_before at those indices against the
oracle's, over the whole tensor sum(dp) and sum(dp^2) in fp64, and for fp32
params of C1, C2, C4 and C5 the fp64 sums of dp along every axis (every row
and column of a matrix), so an O(rms) error in a single element of any row
or column that the samples miss exceeds its tolerance.
"""

from __future__ import annotations

import json
from functools import lru_cache
from pathlib import Path

import numpy as np
import pytest
import torch

from gpu_util import DP_RTOL, F32_TOL, announce, check_low_precision_param, check_update, needs_gpu, same_sum

pytestmark = [pytest.mark.gpu, needs_gpu]

HERE = Path(__file__).resolve().parent


@lru_cache(maxsize=None)
def _load(path: str):
    """The vectors as per-tensor entries (``<pre>stack/<key>`` rows become ``<pre>t{i}/<key>``)."""
    out = {}
    with np.load(path, allow_pickle=False) as z:
        for k in z.files:
            v = z[k]
            if "stack/" in k:
                pre, key = k.split("stack/", 1)
                for i in range(v.shape[0]):
                    out[f"{pre}t{i}/{key}"] = v[i]
            else:
                out[k] = v
    return out


def _states_close(got: dict, z: dict, pre: str, what: str, tol=F32_TOL) -> None:
    keys = [k[len(pre):] for k in z if k.startswith(pre) and "/" not in k[len(pre):]]
    skip = {"sample", "sum", "sumsq", "dsum", "dsumsq", "grad_sum"}
    for k in keys:
        if k in skip or k.startswith("dm"):   # dm{a}: marginal sums of dp, checked in _check_param
            continue
        assert k in got, f"{what}: state {k} missing"
        v = got[k]
        exp = z[pre + k]
        if torch.is_tensor(v):
            assert tuple(v.shape) == tuple(exp.shape), (what, k)
            if v.dtype == torch.long:
                np.testing.assert_array_equal(v.cpu().numpy(), exp, err_msg=f"{what} {k}")
            else:
                np.testing.assert_allclose(v.double().cpu().numpy(), exp.astype(np.float64), **tol,
                                           err_msg=f"{what} {k}")
        else:
            assert int(v) == int(exp), (what, k, v, exp)


class _Run:
    """Step the HIP optimizer on a recipe's inputs and compare each step with stored vectors."""

    def __init__(self, params, grads, kwargs, pool):
        import cresso_amd

        self.hp = [torch.nn.Parameter(p.detach().clone().cuda()) for p in params]
        self.gdev = [[g.cuda() for g in gs] for gs in grads]
        self.pool = pool
        self.opt = cresso_amd.CRESSO5(self.hp, cuda_ops="required", **kwargs)

    def step(self, k):
        for p, g in zip(self.hp, self.gdev[k % self.pool]):
            p.grad = g
        before = [p.detach().clone() for p in self.hp]
        self.opt.step()
        torch.cuda.synchronize()
        return before


def _check_param(i, p, before, z, pre, idx, prev_sample, what, worst):
    flat = p.detach().reshape(-1)
    got = flat[idx].double().cpu().numpy()
    exp = z[pre + "sample"].astype(np.float64)
    if p.dtype in (torch.bfloat16, torch.float16):
        got_prev = before.reshape(-1)[idx].double().cpu().numpy()
        worst["frac"] = max(worst.get("frac", 0.0),
                            check_low_precision_param(got, exp, p.dtype, what, prev_sample, got_prev))
        return
    np.testing.assert_allclose(got, exp, **F32_TOL, err_msg=f"{what} param sample")
    dg = got - before.reshape(-1)[idx].double().cpu().numpy()
    de = exp - prev_sample
    worst["dp"] = max(worst["dp"], check_update(dg, de, DP_RTOL[torch.float32], what))
    # whole-tensor checksums of the update
    dp = flat.double() - before.reshape(-1).double()
    n = flat.numel()
    dsum_e, dsq_e = float(z[pre + "dsum"]), float(z[pre + "dsumsq"])
    rms = (dsq_e / n) ** 0.5
    dsum_g = float(dp.sum())
    dsq_g = float((dp * dp).sum())
    worst["dsum"] = max(worst["dsum"], abs(dsum_g - dsum_e) / (rms * n ** 0.5 + 1e-30))
    # random per-element noise moves sum(dp) by ~1e-6 rms sqrt(n); a coherent
    # relative error of ~1e-7 (fp32 means over n elements, on either side) by
    # up to 1e-7 n rms; an error of O(rms) in m elements by m rms
    tol = 2e-7 * n * rms + 1e-4 * rms * n ** 0.5 + 1e-12
    assert abs(dsum_g - dsum_e) <= tol, f"{what}: sum(dp) {dsum_g!r} vs {dsum_e!r} (tolerance {tol:.3g})"
    np.testing.assert_allclose(dsq_g, dsq_e, rtol=1e-5, err_msg=f"{what}: sum(dp^2)")
    np.testing.assert_allclose(float(flat.double().pow(2).sum()), float(z[pre + "sumsq"]), rtol=1e-6,
                               err_msg=f"{what}: sum(p^2)")
    # marginal sums of dp along every axis (each row and each column of a
    # matrix), same tolerance per marginal of m elements: an O(rms) error in
    # one element of a row or column exceeds it
    full = dp.view(tuple(p.shape))
    a = 0
    while pre + f"dm{a}" in z:
        exp_m = z[pre + f"dm{a}"].astype(np.float64)
        others = tuple(d for d in range(p.ndim) if d != a)
        got_m = (full.sum(dim=others) if others else full).cpu().numpy()
        m = n // int(p.shape[a])
        tol_m = 2e-7 * m * rms + 1e-4 * rms * m ** 0.5 + 1e-12
        err = np.abs(got_m - exp_m) / tol_m
        worst["dm"] = max(worst.get("dm", 0.0), float(err.max()))
        bad = np.flatnonzero(err > 1.0)
        assert bad.size == 0, (f"{what}: sums of dp along axis {a} differ at coordinates {bad[:8].tolist()} "
                               f"(worst {err.max():.2f} x the tolerance)")
        worst["marginals"] = worst.get("marginals", 0) + exp_m.size
        a += 1


def _run_oracle_vectors(name: str, maker, state_tol=F32_TOL, on_step=None):
    import bench

    z = _load(str(HERE / "oracle_full" / f"{name}.npz"))
    meta = json.loads(str(z["meta"]))
    rkw = dict(meta["recipe_kwargs"])
    if "shapes" in rkw:
        rkw["shapes"] = [tuple(s) for s in rkw["shapes"]]
    params, grads, kwargs, shapes, _ = maker(torch.device("cpu"), **rkw)
    assert kwargs == meta["kwargs"], (kwargs, meta["kwargs"])
    for i, p in enumerate(params):
        assert same_sum(float(p.detach().double().sum()), float(z[f"t{i}/p0_sum"])), f"regenerated p0 {i} differs"
    for k in range(min(meta["steps"], meta["pool"])):
        for i, g in enumerate(grads[k]):
            assert same_sum(float(g.double().sum()), float(z[f"s{k}/t{i}/grad_sum"])), f"regenerated grad {k}/{i}"
    run = _Run(params, grads, kwargs, meta["pool"])
    idx = [torch.from_numpy(z[f"t{i}/index"]).cuda() for i in range(len(params))]
    prev = [z[f"t{i}/p0_sample"].astype(np.float64) for i in range(len(params))]
    worst = {"dp": 0.0, "dsum": 0.0, "frac": 0.0}
    for k in range(meta["steps"]):
        before = run.step(k)
        for i, p in enumerate(run.hp):
            pre = f"s{k}/t{i}/"
            what = f"{name} step {k + 1} tensor {i} {tuple(p.shape)} {p.dtype}"
            _states_close(run.opt.state[p], z, pre, what, state_tol)
            _check_param(i, p, before[i], z, pre, idx[i], prev[i], what, worst)
            prev[i] = z[pre + "sample"].astype(np.float64)
        if on_step is not None:
            on_step(k, run, z)
    announce(f"{name}: worst update error {worst['dp']:.2e} of its scale, sum(dp) {worst['dsum']:.2e} of "
             f"rms*sqrt(n), {worst.get('marginals', 0)} marginal sums of dp (worst {worst.get('dm', 0.0):.2f} of the "
             f"tolerance), low-precision params: {100 * worst['frac']:.2f}% of samples differ")


def test_c1_against_reference_golden_and_fp64_oracle_10_steps():
    """C1 on the HIP path: (a) every check above against the oracle with fp64
    hash-bin sums; (b) against the reference's own output (cresso_v5.py with
    cuda_ops="off", tests/golden/c1_2048.npz) at the fp32 tolerance, except
    where the reference itself is the side further from exact: with 65536
    elements per hash bin its sequential fp32 scatter_add carries ~1e-5
    relative error, so a value that misses the tolerance must be closer to the
    fp64-accumulation oracle than the reference's value is."""
    import bench
    from golden_inputs import load

    announce("C1 (2048,2048) x 10 steps vs the fp64 oracle and the reference's output")
    ref = load("c1_2048")
    ridx = torch.from_numpy(ref["sample_index"]).cuda()
    stats = {"ref_misses": 0, "checked": 0}

    def closer(got, r, o64, what):
        got, r, o64 = (np.asarray(v, dtype=np.float64) for v in (got, r, o64))
        ok = np.abs(got - r) <= 1e-6 + 1e-5 * np.abs(r)
        stats["checked"] += ok.size
        if ok.all():
            return
        bad = ~ok
        stats["ref_misses"] += int(bad.sum())
        assert (np.abs(got - o64)[bad] < np.abs(r - o64)[bad]).all(), \
            f"C1 {what}: differs from the reference beyond tolerance and is not the side closer to exact"

    def on_step(k, run, z):
        p = run.hp[0]
        st = run.opt.state[p]
        got = p.detach().reshape(-1)[ridx].double().cpu().numpy()
        o64 = None
        for key in ref:
            if not key.startswith(f"step{k}/state/"):
                continue
            sk = key.split("/")[-1]
            v = st[sk]
            if not torch.is_tensor(v):
                assert int(v) == int(ref[key])
            elif v.dtype == torch.long:
                assert torch.equal(v.cpu(), torch.from_numpy(ref[key]))
            else:
                closer(v.double().cpu().numpy(), ref[key], z[f"s{k}/t0/{sk}"], f"step {k + 1} {sk}")
        # the param at the reference's sampled indices: the fp64 oracle has no
        # value there, so these are held to the fp32 tolerance outright
        np.testing.assert_allclose(got, ref[f"step{k}/param_sample"].astype(np.float64), rtol=1e-5, atol=1e-6,
                                   err_msg=f"C1 step {k + 1} param at the reference's samples")

    _run_oracle_vectors("c1_fp64", bench.make_c1, on_step=on_step)
    announce(f"C1: {stats['ref_misses']} of {stats['checked']} state values outside the fp32 tolerance of the "
             f"reference, each closer to the fp64-accumulation oracle than the reference")


def test_c2_bench_inputs_25_steps():
    import bench

    announce("C2 (4096,4096) x 25 steps on the bench's inputs")
    _run_oracle_vectors("c2_bench", bench.make_c2)


def test_c3_all_840_tensors_steady_state():
    import bench

    announce("C3 840 LoRA-thin tensors x 4 steps (steps 2-4 on the steady-state path)")
    _run_oracle_vectors("c3_840", bench.make_c3)


def test_c4_each_shape():
    import bench

    announce("C4 shapes (32000,2048) (2048,2048) (5632,2048) (2048,5632) (2048,) x 2 steps")
    _run_oracle_vectors("c4_shapes", bench.make_c4)


def test_c5_rank16_t4_b256():
    import bench

    announce("C5 bf16 (8192,8192), (512,256,3,3), (256,256,3,3), (64,512,512) x 2 steps, rank 16, T=4, B=256")
    _run_oracle_vectors("c5", bench.make_c5)


def _c4_run(params0, grads, kwargs, batch: bool, lanes: int, steps: int):
    """Step a copy of the C4 params `steps` times with the spectral engine set to
    (BATCH, LANES); -> (params, optimizer) after the last step."""
    import cresso_amd
    from cresso_amd import spectral

    old = (spectral.SpectralEngine.BATCH, spectral.SpectralEngine.LANES)
    try:
        spectral.SpectralEngine.BATCH, spectral.SpectralEngine.LANES = batch, lanes
        ps = [torch.nn.Parameter(p.detach().clone()) for p in params0]
        opt = cresso_amd.CRESSO5(ps, cuda_ops="required", **kwargs)
        for k in range(steps):
            for p, g in zip(ps, grads[k % len(grads)]):
                p.grad = g
            opt.step()
        torch.cuda.synchronize()
        eng = opt._spectral_engine
        units = eng._units([eng._prepare(p, p.grad, opt.state[p], opt.param_groups[0]) for p in ps],
                           [opt.state[p] for p in ps])
    finally:
        spectral.SpectralEngine.BATCH, spectral.SpectralEngine.LANES = old
    return ps, opt, units


def test_c4_full_set_as_benched_batched_matches_per_tensor():
    """C4's 199 tensors (1.2 B fp32 elements) stepped the way bench.py times
    them -- same-plan tensors in batches of at most BATCH_BYTES of per-tensor
    scratch over LANES side streams, so the 88 (2048,2048) tensors go out as
    multi-round batches of about 30 that merge their histograms with atomics --
    against every tensor stepped on its own on one stream (one-round launches
    merge with partial rows).  Two steps; params and every state tensor must
    be bit-identical.  Parity of the per-tensor step itself against the oracle
    is test_c4_each_shape; the reference steps these tensors one by one
    (cresso_v5.py:828-844)."""
    import bench
    from cresso_amd import spectral

    announce("C4 full 199-tensor set: default batched engine (4 lanes) vs per-tensor steps on one stream, 2 steps")
    dev = torch.device("cuda:0")
    params, grads, kwargs, shapes, _ = bench.make_c4(dev, pool=2, on_device=True)
    a_ps, a_opt, a_units = _c4_run(params, grads, kwargs, True, spectral.SpectralEngine.LANES, 2)
    biggest = max(len(u[3]) for u in a_units)
    sq = [len(u[3]) for u in a_units if u[1][1] == (2048, 2048)]
    announce(f"batched engine: {len(a_units)} units, largest batch {biggest} tensors, (2048,2048) batches {sq}")
    assert biggest >= 20 and len(sq) >= 2, "the default engine no longer forms multi-round batches"
    b_ps, b_opt, b_units = _c4_run(params, grads, kwargs, False, 1, 2)
    assert max(len(u[3]) for u in b_units) == 1
    del params, grads
    for i, (a, b) in enumerate(zip(a_ps, b_ps)):
        what = f"C4 tensor {i} {tuple(a.shape)}"
        assert torch.equal(a.detach(), b.detach()), f"{what}: param differs"
        sa, sb = a_opt.state[a], b_opt.state[b]
        assert set(sa) == set(sb), what
        for k, v in sa.items():
            if torch.is_tensor(v):
                assert torch.equal(v, sb[k]), f"{what}: state {k} differs"
            else:
                assert v == sb[k], (what, k)
