"""Helpers of the GPU parity tests: run the HIP optimizer and the CPU oracle
on identical seeded inputs and compare params and every state tensor."""

from __future__ import annotations

import weakref

import numpy as np
import pytest
import torch

from oracle.cresso_oracle import OracleCRESSO5

needs_gpu = pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X GPU")

# north-star tolerances
F32_TOL = dict(rtol=1e-5, atol=1e-6)
# bf16/fp16 params: each element within one ulp of the param dtype plus one
# ulp of the rounded update (the reference rounds drive*gain to the param
# dtype before applying it, p.add_(u.to(p.dtype), alpha=-lr), cresso_v5.py:1353,
# so an fp32 rounding tie of u moves p by lr*ulp(u), about 2*ulp(|dp|)), and at
# most ULP_FRACTION of the elements different at all
BF16_PARAM_TOL = dict(ulp=1)
ULP_FRACTION = 0.02
# per-step update dp = p_after - p_before against the oracle's, element-wise,
# relative to |dp| plus the rms of the oracle's dp (the update's own scale)
DP_RTOL = {torch.float32: 1e-4, torch.float64: 1e-9}

_PREV = weakref.WeakKeyDictionary()   # hip optimizer -> (hip params, oracle params) before the last step


def same_sum(a: float, b: float) -> bool:
    """Checksums of regenerated inputs: torch's CPU fp64 sum order differs
    between hosts (vector width), so the last digits may differ."""
    return abs(a - b) <= 1e-12 * max(1.0, abs(a), abs(b))


def announce(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


def run_pair(shapes, dtype, kwargs, steps, seed=0, grad_std=1e-2, param_std=0.05, grad_scales=None):
    """-> (hip params, hip optimizer, oracle params, oracle optimizer) after `steps` steps."""
    import cresso_amd

    gen = torch.Generator().manual_seed(seed)
    p0 = [(param_std * torch.randn(s, generator=gen)).to(dtype) for s in shapes]
    grads = []
    for _ in range(steps):
        gs = []
        for i, s in enumerate(shapes):
            sc = 1.0 if grad_scales is None else grad_scales[i]
            gs.append((sc * grad_std * torch.randn(s, generator=gen)).to(dtype))
        grads.append(gs)
    hp = [torch.nn.Parameter(p.clone().cuda()) for p in p0]
    op = [p.clone() for p in p0]
    hopt = cresso_amd.CRESSO5(hp, cuda_ops="required", **kwargs)
    oopt = OracleCRESSO5(op, **kwargs)
    for k, gs in enumerate(grads):
        if k == len(grads) - 1:
            torch.cuda.synchronize()
            _PREV[hopt] = ([p.detach().clone() for p in hp], [p.clone() for p in op])
        for p, g in zip(hp, gs):
            p.grad = g.cuda()
        hopt.step()
        oopt.step(gs)
    torch.cuda.synchronize()
    return hp, hopt, op, oopt


def _ulp(x: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """Spacing of the dtype's values at |x| (float64 array)."""
    mant, emin = {torch.bfloat16: (7, -126), torch.float16: (10, -14)}[dtype]
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** emin)))
    return 2.0 ** (e - mant)


def check_low_precision_param(got: np.ndarray, exp: np.ndarray, dtype: torch.dtype, what: str,
                              exp_prev=None, got_prev=None) -> float:
    """bf16/fp16 param values (as float64) against the oracle's after one step.

    exp_prev / got_prev: the oracle's / HIP side's param before the step.  Each
    element may differ by the difference it already had before the step
    (carried), plus one ulp of the new value (rounding tie of p), plus one ulp
    of the rounded update (tie of u = cast(drive*gain), which moves p by
    lr*ulp(u) <= 2*ulp(|dp|)).  At most ULP_FRACTION of the elements (or 4)
    may differ by more than they already did.  -> that fraction."""
    diff = np.abs(got - exp)
    carried = np.zeros_like(diff) if got_prev is None else np.abs(got_prev - exp_prev)
    allow = carried + _ulp(np.maximum(np.abs(got), np.abs(exp)), dtype)
    if exp_prev is not None:
        allow = allow + 2.0 * _ulp(np.abs(exp - exp_prev), dtype)
    worst = float((diff / allow).max()) if diff.size else 0.0
    newly = int((diff > carried).sum())
    frac = newly / diff.size if diff.size else 0.0
    assert worst <= 1.0 + 1e-9, f"{what}: {worst:.2f} x the allowed difference (max)"
    # (a few ties are allowed in tiny tensors)
    assert newly <= max(ULP_FRACTION * diff.size, 4), f"{what}: {100 * frac:.2f}% of the elements newly differ"
    return frac


def check_update(dg: np.ndarray, de: np.ndarray, rtol: float, what: str) -> float:
    """Per-step update of the HIP side (dg) against the oracle's (de); -> worst normalized error."""
    scale = float(np.sqrt(np.mean(de * de))) if de.size else 0.0
    err = np.abs(dg - de) / (np.abs(de) + scale + 1e-30)
    worst = float(err.max()) if err.size else 0.0
    assert worst <= rtol, f"{what}: update differs by {worst:.3e} of its scale (limit {rtol:.1e})"
    return worst


def compare(hp, hopt, op, oopt, param_tol=F32_TOL, state_tol=F32_TOL, skip_keys=(), dp_rtol=None):
    prev = _PREV.get(hopt)
    for i, (a, b) in enumerate(zip(hp, op)):
        what = f"param {i} shape {tuple(b.shape)} {b.dtype}"
        got = a.detach().double().cpu().numpy()
        exp = b.double().numpy()
        if b.dtype in (torch.bfloat16, torch.float16):
            check_low_precision_param(got, exp, b.dtype, what,
                                      None if prev is None else prev[1][i].double().numpy(),
                                      None if prev is None else prev[0][i].double().cpu().numpy())
        else:
            np.testing.assert_allclose(got, exp, **param_tol, err_msg=what)
            if prev is not None and b.dtype in DP_RTOL:
                dg = got - prev[0][i].double().cpu().numpy()
                de = exp - prev[1][i].double().numpy()
                check_update(dg, de, DP_RTOL[b.dtype] if dp_rtol is None else dp_rtol, what)
        sa = hopt.state[a]
        sb = oopt.state[i]
        assert set(sa.keys()) == set(sb.keys()), (sorted(sa), sorted(sb))
        for k, v in sb.items():
            if k in skip_keys:
                continue
            got = sa[k]
            if torch.is_tensor(v):
                assert got.dtype == v.dtype, (k, got.dtype, v.dtype)
                assert tuple(got.shape) == tuple(v.shape), k
                np.testing.assert_allclose(got.double().cpu().numpy(), v.double().numpy(), **state_tol,
                                           err_msg=f"param {i} shape {tuple(b.shape)} state {k}")
            else:
                assert got == v, (k, got, v)
