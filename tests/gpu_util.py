"""Helpers of the GPU parity tests: run the HIP optimizer and the CPU oracle
on identical seeded inputs and compare params and every state tensor."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.cresso_oracle import OracleCRESSO5

needs_gpu = pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X GPU")

# north-star tolerances
F32_TOL = dict(rtol=1e-5, atol=1e-6)
BF16_PARAM_TOL = dict(rtol=1e-2, atol=1e-2)


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
    for gs in grads:
        for p, g in zip(hp, gs):
            p.grad = g.cuda()
        hopt.step()
        oopt.step(gs)
    torch.cuda.synchronize()
    return hp, hopt, op, oopt


def compare(hp, hopt, op, oopt, param_tol=F32_TOL, state_tol=F32_TOL, skip_keys=()):
    for i, (a, b) in enumerate(zip(hp, op)):
        np.testing.assert_allclose(a.detach().double().cpu().numpy(), b.double().numpy(), **param_tol,
                                   err_msg=f"param {i} shape {tuple(b.shape)}")
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
