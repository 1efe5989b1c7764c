"""GPU parity of the scalar (LoRA-thin / small tensor) route against the CPU oracle."""

import pytest
import torch

from gpu_util import BF16_PARAM_TOL, F32_TOL, announce, compare, needs_gpu, run_pair

pytestmark = [pytest.mark.gpu, needs_gpu]

SCALAR_KW = dict(lr=2e-3, rank=4, hash_bins=64, hash_tables=2)


# (4096,16), (16,4096), (1024,64): every thread holds 16 float4 slots (the fast
# resident kernel); (1024,16), (2048,8), (8,4096): the fast kernel with 4, 4
# and 8 slots; (128,16), (64,16), (256,4): the general resident kernel
@pytest.mark.parametrize("shape", [(4096, 16), (16, 4096), (128, 16), (16, 300), (64, 16), (1024, 64), (256, 4),
                                   (1024, 16), (2048, 8), (8, 4096)])
def test_scalar_2d_matches_oracle(shape):
    announce(f"scalar 2d {shape}")
    res = run_pair([shape], torch.float32, SCALAR_KW, steps=4, seed=1)
    compare(*res)


# 2-D tensors beyond the resident limit, row/column axis sums.  More than 64 Ki
# elements, or 16 Ki when a plan has fewer than 256 such tensors: the wide form
# (chunks over the whole GPU); otherwise one workgroup per tensor.  (8192,64) and (64,8192): one row per wave; (8192,16): rows in groups
# of 16 lanes; (16,8192): a wave inside one row; (1000,60), (3000,33) and
# (5000,33): neither, per-element row and column sums
@pytest.mark.parametrize("shape", [(8192, 16), (16, 8192), (8192, 64), (64, 8192), (1000, 60), (3000, 33), (5000, 33)])
def test_scalar_streaming_2d_matches_oracle(shape):
    announce(f"scalar streaming 2d {shape}")
    res = run_pair([shape], torch.float32, SCALAR_KW, steps=3, seed=3)
    compare(*res)


def test_scalar_streaming_2d_options_and_dtypes():
    announce("scalar streaming 2d options")
    kw = dict(SCALAR_KW, maximize=True, weight_decay=0.01, instant_metric_power=0.7, local_sharpness=0.3)
    compare(*run_pair([(8192, 16), (2000, 48)], torch.float32, kw, steps=3, seed=4))
    # a coupling this strong can push a product of axis factors past fp32's
    # range, so the factors are kept as logs (summed, then one exp)
    announce("scalar streaming 2d strong coupling")
    kw = dict(SCALAR_KW, instant_metric_coupling=6.0)
    compare(*run_pair([(8192, 16), (3000, 33), (16, 8192), (64, 48, 50)], torch.float32, kw, steps=3, seed=13))
    announce("scalar streaming 2d bf16 / f64")
    res = run_pair([(8192, 16), (40, 1000)], torch.bfloat16, SCALAR_KW, steps=3, seed=5)
    compare(*res, param_tol=BF16_PARAM_TOL, state_tol=F32_TOL)
    # f64 params are never resident: (256,32), (16,512) and (512,16) take the
    # one-workgroup kernel's wave, lane-group and per-thread column sums; the
    # others the wide form
    res = run_pair([(8192, 16), (40, 1000), (1024, 64), (256, 32), (16, 512), (512, 16)], torch.float64, SCALAR_KW,
                   steps=3, seed=6)
    compare(*res, param_tol=dict(rtol=1e-9, atol=1e-12), state_tol=dict(rtol=1e-9, atol=1e-12))


def test_scalar_wide_form_1d_and_3d():
    # large 1-D (instant metric from the element's own density) and 3-D
    # (per-axis sums) tensors in the wide form, next to a resident tensor
    announce("scalar wide 1d / 3d")
    shapes = [(300000,), (64, 48, 50), (4096, 16), (2, 70000)]
    compare(*run_pair(shapes, torch.float32, dict(SCALAR_KW, weight_decay=0.01), steps=3, seed=12))


def test_scalar_wide_form_no_instant_metric_and_bf16_grads():
    # instant_metric_coupling = 0 (no axis sums) in the wide form; then bf16
    # grads on fp32 params (never resident), wide and one-workgroup tensors
    import cresso_amd
    from oracle.cresso_oracle import OracleCRESSO5
    import numpy as np

    announce("scalar wide no instant metric")
    kw = dict(SCALAR_KW, instant_metric_coupling=0.0)
    compare(*run_pair([(8192, 16), (16, 8192), (3000, 33)], torch.float32, kw, steps=3, seed=14))

    announce("scalar wide bf16 grads on fp32 params")
    gen = torch.Generator().manual_seed(15)
    shapes = [(8192, 16), (16, 8192), (120, 30)]
    p0 = [0.02 * torch.randn(s, generator=gen) for s in shapes]
    gs = [[(1e-2 * torch.randn(s, generator=gen)).to(torch.bfloat16) for s in shapes] for _ in range(3)]
    hp = [torch.nn.Parameter(p.clone().cuda()) for p in p0]
    for p in hp:
        p.grad_dtype = None   # allow grads of another dtype
    op = [p.clone() for p in p0]
    hopt = cresso_amd.CRESSO5(hp, cuda_ops="required", **SCALAR_KW)
    oopt = OracleCRESSO5(op, **SCALAR_KW)
    for step in gs:
        for p, g in zip(hp, step):
            p.grad = g.cuda()
        hopt.step()
        oopt.step(step)
    torch.cuda.synchronize()
    compare(hp, hopt, op, oopt)


def test_scalar_mixed_batch_one_launch_per_variant():
    # resident row-group, resident column-block, streaming 1D / 3D / 0-d /
    # odd 2D / large thin 2D, all in one optimizer group
    shapes = [(4096, 16), (16, 4096), (100,), (4, 5, 6), (), (33, 7), (7, 1000), (32768, 16), (8, 8)]
    announce(f"scalar mixed {shapes}")
    res = run_pair(shapes, torch.float32, dict(SCALAR_KW, weight_decay=0.01), steps=3, seed=2)
    compare(*res)


def test_scalar_options_maximize_local_sharpness_no_warmup():
    announce("scalar options")
    kw = dict(SCALAR_KW, maximize=True, local_sharpness=0.3, warmup_steps=0, instant_metric_power=1.5)
    res = run_pair([(4096, 16), (16, 4096), (300,)], torch.float32, kw, steps=3, seed=3)
    compare(*res)


def test_scalar_maximize_fast_kernel():
    # maximize alone keeps the fast resident kernel (the force is -grad)
    announce("scalar maximize fast")
    kw = dict(SCALAR_KW, maximize=True, warmup_steps=0)
    res = run_pair([(4096, 16), (16, 4096), (1024, 16)], torch.float32, kw, steps=3, seed=10)
    compare(*res)


def test_scalar_exact_zero_gradients():
    # rows and single entries of exactly zero grad: t == 0 there, where the
    # root channel sign(t) sqrt(min(|t|, clip^2) + eps) is 0, not sqrt(eps)
    announce("scalar exact zeros")
    import cresso_amd
    from oracle.cresso_oracle import OracleCRESSO5
    import numpy as np

    gen = torch.Generator().manual_seed(11)
    shapes = [(4096, 16), (16, 4096), (128, 16)]
    p0 = [0.05 * torch.randn(s, generator=gen) for s in shapes]
    gs = []
    for _ in range(3):
        step = []
        for s in shapes:
            g = 1e-2 * torch.randn(s, generator=gen)
            g[::3] = 0.0
            g[torch.rand(s, generator=gen) < 0.2] = 0.0
            step.append(g)
        gs.append(step)
    hp = [torch.nn.Parameter(p.clone().cuda()) for p in p0]
    op = [p.clone() for p in p0]
    hopt = cresso_amd.CRESSO5(hp, cuda_ops="required", **SCALAR_KW)
    oopt = OracleCRESSO5(op, **SCALAR_KW)
    for step in gs:
        for p, g in zip(hp, step):
            p.grad = g.cuda()
        hopt.step()
        oopt.step(step)
    torch.cuda.synchronize()
    compare(hp, hopt, op, oopt)


def test_scalar_tiny_gradients_eps_dominated():
    # sigma ~ 1e-6: the eps inside sqrt(mean f^2 + eps) dominates the force RMS
    announce("scalar tiny grads")
    res = run_pair([(4096, 16), (16, 4096)], torch.float32, SCALAR_KW, steps=3, seed=4, grad_std=1e-6)
    compare(*res)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_scalar_half_params(dtype):
    announce(f"scalar {dtype}")
    res = run_pair([(64, 16), (4096, 16), (16, 4096), (100,)], dtype, dict(SCALAR_KW, lr=1e-3), steps=2, seed=5,
                   grad_std=0.05)
    compare(*res, param_tol=BF16_PARAM_TOL, state_tol=F32_TOL)


def test_scalar_lora_mix_long_trajectory():
    # C3-like: alternating (4096,16)/(16,4096) with log-uniform per-tensor scales, 10 steps
    announce("scalar lora 10 steps")
    gen = torch.Generator().manual_seed(6)
    scales = (10.0 ** (torch.rand(8, generator=gen) * 3.0 - 4.0)).tolist()
    shapes = [(4096, 16) if i % 2 == 0 else (16, 4096) for i in range(8)]
    res = run_pair(shapes, torch.float32, SCALAR_KW, steps=10, seed=7, grad_scales=scales)
    compare(*res)


def test_scalar_deterministic_and_state_identity():
    import cresso_amd

    announce("scalar determinism")
    # resident, one-workgroup streaming and wide-form tensors
    shapes = [(4096, 16) if i % 2 == 0 else (16, 4096) for i in range(64)] + [(33, 7), (5, 6, 7), (8192, 16),
                                                                              (16, 8192), (3000, 33)]
    gen = torch.Generator().manual_seed(8)
    p0 = [0.02 * torch.randn(s, generator=gen) for s in shapes]
    g = [1e-3 * torch.randn(s, generator=gen) for s in shapes]
    outs = []
    for _ in range(2):
        ps = [torch.nn.Parameter(p.clone().cuda()) for p in p0]
        opt = cresso_amd.CRESSO5(ps, cuda_ops="required", **SCALAR_KW)
        ids = None
        for _ in range(3):
            for p, gg in zip(ps, g):
                p.grad = gg.cuda()
            opt.step()
            cur = [id(opt.state[p]["q"]) for p in ps]
            assert ids is None or cur == ids  # state tensors are updated in place
            ids = cur
        torch.cuda.synchronize()
        outs.append(([p.detach().cpu() for p in ps], [{k: v.cpu() if torch.is_tensor(v) else v
                                                        for k, v in opt.state[p].items()} for p in ps]))
    for a, b in zip(outs[0][0], outs[1][0]):
        assert torch.equal(a, b)
    for a, b in zip(outs[0][1], outs[1][1]):
        for k in a:
            assert (torch.equal(a[k], b[k]) if torch.is_tensor(a[k]) else a[k] == b[k]), k


def test_scalar_state_dict_roundtrip_resumes_identically():
    import cresso_amd

    announce("scalar state_dict")
    gen = torch.Generator().manual_seed(9)
    shapes = [(4096, 16), (64, 16)]
    p0 = [(0.02 * torch.randn(s, generator=gen)).to(torch.bfloat16) for s in shapes]
    gs = [[(1e-2 * torch.randn(s, generator=gen)).to(torch.bfloat16) for s in shapes] for _ in range(4)]
    ps = [torch.nn.Parameter(p.clone().cuda()) for p in p0]
    opt = cresso_amd.CRESSO5(ps, cuda_ops="required", **SCALAR_KW)
    for k in range(2):
        for p, g in zip(ps, gs[k]):
            p.grad = g.cuda()
        opt.step()
    sd = opt.state_dict()
    ps2 = [torch.nn.Parameter(p.detach().clone()) for p in ps]
    opt2 = cresso_amd.CRESSO5(ps2, cuda_ops="required", **SCALAR_KW)
    opt2.load_state_dict(sd)
    for p in ps2:
        assert opt2.state[p]["q"].dtype == torch.float32  # not cast to bf16 by torch's loader
        assert opt2.state[p]["step"] == 2
    for k in range(2, 4):
        for p, p2, g in zip(ps, ps2, gs[k]):
            p.grad = g.cuda()
            p2.grad = g.cuda()
        opt.step()
        opt2.step()
    torch.cuda.synchronize()
    for a, b in zip(ps, ps2):
        assert torch.equal(a, b)


def test_scalar_steady_state_replans_on_changes():
    # the steady-state path (C++ guard) must notice a grad dtype change, a
    # replaced parameter storage and a hyperparameter change, and re-plan
    announce("scalar steady-state changes")
    import cresso_amd
    from oracle.cresso_oracle import OracleCRESSO5

    gen = torch.Generator().manual_seed(12)
    shapes = [(4096, 16), (16, 4096), (128, 16)]
    p0 = [0.02 * torch.randn(s, generator=gen) for s in shapes]
    hp = [torch.nn.Parameter(p.clone().cuda()) for p in p0]
    for p in hp:
        p.grad_dtype = None   # allow grads of another dtype
    op = [p.clone() for p in p0]
    hopt = cresso_amd.CRESSO5(hp, cuda_ops="required", **SCALAR_KW)
    oopt = OracleCRESSO5(op, **SCALAR_KW)
    for k in range(6):
        gs = [1e-2 * torch.randn(s, generator=gen) for s in shapes]
        if k == 2:      # bf16 grads on fp32 params
            gs = [g.to(torch.bfloat16) for g in gs]
        if k == 3:      # new storage for one parameter (same values)
            hp[1].data = hp[1].data.clone()
        if k == 4:      # learning-rate change
            for grp in hopt.param_groups:
                grp["lr"] = 1e-3
            oopt.h["lr"] = 1e-3
        for p, g in zip(hp, gs):
            p.grad = g.cuda()
        hopt.step()
        oopt.step(gs)
    torch.cuda.synchronize()
    compare(hp, hopt, op, oopt)


def test_scalar_plan_step_null_grads_reuse_the_previous_pointers():
    # C ABI: grads == NULL reuses the previous call's grad pointers, here the
    # staged ones of a step whose grads differ from the plan's upload
    import ctypes

    import cresso_amd
    from cresso_amd import _native
    from oracle.cresso_oracle import OracleCRESSO5

    announce("scalar plan step with NULL grads")
    gen = torch.Generator().manual_seed(16)
    shapes = [(4096, 16), (16, 4096), (33, 7)]
    p0 = [0.02 * torch.randn(s, generator=gen) for s in shapes]
    g1 = [1e-2 * torch.randn(s, generator=gen) for s in shapes]
    g2 = [1e-2 * torch.randn(s, generator=gen) for s in shapes]
    hp = [torch.nn.Parameter(p.clone().cuda()) for p in p0]
    op = [p.clone() for p in p0]
    hopt = cresso_amd.CRESSO5(hp, cuda_ops="required", **SCALAR_KW)
    oopt = OracleCRESSO5(op, **SCALAR_KW)
    for gs in (g1, g2):
        for p, g in zip(hp, gs):
            p.grad = g.cuda()
        hopt.step()
        oopt.step(gs)
    batch = next(b for k, b in hopt._batches.items() if k[1] == "scalar")
    hyper = _native.hyper_from_group(hopt.param_groups[0])
    rc = batch.lib.cresso_scalar_plan_step(batch.plan, ctypes.c_void_p(batch.table.data_ptr()), None,
                                           ctypes.byref(hyper), ctypes.c_void_p(_native.stream_handle(hp[0].device)))
    _native.check(rc, "scalar plan step (NULL grads)")
    for st in batch.states:
        st["step"] += 1
    oopt.step(g2)
    torch.cuda.synchronize()
    compare(hp, hopt, op, oopt)


@pytest.mark.parametrize("extra", [{}, dict(micro_field_max_size=64)], ids=["scalar_route", "micro_route"])
def test_empty_parameters_follow_the_reference(extra):
    """Parameters with no elements beside ordinary ones: nothing to update, and
    the state entries the reference computes as means over no elements are
    NaN (compare treats NaN as equal to NaN); the ordinary tensors step as
    usual.  (min_spectral_size >= 1, so an empty parameter never takes the
    spectral route.)"""
    import cresso_amd
    from oracle.cresso_oracle import OracleCRESSO5

    announce(f"empty parameters {extra}")
    gen = torch.Generator().manual_seed(37)
    shapes = [(0, 8), (128, 96), (0,), (4096, 16)]
    kw = dict(rank=8, hash_bins=64, hash_tables=2, **extra)
    p0 = [0.02 * torch.randn(s, generator=gen) for s in shapes]
    hp = [torch.nn.Parameter(p.clone().cuda()) for p in p0]
    op = [p.clone() for p in p0]
    hopt = cresso_amd.CRESSO5(hp, cuda_ops="required", **kw)
    oopt = OracleCRESSO5(op, **kw)
    for k in range(3):
        gs = [1e-3 * torch.randn(s, generator=gen) for s in shapes]
        for p, g in zip(hp, gs):
            p.grad = g.cuda()
        hopt.step()
        oopt.step(gs)
    torch.cuda.synchronize()
    compare(hp, hopt, op, oopt)


def test_non_contiguous_grads_follow_the_reference():
    """Grads in a transposed layout (the parameter's shape, other strides) on
    the scalar and spectral routes are read in the parameter's element order
    (through a contiguous copy); contiguous grads before and after take the
    steady-state path."""
    import cresso_amd
    from oracle.cresso_oracle import OracleCRESSO5

    announce("non-contiguous grads")
    gen = torch.Generator().manual_seed(41)
    shapes = [(4096, 16), (16, 4096), (128, 96)]
    kw = dict(rank=8, hash_bins=64, hash_tables=2)
    p0 = [0.02 * torch.randn(s, generator=gen) for s in shapes]
    hp = [torch.nn.Parameter(p.clone().cuda()) for p in p0]
    op = [p.clone() for p in p0]
    hopt = cresso_amd.CRESSO5(hp, cuda_ops="required", **kw)
    oopt = OracleCRESSO5(op, **kw)
    for k in range(5):
        gs = [1e-3 * torch.randn(s, generator=gen) for s in shapes]
        for p, g in zip(hp, gs):
            gd = g.cuda()
            if k in (1, 2):
                gd = gd.t().contiguous().t()   # same values, column-major strides
                assert not gd.is_contiguous()
            p.grad = gd
        hopt.step()
        oopt.step(gs)
    torch.cuda.synchronize()
    compare(hp, hopt, op, oopt)


def test_non_contiguous_params_follow_the_reference():
    """Parameters in other layouts (a channels-last convolution weight and a
    transposed matrix on the spectral route, a transposed LoRA-thin matrix on
    the scalar route) step in their logical element order and keep their
    layout; values and state follow the oracle on contiguous copies."""
    import cresso_amd
    from oracle.cresso_oracle import OracleCRESSO5

    announce("non-contiguous params")
    gen = torch.Generator().manual_seed(43)
    shapes = [(64, 32, 3, 3), (96, 128), (4096, 16)]
    kw = dict(rank=8, hash_bins=64, hash_tables=2)
    p0 = [0.02 * torch.randn(s, generator=gen) for s in shapes]
    dev = [p0[0].cuda().contiguous(memory_format=torch.channels_last),
           p0[1].t().contiguous().cuda().t(),
           p0[2].t().contiguous().cuda().t()]
    hp = [torch.nn.Parameter(d) for d in dev]
    assert not any(p.is_contiguous() for p in hp)
    strides = [p.stride() for p in hp]
    op = [p.clone() for p in p0]
    hopt = cresso_amd.CRESSO5(hp, cuda_ops="required", **kw)
    oopt = OracleCRESSO5(op, **kw)
    for k in range(3):
        gs = [1e-3 * torch.randn(s, generator=gen) for s in shapes]
        for p, g in zip(hp, gs):
            p.grad = g.cuda()
        hopt.step()
        oopt.step(gs)
    torch.cuda.synchronize()
    assert [p.stride() for p in hp] == strides
    compare(hp, hopt, op, oopt)
