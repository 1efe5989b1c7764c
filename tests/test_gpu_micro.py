"""GPU parity of the micro-field route (micro_field_max_size > 0,
cresso_v5.py:1355-1432) against the CPU oracle and the reference's golden
trajectory."""

import numpy as np
import pytest
import torch

from golden_inputs import trajectory
from gpu_util import BF16_PARAM_TOL, F32_TOL, announce, compare, needs_gpu, run_pair

pytestmark = [pytest.mark.gpu, needs_gpu]

MICRO_KW = dict(lr=2e-3, rank=4, micro_field_max_size=20000)


def test_micro_golden_trajectory():
    # the reference's own (12,10) fp32 micro trajectory, param and every state
    announce("micro golden micro_12x10_f32")
    import cresso_amd

    meta, p0, grads, steps, sidx = trajectory("micro_12x10_f32")
    p = torch.nn.Parameter(p0.clone().cuda())
    opt = cresso_amd.CRESSO5([p], cuda_ops="required", **meta["kwargs"])
    for k, g in enumerate(grads):
        p.grad = g.cuda()
        opt.step()
        torch.cuda.synchronize()
        exp = steps[k]
        got = p.detach().float().cpu()
        if "param" in exp:
            np.testing.assert_allclose(got.numpy(), exp["param"], **F32_TOL, err_msg=f"step {k} param")
        np.testing.assert_allclose(got.reshape(-1)[torch.from_numpy(sidx)].numpy(), exp["param_sample"], **F32_TOL)
        st = opt.state[p]
        for key, v in exp.items():
            if not key.startswith("state/"):
                continue
            sk = key[len("state/"):]
            if torch.is_tensor(st[sk]):
                np.testing.assert_allclose(st[sk].double().cpu().numpy(), v, **F32_TOL, err_msg=f"step {k} {sk}")
            else:
                assert st[sk] == int(v), (sk, st[sk], v)


# (12,10) and (64,64): axis sums in LDS; (2,5000): 5002 axis entries, beyond
# the LDS table, in the plan's global scratch; 1-D; 3-D; a single element
# (instant metric off)
@pytest.mark.parametrize("shape", [(12, 10), (64, 64), (2, 5000), (300,), (4, 5, 6), (1,), (3, 1, 7, 2)])
def test_micro_matches_oracle(shape):
    announce(f"micro {shape}")
    res = run_pair([shape], torch.float32, MICRO_KW, steps=4, seed=31)
    compare(*res)


def test_micro_mixed_group_with_scalar_and_spectral():
    # micro, scalar (resident and streaming) and spectral tensors in one group
    shapes = [(12, 10), (50,), (4096, 16), (16, 300), (256, 256), (2, 3, 4)]
    announce(f"micro mixed {shapes}")
    kw = dict(lr=2e-3, rank=4, hash_bins=64, hash_tables=2, micro_field_max_size=256)
    res = run_pair(shapes, torch.float32, kw, steps=3, seed=32)
    compare(*res)


def test_micro_options():
    # weight decay, maximize, no instant metric, energy power != 1, metric coupling off
    announce("micro options")
    kw = dict(MICRO_KW, weight_decay=0.02, maximize=True, warmup_steps=0, energy_power=1.5,
              instant_metric_power=0.7)
    compare(*run_pair([(12, 10), (40,), (3, 4, 5)], torch.float32, kw, steps=4, seed=33))
    kw = dict(MICRO_KW, instant_metric_coupling=0.0, hash_metric_coupling=0.0)
    compare(*run_pair([(12, 10), (40,)], torch.float32, kw, steps=3, seed=34))


def test_micro_grad_scales_and_zeros():
    # tiny and large gradient scales (rel clamps at eps and 1e4), exact zeros
    announce("micro scales")
    import cresso_amd
    from oracle.cresso_oracle import OracleCRESSO5

    gen = torch.Generator().manual_seed(35)
    shapes = [(16, 12), (200,)]
    p0 = [0.05 * torch.randn(s, generator=gen) for s in shapes]
    hp = [torch.nn.Parameter(p.clone().cuda()) for p in p0]
    op = [p.clone() for p in p0]
    hopt = cresso_amd.CRESSO5(hp, cuda_ops="required", **MICRO_KW)
    oopt = OracleCRESSO5(op, **MICRO_KW)
    for sc in (1e-9, 1.0, 1e3):
        step = []
        for s in shapes:
            g = sc * torch.randn(s, generator=gen)
            g[torch.rand(s, generator=gen) < 0.2] = 0.0
            step.append(g)
        for p, g in zip(hp, step):
            p.grad = g.cuda()
        hopt.step()
        oopt.step(step)
    torch.cuda.synchronize()
    compare(hp, hopt, op, oopt)


def test_micro_bf16_and_f64_params():
    announce("micro bf16")
    res = run_pair([(12, 10), (33,)], torch.bfloat16, MICRO_KW, steps=3, seed=36)
    compare(*res, param_tol=BF16_PARAM_TOL, state_tol=F32_TOL)
    announce("micro f64")
    res = run_pair([(12, 10), (2, 3, 4)], torch.float64, MICRO_KW, steps=3, seed=37)
    compare(*res, param_tol=dict(rtol=1e-9, atol=1e-12), state_tol=dict(rtol=1e-9, atol=1e-12))


def test_micro_state_dict_round_trip():
    # resume from a state_dict: the dense fields come back on the device
    announce("micro state_dict")
    import cresso_amd
    from oracle.cresso_oracle import OracleCRESSO5

    gen = torch.Generator().manual_seed(38)
    p0 = 0.05 * torch.randn(12, 10, generator=gen)
    grads = [1e-2 * torch.randn(12, 10, generator=gen) for _ in range(4)]
    hp = torch.nn.Parameter(p0.clone().cuda())
    hopt = cresso_amd.CRESSO5([hp], cuda_ops="required", **MICRO_KW)
    op = p0.clone()
    oopt = OracleCRESSO5([op], **MICRO_KW)
    for g in grads[:2]:
        hp.grad = g.cuda()
        hopt.step()
        oopt.step([g])
    sd = hopt.state_dict()
    hp2 = torch.nn.Parameter(hp.detach().clone())
    hopt2 = cresso_amd.CRESSO5([hp2], cuda_ops="required", **MICRO_KW)
    hopt2.load_state_dict(sd)
    assert list(hopt2.state[hp2].keys()) == ["step", "force_rms", "drive_energy", "surprise", "action",
                                             "micro_energy", "micro_impulse", "micro_refractory"]
    for g in grads[2:]:
        hp2.grad = g.cuda()
        hopt2.step()
        oopt.step([g])
    torch.cuda.synchronize()
    compare([hp2], hopt2, [op], oopt)
