"""The reference's own fp16 and fp64 trajectories (tests/golden/
trajectories_f16_f64.npz, written by running cresso_v5.py with
cuda_ops="off") stepped on the HIP path: spectral, scalar and micro routes.

fp64 params compute in fp64 on every route (the reference's work dtype for
them, cresso_v5.py:119-124): params and every state tensor within rtol 1e-9.
fp16 params: fp32 state within the fp32 tolerance, the param within one ulp
of the fp16 value plus one ulp of the rounded update (check_low_precision_param).
"""

import numpy as np
import pytest
import torch

from golden_inputs import trajectory, trajectory_names
from gpu_util import F32_TOL, announce, check_low_precision_param, needs_gpu

pytestmark = [pytest.mark.gpu, needs_gpu]

FILE = "trajectories_f16_f64"
F64_TOL = dict(rtol=1e-9, atol=1e-12)


@pytest.mark.parametrize("name", trajectory_names(FILE))
def test_reference_trajectory_on_gpu(name):
    import cresso_amd

    meta, p0, grads, steps, sidx = trajectory(name, FILE)
    announce(f"golden {name} {tuple(meta['shape'])} {meta['dtype']}")
    p = torch.nn.Parameter(p0.clone().cuda())
    opt = cresso_amd.CRESSO5([p], cuda_ops="required", **meta["kwargs"])
    f64 = meta["dtype"] == "float64"
    idx = torch.from_numpy(sidx).cuda()
    prev_exp = p0.double().reshape(-1)[torch.from_numpy(sidx)].numpy()
    for k, g in enumerate(grads):
        before = p.detach().reshape(-1)[idx].double().cpu().numpy()
        p.grad = g.cuda()
        opt.step()
        torch.cuda.synchronize()
        exp = steps[k]
        got = p.detach().reshape(-1)[idx].double().cpu().numpy()
        what = f"{name} step {k + 1}"
        if f64:
            np.testing.assert_allclose(got, exp["param_sample"], **F64_TOL, err_msg=f"{what} param")
            if "param" in exp:
                np.testing.assert_allclose(p.detach().double().cpu().numpy(), exp["param"], **F64_TOL,
                                           err_msg=f"{what} dense param")
        else:
            check_low_precision_param(got, exp["param_sample"].astype(np.float64), p.dtype, what, prev_exp, before)
        prev_exp = exp["param_sample"].astype(np.float64)
        st = opt.state[p]
        for key, v in exp.items():
            if not key.startswith("state/"):
                continue
            sk = key[len("state/"):]
            val = st[sk]
            if not torch.is_tensor(val):
                assert int(val) == int(v), (what, sk)
                continue
            if not val.is_floating_point():
                np.testing.assert_array_equal(val.cpu().numpy(), v, err_msg=f"{what} {sk}")
                continue
            if f64:
                assert val.dtype == torch.float64, (what, sk, val.dtype)
            np.testing.assert_allclose(val.double().cpu().numpy(), v.astype(np.float64),
                                       **(F64_TOL if f64 else F32_TOL), err_msg=f"{what} state {sk}")
