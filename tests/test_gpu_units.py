"""GPU parity of the spectral route's unit entry points (include/cresso_hip.h,
"Unit operations") against the oracle's unit functions, called through the C
ABI on identical seeded inputs: hash metric and hash impulse (bins and counts
follow the reference's hash bit for bit; bin sums in fp64 in the oracle),
metric oscillator, confidence, contact oscillator and the drive update."""

import ctypes

import numpy as np
import pytest
import torch

import oracle.cresso_oracle as O
from gpu_util import F32_TOL, announce, check_low_precision_param, check_update, needs_gpu

pytestmark = [pytest.mark.gpu, needs_gpu]


def _lib():
    from cresso_amd import _native

    return _native, _native.load()


_KEEP = []   # device copies stay referenced until the test ends (a dropped
             # temporary's block could be handed to the next copy before the kernel runs)


def _dev(t):
    if t is None:
        return None
    d = t.cuda().contiguous()
    _KEEP.append(d)
    return d


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


@pytest.fixture(autouse=True)
def _release():
    yield
    torch.cuda.synchronize()
    _KEEP.clear()


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ws(lib, bins):
    nbytes = int(lib.cresso_unit_workspace_bytes(bins))
    buf = torch.empty(nbytes + 256, dtype=torch.uint8, device="cuda")
    off = (-buf.data_ptr()) % 256
    return buf, ctypes.c_void_p(buf.data_ptr() + off), ctypes.c_size_t(nbytes)


def _close(got, exp, what, tol=F32_TOL):
    np.testing.assert_allclose(got.double().cpu().numpy(), exp.double().numpy(), **tol, err_msg=what)


H = dict(O.DEFAULTS)


@pytest.mark.parametrize("shape,bins,salt,step", [((250, 200), 64, 0, 1), ((250, 200), 37, 1, 3),
                                                  ((3000,), 256, 2, 2), ((7, 9, 11), 4096, 0, 4)])
def test_hash_metric_update_log(shape, bins, salt, step):
    native, lib = _lib()
    announce(f"unit hash metric {shape} bins {bins} salt {salt} step {step}")
    gen = torch.Generator().manual_seed(41)
    n = int(np.prod(shape))
    rel = (torch.randn(shape, generator=gen).abs() * 3.0 + 1e-8).clamp(max=1e4)
    dsrc = rel.pow(1.2)
    energy0 = torch.rand(bins, generator=gen) * 2.0 + 0.1
    e_ref = energy0.clone()
    idx = O.hash_index(shape, bins, salt)
    term_ref = O.hash_metric_update_log(dsrc, e_ref, idx, bins, step, H, torch.float32, accum="fp64")
    e_gpu = energy0.cuda()
    out = torch.empty(n, device="cuda")
    buf, ws, nb = _ws(lib, bins)
    native.check(lib.cresso_hash_metric_update_log(_ptr(_dev(dsrc)), n, _ptr(e_gpu), bins, salt, step,
                                                   H["hash_decay"], H["hash_metric_coupling"], H["energy_power"],
                                                   H["eps"], _ptr(out), ws, nb, _stream()), "hash metric")
    torch.cuda.synchronize()
    _close(e_gpu, e_ref, "hash_energy")
    _close(out, term_ref.reshape(-1), "log term")


@pytest.mark.parametrize("shape,bins,salt", [((250, 200), 64, 0), ((129, 77), 37, 3), ((50000,), 4096, 1)])
def test_hash_impulse_update_gather(shape, bins, salt):
    native, lib = _lib()
    announce(f"unit hash impulse {shape} bins {bins} salt {salt}")
    gen = torch.Generator().manual_seed(42)
    n = int(np.prod(shape))
    psrc = torch.randn(shape, generator=gen) * 0.7 + 0.05
    ref0 = torch.rand(bins, generator=gen) * 0.3
    imp0 = torch.randn(bins, generator=gen) * 0.1
    r_ref, i_ref = ref0.clone(), imp0.clone()
    idx = O.hash_index(shape, bins, salt)
    got_ref = O.hash_impulse_update_gather(psrc, r_ref, i_ref, idx, bins, H, torch.float32, accum="fp64")
    r_gpu, i_gpu = ref0.cuda(), imp0.cuda()
    out = torch.empty(n, device="cuda")
    buf, ws, nb = _ws(lib, bins)
    native.check(lib.cresso_hash_impulse_update_gather(_ptr(_dev(psrc)), n, _ptr(r_gpu), _ptr(i_gpu),
                                                       bins, salt, H["hash_decay"], H["hash_impulse_decay"],
                                                       H["refractory_gain"], _ptr(out), ws, nb, _stream()),
                 "hash impulse")
    torch.cuda.synchronize()
    _close(r_gpu, r_ref, "hash_refractory")
    _close(i_gpu, i_ref, "hash_impulse")
    _close(out, got_ref.reshape(-1), "retrieved")


@pytest.mark.parametrize("rank", [8, 16, 100, 4096])
def test_rank_level_updates(rank):
    native, lib = _lib()
    announce(f"unit rank updates rank {rank}")
    gen = torch.Generator().manual_seed(43)
    v = lambda s=1.0: (torch.randn(rank, generator=gen) * s)   # noqa: E731
    omega = torch.sqrt(1.0 + (torch.randint(0, 8, (rank,), generator=gen).float() ** 2))
    # metric oscillator, both banks
    mq_c, mq_s, mp_c, mp_s, port_c, port_s = v(0.5), v(0.5), v(0.2), v(0.2), v(0.3), v(0.3)
    ref = [t.clone() for t in (mq_c, mq_s, mp_c, mp_s)]
    O.metric_update(*ref, port_c, port_s, omega, H["metric_dt"], H["metric_friction"])
    gpu = [t.cuda() for t in (mq_c, mq_s, mp_c, mp_s)]
    native.check(lib.cresso_metric_update(*map(_ptr, gpu), _ptr(_dev(port_c)), _ptr(_dev(port_s)), _ptr(_dev(omega)),
                                          rank, H["metric_dt"], H["metric_friction"], _stream()), "metric")
    # confidence
    conf, pc, ps, qc, qs = v(1.0), v(0.3), v(0.3), v(0.5), v(0.5)
    conf_ref = conf.clone()
    O.confidence_update(conf_ref, pc, ps, qc, qs, H["confidence_decay"], H["eps"])
    conf_gpu = conf.cuda()
    native.check(lib.cresso_confidence_update(_ptr(conf_gpu), _ptr(_dev(pc)), _ptr(_dev(ps)), _ptr(_dev(qc)),
                                              _ptr(_dev(qs)), rank, H["confidence_decay"], H["eps"], _stream()),
                 "confidence")
    # contact: cos bank then sin bank with the shared action
    q, p, port, calcium = [v(0.4), v(0.4)], [v(0.2), v(0.2)], [v(0.3), v(0.3)], [v(0.1).abs(), v(0.1).abs()]
    action, surprise = torch.tensor(0.05), torch.tensor(0.7)
    rq, rp, rc, ra = [t.clone() for t in q], [t.clone() for t in p], [t.clone() for t in calcium], action.clone()
    for k in range(2):
        ra = O.contact_update_pair(rq[k], rp[k], port[k], omega, rc[k], ra, surprise, H)
    gq, gp, gc, ga = [t.cuda() for t in q], [t.cuda() for t in p], [t.cuda() for t in calcium], action.cuda()
    gs = surprise.cuda()
    for k in range(2):
        native.check(lib.cresso_contact_update_pair(
            _ptr(gq[k]), _ptr(gp[k]), _ptr(_dev(port[k])), _ptr(_dev(omega)), _ptr(gc[k]), _ptr(ga), _ptr(gs), rank,
            H["dt"], H["refractory_decay"], H["refractory_gain"], H["surprise_gain"], H["surprise_brake"],
            H["impulse_friction"], H["contact_gain"], H["restoring"], H["cubic"], _stream()), "contact")
    torch.cuda.synchronize()
    for name, a, b in zip(("metric_cos", "metric_sin", "metric_p_cos", "metric_p_sin"), gpu, ref):
        _close(a, b, name)
    _close(conf_gpu, conf_ref, "mode_confidence")
    for k in range(2):
        _close(gq[k], rq[k], f"q bank {k}")
        _close(gp[k], rp[k], f"p bank {k}")
        _close(gc[k], rc[k], f"calcium bank {k}")
    _close(ga, ra, "action")


@pytest.mark.parametrize("dtype,hard,echo,hashp,step", [
    (torch.float32, True, True, True, 1), (torch.float32, True, True, True, 4), (torch.float32, False, False, False, 2),
    (torch.float32, True, False, True, 12), (torch.bfloat16, True, True, True, 3), (torch.float16, True, True, False, 2)])
def test_drive_update(dtype, hard, echo, hashp, step):
    native, lib = _lib()
    announce(f"unit drive {dtype} hard {hard} echo {echo} hash {hashp} step {step}")
    gen = torch.Generator().manual_seed(44)
    shape = (300, 211)
    n = shape[0] * shape[1]
    p0 = (0.02 * torch.randn(shape, generator=gen)).to(dtype)
    t = torch.randn(shape, generator=gen) * 1.5
    t[0, :5] = torch.tensor([0.0, 40.0, -40.0, 1e-6, 1e4])   # zero, beyond clip^2, tiny, clamp bound
    pred = 0.3 * torch.randn(shape, generator=gen)
    err = t - pred
    echo_f = torch.randn(shape, generator=gen) * 0.4 if echo else None
    hp = torch.randn(shape, generator=gen) * 0.05 if hashp else None
    surprise = torch.tensor(0.6)
    de0 = torch.tensor(1.7)
    # a hard tensor has an echo field unless echo_mix is 0 (cresso_v5.py:1262-1265)
    kw = dict(lr=2e-3) if (echo or not hard) else dict(lr=2e-3, echo_mix=0.0)
    po = p0.clone()
    st = {"surprise": surprise.clone(), "drive_energy": de0.clone()}
    opt = O.OracleCRESSO5([po], **kw)
    opt._drive_apply(po, st, t, pred, err, echo_f, hp if hp is not None else 0.0, hard, step, torch.float32, True)
    pg = p0.cuda()
    de_g = de0.cuda()
    hyper = native.hyper_from_group(dict(opt.h))
    buf, ws, nb = _ws(lib, 1)
    rc = lib.cresso_drive_update(_ptr(pg), native.DTYPE_CODE[dtype], _ptr(_dev(t)), _ptr(_dev(pred)),
                                 _ptr(_dev(err)), _ptr(_dev(echo_f)),
                                 _ptr(_dev(hp)), _ptr(_dev(surprise)), _ptr(de_g), n, step,
                                 1 if hard else 0, ctypes.byref(hyper), ws, nb, _stream())
    native.check(rc, "drive update")
    torch.cuda.synchronize()
    _close(de_g, st["drive_energy"], "drive_energy")
    got, exp, before = pg.double().cpu().numpy(), po.double().numpy(), p0.double().numpy()
    if dtype == torch.float32:
        np.testing.assert_allclose(got, exp, **F32_TOL, err_msg="param")
        check_update(got - before, exp - before, 1e-4, "param update")
    else:
        check_low_precision_param(got, exp, dtype, "param", before, before)


def test_unit_ops_reject_bad_arguments():
    native, lib = _lib()
    buf, ws, nb = _ws(lib, 64)
    x = torch.zeros(16, device="cuda")
    e = torch.zeros(64, device="cuda")
    assert lib.cresso_hash_metric_update_log(_ptr(x), 16, _ptr(e), 5000, 0, 1, 0.9, 0.4, 1.2, 1e-8, _ptr(x), ws, nb,
                                             _stream()) == -1
    assert b"bins" in lib.cresso_hip_last_error()
    assert lib.cresso_hash_metric_update_log(_ptr(x), 16, _ptr(e), 64, 0, 1, 0.9, 0.4, 1.2, 1e-8, _ptr(x), ws,
                                             ctypes.c_size_t(16), _stream()) == -1
    assert b"workspace" in lib.cresso_hip_last_error()
    assert lib.cresso_metric_update(*([_ptr(x)] * 7), 0, 0.1, 0.2, _stream()) == -1
    assert b"rank" in lib.cresso_hip_last_error()


@pytest.mark.parametrize("shape,bins,salt,scale", [((250, 200), 64, 0, 1.0), ((129, 77), 37, 3, 1.0),
                                                   ((50000,), 4096, 1, 1.0), ((3000,), 64, 0, 1e-25),
                                                   ((3000,), 64, 1, 0.0)])
def test_hash_reduce_mean(shape, bins, salt, scale):
    """Bin means (hash_reduce_mean_cuda, cu:1222-1253) against the oracle's fp64
    scatter-add; also all-zero and ~1e-25 inputs (the fixed-point scale is
    capped so x * scale stays finite and exact zeros stay zero)."""
    native, lib = _lib()
    announce(f"unit hash reduce mean {shape} bins {bins} salt {salt} scale {scale}")
    gen = torch.Generator().manual_seed(44)
    n = int(np.prod(shape))
    x = (torch.randn(shape, generator=gen) * 0.7 + 0.05) * scale
    idx = O.hash_index(shape, bins, salt)
    ref = O.hash_reduce_mean(x.reshape(-1), idx.reshape(-1), bins, accum="fp64")
    out = torch.full((bins,), float("nan"), device="cuda")
    buf, ws, nb = _ws(lib, bins)
    native.check(lib.cresso_hash_reduce_mean(_ptr(_dev(x)), n, bins, salt, _ptr(out), ws, nb, _stream()),
                 "hash reduce mean")
    torch.cuda.synchronize()
    got = out.double().cpu().numpy()
    assert np.isfinite(got).all()
    # relative tolerance only: the values may be ~1e-25
    np.testing.assert_allclose(got, ref.double().numpy(), rtol=1e-5, atol=1e-6 * scale, err_msg="bin means")


@pytest.mark.parametrize("scale", [0.0, 1e-25])
def test_hash_impulse_zero_and_tiny_sources(scale):
    native, lib = _lib()
    announce(f"unit hash impulse with port source scale {scale}")
    gen = torch.Generator().manual_seed(45)
    shape, bins, salt = (4000,), 64, 1
    n = shape[0]
    psrc = torch.randn(shape, generator=gen) * scale
    ref0 = torch.rand(bins, generator=gen) * 0.3 * max(scale, 1e-30)
    imp0 = torch.randn(bins, generator=gen) * 0.1 * max(scale, 1e-30)
    r_ref, i_ref = ref0.clone(), imp0.clone()
    idx = O.hash_index(shape, bins, salt)
    got_ref = O.hash_impulse_update_gather(psrc, r_ref, i_ref, idx, bins, H, torch.float32, accum="fp64")
    r_gpu, i_gpu = ref0.cuda(), imp0.cuda()
    out = torch.empty(n, device="cuda")
    buf, ws, nb = _ws(lib, bins)
    native.check(lib.cresso_hash_impulse_update_gather(_ptr(_dev(psrc)), n, _ptr(r_gpu), _ptr(i_gpu), bins, salt,
                                                       H["hash_decay"], H["hash_impulse_decay"],
                                                       H["refractory_gain"], _ptr(out), ws, nb, _stream()),
                 "hash impulse")
    torch.cuda.synchronize()
    tol = dict(rtol=1e-5, atol=1e-6 * scale)
    for got, exp, what in ((r_gpu, r_ref, "hash_refractory"), (i_gpu, i_ref, "hash_impulse"),
                           (out, got_ref.reshape(-1), "retrieved")):
        g = got.double().cpu().numpy()
        assert np.isfinite(g).all(), what
        np.testing.assert_allclose(g, exp.double().numpy(), **tol, err_msg=what)


@pytest.mark.parametrize("bins,salt", [(64, 0), (37, 2), (5000, 1)])
def test_hash_gather(bins, salt):
    """hash_gather_cuda (cu:1255-1276): out[i] = values[bin(i)], exact."""
    native, lib = _lib()
    announce(f"unit hash gather bins {bins} salt {salt}")
    gen = torch.Generator().manual_seed(46)
    shape = (123, 457)
    n = int(np.prod(shape))
    vals = torch.randn(bins, generator=gen)
    idx = O.hash_index(shape, bins, salt).reshape(-1)
    out = torch.empty(n, device="cuda")
    native.check(lib.cresso_hash_gather(_ptr(_dev(vals)), bins, n, salt, _ptr(out), _stream()), "hash gather")
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), vals[idx])


@pytest.mark.parametrize("shape,power,coupling,lo,hi", [((300, 257), 1.0, 0.55, 1e-3, 5.0),
                                                        ((64, 4096), 1.7, 0.55, 1e-9, 2e4),
                                                        ((5000, 3), 0.1, 1.3, 0.0, 3.0),
                                                        ((17, 19), 1.0, 0.0, 0.0, 1.0),
                                                        ((1, 1), 1.0, 0.55, 0.5, 0.5)])
def test_instant_axis_metric_2d(shape, power, coupling, lo, hi):
    """instant_axis_metric_2d_cuda (cu:1766-1827) against the oracle's
    instant_axis_metric (cresso_v5.py:243-262), fp32 tolerance; densities
    clamped at 1e6 and power below the 0.25 floor included."""
    native, lib = _lib()
    announce(f"unit instant axis metric 2d {shape} power {power} coupling {coupling}")
    gen = torch.Generator().manual_seed(47)
    rel = lo + (hi - lo) * torch.rand(shape, generator=gen) ** 3
    ref = O.instant_axis_metric(rel, power, coupling, H["eps"])
    rows, cols = shape
    nbytes = int(lib.cresso_instant_axis_metric_2d_workspace_bytes(rows, cols))
    buf = torch.empty(nbytes + 256, dtype=torch.uint8, device="cuda")
    ws = ctypes.c_void_p(buf.data_ptr() + (-buf.data_ptr()) % 256)
    out = torch.full(shape, float("nan"), device="cuda")
    native.check(lib.cresso_instant_axis_metric_2d(_ptr(_dev(rel)), rows, cols, power, coupling, H["eps"], _ptr(out),
                                                   ws, nbytes, _stream()), "instant axis metric")
    torch.cuda.synchronize()
    _close(out, ref, "instant axis metric")
