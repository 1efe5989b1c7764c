"""cresso_spectral_step_noalloc (workspace in the library's static device
array) against cresso_spectral_step (caller workspace) through the C ABI:
identical inputs must give bit-identical params and states, call after call,
also when consecutive calls switch to a smaller tensor (another plan) and back."""

import ctypes

import pytest
import torch

from gpu_util import announce, needs_gpu

pytestmark = [pytest.mark.gpu, needs_gpu]

KW = dict(lr=2e-3, rank=8, max_frequency=5, hash_bins=64, hash_tables=2)


class _Side:
    """One param with its spectral state, stepped through one entry point."""

    def __init__(self, p0: torch.Tensor):
        import cresso_amd

        self.p = torch.nn.Parameter(p0.clone().cuda())
        self.opt = cresso_amd.CRESSO5([self.p], cuda_ops="required", **KW)
        self.group = self.opt.param_groups[0]
        self.st = self.opt._init_spectral(self.p, self.group)

    def snapshot(self):
        out = {"param": self.p.detach().clone()}
        for k, v in self.st.items():
            out[k] = v.clone() if torch.is_tensor(v) else v
        return out


def _step(engine, side: _Side, grad: torch.Tensor, noalloc: bool) -> None:
    from cresso_amd import _native

    lib = engine.lib
    key, rank, d = engine._prepare(side.p, grad, side.st, side.group)
    ws = engine._workspace(key, 0, rank, side.group)   # the plan (and the caller workspace of the regular entry)
    hyper = _native.hyper_from_group(side.group)
    stream = ctypes.c_void_p(_native.stream_handle(side.p.device))
    if noalloc:
        rc = lib.cresso_spectral_step_noalloc(ws.plan, ctypes.byref(d), ctypes.byref(hyper), stream)
    else:
        rc = lib.cresso_spectral_step(ws.plan, ctypes.byref(d), ctypes.c_void_p(ws.buf.data_ptr()),
                                      ctypes.c_size_t(ws.buf.numel()), ctypes.byref(hyper), stream)
    _native.check(rc, "noalloc test step")
    side.st["step"] += 1


def _assert_same(a: dict, b: dict, what: str) -> None:
    assert set(a) == set(b), what
    for k in a:
        if torch.is_tensor(a[k]):
            assert a[k].dtype == b[k].dtype and a[k].shape == b[k].shape, (what, k)
            assert torch.equal(a[k], b[k]), f"{what}: {k} differs (max |diff| " \
                f"{(a[k].double() - b[k].double()).abs().max().item():.3e})"
        else:
            assert a[k] == b[k], (what, k)


def test_spectral_noalloc_matches_workspace_entry():
    from cresso_amd.spectral import SpectralEngine

    engine = SpectralEngine()
    gen = torch.Generator().manual_seed(21)
    big, small = (640, 512), (300, 200)   # the second call's tensor is smaller (another plan)
    sides = {}
    for shape in (big, small):
        p0 = 0.02 * torch.randn(shape, generator=gen)
        sides[shape] = (_Side(p0), _Side(p0))
    # big step 1, small step 1, big step 2, small step 2: every call switches plans
    for shape in (big, small, big, small):
        announce(f"noalloc spectral {shape}")
        g = 1e-3 * torch.randn(shape, generator=gen)
        g = torch.where(torch.rand(shape, generator=gen) < 0.01, g * 50.0, g).cuda()
        ref, na = sides[shape]
        _step(engine, ref, g, noalloc=False)
        _step(engine, na, g, noalloc=True)
        torch.cuda.synchronize()
        _assert_same(ref.snapshot(), na.snapshot(), f"shape {shape} step {ref.st['step']}")
    # the same plan twice in a row reuses the tables without a rebuild
    announce("noalloc spectral repeat")
    for _ in range(2):
        g = (1e-3 * torch.randn(small, generator=gen)).cuda()
        ref, na = sides[small]
        _step(engine, ref, g, noalloc=False)
        _step(engine, na, g, noalloc=True)
    torch.cuda.synchronize()
    _assert_same(ref.snapshot(), na.snapshot(), "repeat")


def test_spectral_noalloc_rejects_oversized_plan():
    from cresso_amd import _native
    from cresso_amd.modes import mode_list

    lib = _native.load()
    shape = (4096, 4096)   # ~100 MB of workspace at T = 2
    freqs = [f for m in mode_list(8, 2, 5) for f in m]
    plan = lib.cresso_spectral_plan_create((ctypes.c_int64 * 8)(*shape), 2, (ctypes.c_int64 * len(freqs))(*freqs),
                                           8, 64, 2)
    assert plan
    try:
        need = lib.cresso_spectral_workspace_bytes(ctypes.c_void_p(plan))
        assert need > _native.SPECTRAL_NOALLOC_MAX_BYTES
        d = _native.SpectralDesc()
        h = _native.Hyper()
        rc = lib.cresso_spectral_step_noalloc(ctypes.c_void_p(plan), ctypes.byref(d), ctypes.byref(h), None)
        assert rc == -1
        assert b"static scratch" in lib.cresso_hip_last_error()
    finally:
        lib.cresso_spectral_plan_destroy(ctypes.c_void_p(plan))


def _noalloc_call(engine, side: _Side, d, stream: int) -> int:
    from cresso_amd import _native

    key, rank, _ = engine._prepare(side.p, side.p.grad, side.st, side.group)
    ws = engine._workspace(key, 0, rank, side.group)
    hyper = _native.hyper_from_group(side.group)
    return engine.lib.cresso_spectral_step_noalloc(ws.plan, ctypes.byref(d), ctypes.byref(hyper),
                                                   ctypes.c_void_p(stream))


def test_spectral_noalloc_graph_capture_and_plan_switch():
    """With its plan's tables resident, a no-alloc call launches kernels only:
    captured into a graph and replayed three times (eager work and a
    synchronization between the replays), it matches three eager calls with
    the same descriptor bit for bit.  After a call with another plan, a call
    that would rebuild the tables is refused while the stream captures."""
    from cresso_amd import _native
    from cresso_amd.spectral import SpectralEngine

    engine = SpectralEngine()
    gen = torch.Generator().manual_seed(22)
    shape, other = (512, 384), (256, 320)
    p0 = 0.02 * torch.randn(shape, generator=gen)
    eager, graph = _Side(p0), _Side(p0)
    g = (1e-3 * torch.randn(shape, generator=gen)).cuda()
    eager.p.grad = g
    graph.p.grad = g
    # one uncaptured call per side makes the plan's tables resident
    for side in (eager, graph):
        _step(engine, side, g, noalloc=True)
    torch.cuda.synchronize()
    de = engine._prepare(eager.p, g, eager.st, eager.group)[2]
    dg = engine._prepare(graph.p, g, graph.st, graph.group)[2]
    announce("noalloc spectral: capture a resident-plan call")
    cap = torch.cuda.Stream()
    hg = torch.cuda.CUDAGraph()
    with torch.cuda.graph(hg, stream=cap):
        rc = _noalloc_call(engine, graph, dg, int(cap.cuda_stream))
    assert rc == 0, _native.load().cresso_hip_last_error()
    for k in range(3):
        announce(f"noalloc spectral: replay {k}")
        _native.check(_noalloc_call(engine, eager, de, _native.stream_handle(eager.p.device)), "eager no-alloc")
        hg.replay()
        torch.cuda.synchronize()
        x = torch.randn(1000, device="cuda").sum()   # eager work between replays
        torch.cuda.synchronize()
        assert torch.isfinite(x)
        _assert_same(eager.snapshot(), graph.snapshot(), f"replay {k}")
    # another plan's call rebuilds the static tables; a capture with the first plan is then refused
    announce("noalloc spectral: plan switch, then a capture that would rebuild")
    q0 = 0.02 * torch.randn(other, generator=gen)
    side_b = _Side(q0)
    _step(engine, side_b, (1e-3 * torch.randn(other, generator=gen)).cuda(), noalloc=True)
    torch.cuda.synchronize()
    hg2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(hg2, stream=cap):
        rc = _noalloc_call(engine, graph, dg, int(cap.cuda_stream))
    assert rc == _native.CRESSO_E_INVALID
    assert b"capturing" in _native.load().cresso_hip_last_error()
    del hg2
    torch.cuda.synchronize()
