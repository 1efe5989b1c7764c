"""cresso_spectral_step_batched (several same-plan tensors in every launch,
blockIdx.y = tensor) against cresso_spectral_step of each tensor, through the
C ABI: identical inputs must give bit-identical params and states, on the
matrix-core route and the general one, for every dtype pair kind, with
tensors at different step counts, for a batch smaller than the workspace's
capacity, and for a full batch after it (the unused lanes must not have been
disturbed).  Then the optimizer with batching against the optimizer without."""

import ctypes

import pytest
import torch

from gpu_util import announce, needs_gpu

pytestmark = [pytest.mark.gpu, needs_gpu]

# (name, shape, param dtype, grad dtype, optimizer kwargs)
CASES = [
    ("fast_f32", (640, 512), torch.float32, torch.float32, dict(rank=8, max_frequency=5, hash_bins=64, hash_tables=2)),
    ("fast_bf16", (384, 320), torch.bfloat16, torch.bfloat16, dict(rank=8, max_frequency=5, hash_bins=64, hash_tables=2)),
    ("fast_f32_bf16grad", (256, 768), torch.float32, torch.bfloat16,
     dict(rank=4, max_frequency=3, hash_bins=128, hash_tables=2)),
    ("general_r16_t4", (300, 260), torch.float32, torch.float32,
     dict(rank=16, max_frequency=5, hash_bins=256, hash_tables=4)),
    # rank above 16: the general sweeps instantiated for 32 modes (MODE 1 tiles)
    ("general_r24", (512, 512), torch.float32, torch.float32,
     dict(rank=24, max_frequency=6, hash_bins=64, hash_tables=2)),
    # matrix-core route whose histogram merge adds row groups with atomics into
    # eight histogram copies per lane (1024 bins x 512 or more block partials)
    ("merge_r16_t4", (4096, 2048), torch.float32, torch.float32,
     dict(rank=16, max_frequency=7, hash_bins=256, hash_tables=4)),
    ("general_fp16_3d", (24, 20, 36), torch.float16, torch.float16,
     dict(rank=8, max_frequency=5, hash_bins=64, hash_tables=2)),
    ("one_d", (5000,), torch.float32, torch.float32, dict(rank=8, max_frequency=5, hash_bins=64, hash_tables=2)),
    ("no_hash", (512, 256), torch.float32, torch.float32, dict(rank=8, max_frequency=5, hash_bins=0, hash_tables=2)),
    ("soft_only", (256, 256), torch.float32, torch.float32,
     dict(rank=8, max_frequency=5, hash_bins=64, hash_tables=2, hard_channel_min_size=1 << 30)),
    # rank 8, two tables: 32 tensors of C4's (2048,2048) shape are 8192 blocks,
    # a multi-round batch whose histograms merge with atomics into the eight
    # copies, while each single step is one round (partial-row merge)
    ("multiround_r8_t2", (2048, 2048), torch.float32, torch.float32,
     dict(rank=8, max_frequency=5, hash_bins=64, hash_tables=2), 32),
]

COUNT = 5


class _Side:
    def __init__(self, p0: torch.Tensor, dtype, kw):
        import cresso_amd

        self.p = torch.nn.Parameter(p0.clone().to("cuda", dtype))
        self.opt = cresso_amd.CRESSO5([self.p], cuda_ops="required", lr=2e-3, **kw)
        self.group = self.opt.param_groups[0]
        self.st = self.opt._init_spectral(self.p, self.group)

    def snapshot(self):
        out = {"param": self.p.detach().clone()}
        for k, v in self.st.items():
            out[k] = v.clone() if torch.is_tensor(v) else v
        return out


def _assert_same(a: dict, b: dict, what: str) -> None:
    assert set(a) == set(b), what
    for k in a:
        if torch.is_tensor(a[k]):
            assert a[k].dtype == b[k].dtype and a[k].shape == b[k].shape, (what, k)
            assert torch.equal(a[k], b[k]), f"{what}: {k} differs (max |diff| " \
                f"{(a[k].double() - b[k].double()).abs().max().item():.3e})"
        else:
            assert a[k] == b[k], (what, k)


def _single(engine, side: _Side, grad: torch.Tensor) -> None:
    from cresso_amd import _native

    key, rank, d = engine._prepare(side.p, grad, side.st, side.group)
    ws = engine._workspace(key, 0, rank, side.group)
    hyper = _native.hyper_from_group(side.group)
    rc = engine.lib.cresso_spectral_step(ws.plan, ctypes.byref(d), ctypes.c_void_p(ws.buf.data_ptr()),
                                         ctypes.c_size_t(ws.buf.numel()), ctypes.byref(hyper),
                                         ctypes.c_void_p(_native.stream_handle(side.p.device)))
    _native.check(rc, "single step")
    side.st["step"] += 1


def _batched(engine, sides, grads, capacity: int) -> None:
    from cresso_amd import _native

    prep = [engine._prepare(s.p, g, s.st, s.group) for s, g in zip(sides, grads)]
    key, rank, _ = prep[0]
    ws = engine._workspace(key, 0, rank, sides[0].group, count=capacity)
    assert ws.count == capacity
    arr = (_native.SpectralDesc * len(prep))(*[d for _, _, d in prep])
    hyper = _native.hyper_from_group(sides[0].group)
    rc = engine.lib.cresso_spectral_step_batched(ws.plan, arr, len(prep), ctypes.c_void_p(ws.buf.data_ptr()),
                                                 ctypes.c_size_t(ws.buf.numel()), ctypes.byref(hyper),
                                                 ctypes.c_void_p(_native.stream_handle(sides[0].p.device)))
    _native.check(rc, "batched step")
    for s in sides:
        s.st["step"] += 1


def _grad(shape, dtype, gen, scale):
    g = scale * torch.randn(shape, generator=gen)
    g = torch.where(torch.rand(shape, generator=gen) < 0.01, g * 50.0, g)
    return g.to("cuda", dtype)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_batched_matches_single(case):
    from cresso_amd.spectral import SpectralEngine

    name, shape, pdt, gdt, kw = case[:5]
    count = case[5] if len(case) > 5 else COUNT
    engine = SpectralEngine()
    gen = torch.Generator().manual_seed(sum(map(ord, name)) % 1000)
    p0 = [0.02 * torch.randn(shape, generator=gen) for _ in range(count)]
    ref = [_Side(p, pdt, kw) for p in p0]
    bat = [_Side(p, pdt, kw) for p in p0]
    scales = [10.0 ** (-4 + 0.5 * (i % COUNT)) for i in range(count)]
    # tensor i starts i % COUNT steps ahead: the batch holds tensors at different steps
    for i in range(count):
        for _ in range(i % COUNT):
            g = _grad(shape, gdt, gen, scales[i])
            _single(engine, ref[i], g)
            _single(engine, bat[i], g)
    full = list(range(count))
    plan = [full, full, [3, 0, 4], full]   # full, full, subset, full
    for it, sel in enumerate(plan):
        announce(f"batched {name} {shape} x {count} call {it} tensors {len(sel)}")
        gs = [_grad(shape, gdt, gen, scales[i]) for i in sel]
        for i, g in zip(sel, gs):
            _single(engine, ref[i], g)
        _batched(engine, [bat[i] for i in sel], gs, count)
        torch.cuda.synchronize()
        for i in range(count):
            _assert_same(ref[i].snapshot(), bat[i].snapshot(), f"{name} call {it} tensor {i}")


@pytest.mark.parametrize("shape", [(1024, 768), (300, 257)], ids=["matrix_cores", "general"])
def test_batched_matches_single_with_density_spikes(shape):
    """Energy power 4 and grads at the rel clamp after quiet steps: the density
    histograms take their high words (kept per tensor after its low-word
    copies).  A batch of four, two of them spiking at different positions,
    against single steps, bit for bit, on the spike step and the next."""
    from cresso_amd.spectral import SpectralEngine

    kw = dict(rank=8, max_frequency=5, hash_bins=64, hash_tables=2, energy_power=4.0)
    count = 4
    engine = SpectralEngine()
    gen = torch.Generator().manual_seed(71)
    p0 = [0.02 * torch.randn(shape, generator=gen) for _ in range(count)]
    ref = [_Side(p, torch.float32, kw) for p in p0]
    bat = [_Side(p, torch.float32, kw) for p in p0]
    full = list(range(count))
    for it in range(5):
        announce(f"batched spikes {shape} x {count} call {it}")
        gs = [(1e-3 * torch.randn(shape, generator=gen)).cuda() for _ in full]
        if it == 3:
            gs[1][17, 200] = 30.0
            gs[3][shape[0] - 5, 3] = -30.0
        for i in full:
            _single(engine, ref[i], gs[i])
        _batched(engine, [bat[i] for i in full], gs, count)
        torch.cuda.synchronize()
        for i in full:
            _assert_same(ref[i].snapshot(), bat[i].snapshot(), f"spikes {shape} call {it} tensor {i}")


def test_batched_rejects_mixed_batches():
    from cresso_amd import _native
    from cresso_amd.spectral import SpectralEngine

    engine = SpectralEngine()
    kw = CASES[0][4]
    shape = (256, 128)
    a = _Side(torch.zeros(shape), torch.float32, kw)
    b = _Side(torch.zeros(shape), torch.float32, kw)
    ga = torch.zeros(shape, device="cuda")
    prep = [engine._prepare(a.p, ga, a.st, a.group), engine._prepare(b.p, ga, b.st, b.group)]
    key, rank, _ = prep[0]
    ws = engine._workspace(key, 0, rank, a.group, count=2)
    hyper = _native.hyper_from_group(a.group)
    stream = ctypes.c_void_p(_native.stream_handle(a.p.device))
    lib = engine.lib

    def call(descs, count, nbytes=None):
        arr = (_native.SpectralDesc * len(descs))(*descs)
        return lib.cresso_spectral_step_batched(ws.plan, arr, count, ctypes.c_void_p(ws.buf.data_ptr()),
                                                ctypes.c_size_t(ws.buf.numel() if nbytes is None else nbytes),
                                                ctypes.byref(hyper), stream)

    d0, d1 = prep[0][2], prep[1][2]
    d1.hard = 0
    assert call([d0, d1], 2) == _native.CRESSO_E_INVALID
    d1.hard = d0.hard
    d1.grad_dtype = _native.DTYPE_CODE[torch.bfloat16]
    assert call([d0, d1], 2) == _native.CRESSO_E_INVALID
    d1.grad_dtype = d0.grad_dtype
    assert call([d0, d1], 3) == _native.CRESSO_E_INVALID         # workspace sized for 2
    assert call([d0, d1], 2, nbytes=1024) == _native.CRESSO_E_INVALID
    assert call([d0], 0) == _native.CRESSO_E_INVALID
    torch.cuda.synchronize()
    assert int(a.st["step"]) == 0 and int(b.st["step"]) == 0


def test_optimizer_batching_is_bit_identical():
    # the optimizer's multi-tensor step with batching (chunks forced small so
    # that one shape is cut into several batches over several lanes) against
    # the same step with every tensor on its own
    import cresso_amd
    from cresso_amd import spectral

    shapes = [(256, 256)] * 7 + [(512, 128)] * 3 + [(2048,)] + [(64, 48)] * 2 + [(300, 200)]
    kw = dict(rank=8, hash_bins=64, hash_tables=2)
    gen = torch.Generator().manual_seed(43)
    p0 = [0.02 * torch.randn(s, generator=gen) for s in shapes]
    gs = [[1e-3 * torch.randn(s, generator=gen) for s in shapes] for _ in range(3)]
    outs = []
    old = (spectral.SpectralEngine.BATCH, spectral.SpectralEngine.BATCH_BYTES)
    try:
        for batch, cap in ((False, old[1]), (True, old[1]), (True, 3 * spectral.lane_scratch_bytes(256 * 256))):
            announce(f"optimizer batching={batch} chunk bytes={cap}")
            spectral.SpectralEngine.BATCH = batch
            spectral.SpectralEngine.BATCH_BYTES = cap
            ps = [torch.nn.Parameter(p.clone().cuda()) for p in p0]
            opt = cresso_amd.CRESSO5(ps, cuda_ops="required", **kw)
            for step in gs:
                for p, g in zip(ps, step):
                    p.grad = g.cuda()
                opt.step()
            torch.cuda.synchronize()
            outs.append([p.detach().cpu() for p in ps] + [opt.state[p][k].cpu() for p in ps
                                                          for k in ("q_cos", "hash_energy", "drive_energy")])
    finally:
        spectral.SpectralEngine.BATCH, spectral.SpectralEngine.BATCH_BYTES = old
    for run in outs[1:]:
        for a, b in zip(outs[0], run):
            assert torch.equal(a, b)
