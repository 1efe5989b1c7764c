"""CPU tests of the drop-in contract: constructor validation, routing, state
layout and size, checkpoint dtype repair, failure semantics, C-ABI exports."""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

import cresso_amd
from cresso_amd import CRESSO5, count_optimizer_state_elements, theoretical_state_elements
from cresso_amd import _native
from oracle import cresso_oracle as O

ROOT = Path(__file__).resolve().parents[1]


def test_modes_match_oracle_restatement():
    from cresso_amd.modes import hash_unit, mode_list, omega_tensor, freqs_tensor
    for args in [(8, 2, 5), (16, 2, 7), (16, 4, 7), (16, 3, 7), (8, 1, 5), (4, 2, 0), (40, 2, 2), (30, 1, 5), (0, 2, 5)]:
        assert mode_list(*args) == O.frequency_pack(*args)
        fr = freqs_tensor(*args, device="cpu")
        assert torch.equal(fr, O.make_freqs(*args))
        assert torch.equal(omega_tensor(fr), O.omega_from_freqs(fr))
    # omega is the correctly rounded fp32 square root (numpy's is IEEE): the
    # fp64 route widens this value, so one ulp would show at fp64 precision.
    fr = freqs_tensor(32, 2, 6, device="cpu").numpy().astype(np.float64)
    exact = np.sqrt(1.0 + (fr * fr).sum(axis=1)).astype(np.float32)
    assert np.array_equal(omega_tensor(torch.from_numpy(fr)).numpy(), exact)
    for n in range(20):
        for s in (0, 17, 101, 151, 170):
            assert hash_unit(n, s) == O.hash_unit(n, s)


@pytest.mark.parametrize("kw,msg", [
    (dict(lr=-1.0), "lr must be >= 0.0"),
    (dict(dt=1.5), "dt must be <= 1.0"),
    (dict(eps=float("nan")), "eps must be a finite scalar"),
    (dict(rank=-1), "rank must be non-negative"),
    (dict(hash_tables=0), "hash_tables must be >= 1"),
    (dict(min_spectral_size=0), "min_spectral_size must be >= 1"),
    (dict(thin_matrix_route="dense"), "thin_matrix_route must be one of"),
    (dict(cuda_ops="sometimes"), "cuda_ops must be one of"),
    (dict(min_gain=2.0, max_gain=1.0), "min_gain must be <= max_gain"),
    (dict(drive_clip=0.01), "drive_clip must be >= 0.1"),
    (dict(thin_matrix_min_aspect=0.5), "thin_matrix_min_aspect must be >= 1.0"),
    (dict(warmup_steps=-2), "warmup_steps must be non-negative"),
])
def test_constructor_validation_messages(kw, msg):
    p = torch.nn.Parameter(torch.zeros(4))
    with pytest.raises(ValueError, match=re.escape(msg)):
        CRESSO5([p], **kw)


def test_defaults_and_cuda_ops_normalization():
    p = torch.nn.Parameter(torch.zeros(4))
    g = CRESSO5([p]).param_groups[0]
    assert g["lr"] == 2e-3 and g["rank"] == 8 and g["hash_bins"] == 128 and g["cuda_ops"] == "auto"
    assert CRESSO5([p], cuda_ops=False).param_groups[0]["cuda_ops"] == "off"
    assert CRESSO5([p], cuda_ops=True).param_groups[0]["cuda_ops"] == "auto"
    assert cresso_amd.CRESSO is CRESSO5


@pytest.mark.parametrize("shape,route", [
    ((128, 16), "scalar"), ((4096, 16), "scalar"), ((16, 4096), "scalar"), ((4096, 4096), "spectral"),
    ((2048,), "spectral"), ((1000,), "scalar"), ((40, 30), "spectral"), ((200, 6), "scalar"), ((), "scalar"),
    ((512, 256, 3, 3), "spectral"), ((100, 20), "scalar"), ((64, 65), "spectral"),
])
def test_routing_matches_oracle(shape, route):
    p = torch.nn.Parameter(torch.zeros(shape))
    opt = CRESSO5([p])
    assert opt._route(p, opt.param_groups[0]) == route
    assert O.OracleCRESSO5([p]).route(p) == route


def test_thin_spectral_override_and_state_counts():
    for route, expect in (("scalar", 8), ("spectral", theoretical_state_elements((128, 16), rank=4, thin_matrix_route="spectral"))):
        p = torch.nn.Parameter(torch.zeros(128, 16))
        opt = CRESSO5([p], rank=4, thin_matrix_route=route)
        g = opt.param_groups[0]
        st = opt._init_spectral(p, g) if opt._route(p, g) == "spectral" else opt._init_scalar(p)
        assert count_optimizer_state_elements(opt) == expect
        assert ("q_cos" in st) == (route == "spectral")


def test_theoretical_state_elements_matches_oracle():
    for shape in [(128, 16), (4096, 4096), (2048,), (512, 256, 3, 3), (200, 6), (12, 10)]:
        for kw in [dict(), dict(thin_matrix_route="spectral"), dict(hash_bins=64, hash_tables=3),
                   dict(micro_field_max_size=256), dict(hard_channel_min_size=10**9)]:
            assert theoretical_state_elements(shape, 8, **kw) == O.theoretical_state_elements(shape, 8, **kw)


def test_spectral_state_layout_matches_oracle():
    p = torch.nn.Parameter(torch.zeros(64, 48))
    opt = CRESSO5([p], hash_bins=64, hash_tables=2)
    st = opt._init_spectral(p, opt.param_groups[0])
    orc = O.OracleCRESSO5([p.detach()], hash_bins=64, hash_tables=2)
    ost = {}
    orc._init_spectral(p.detach(), ost, torch.float32)
    assert list(st.keys()) == list(ost.keys())
    for k, v in ost.items():
        if torch.is_tensor(v):
            assert st[k].dtype == v.dtype and torch.equal(st[k], v), k
    assert count_optimizer_state_elements(opt) == theoretical_state_elements((64, 48), 8, hash_bins=64)


def test_load_state_dict_keeps_int_freqs_and_fp32_state_for_bf16_params():
    p = torch.nn.Parameter(torch.zeros(64, 48, dtype=torch.bfloat16))
    opt = CRESSO5([p], hash_bins=64)
    st = opt._init_spectral(p, opt.param_groups[0])
    st["q_cos"].fill_(0.123456789)
    st["step"] = 7
    sd = opt.state_dict()
    p2 = torch.nn.Parameter(torch.zeros(64, 48, dtype=torch.bfloat16))
    opt2 = CRESSO5([p2], hash_bins=64)
    opt2.load_state_dict(sd)
    st2 = opt2.state[p2]
    assert st2["freqs"].dtype == torch.long and torch.equal(st2["freqs"], st["freqs"])
    assert st2["q_cos"].dtype == torch.float32 and torch.equal(st2["q_cos"], st["q_cos"])
    assert st2["step"] == 7


def test_required_rejects_cpu_params():
    p = torch.nn.Parameter(torch.ones(4, 4))
    p.grad = torch.ones_like(p)
    opt = CRESSO5([p], cuda_ops="required", min_spectral_size=1)
    with pytest.raises(RuntimeError, match="cuda_ops='required'.*CUDA parameter"):
        opt.step()


def test_auto_and_off_do_not_silently_fall_back_to_cpu():
    for mode in ("auto", "off"):
        p = torch.nn.Parameter(torch.ones(4, 4))
        p.grad = torch.ones_like(p)
        with pytest.raises(RuntimeError):
            CRESSO5([p], cuda_ops=mode).step()


def test_sparse_grad_rejected():
    p = torch.nn.Parameter(torch.ones(4, 4))
    p.grad = torch.ones(4, 4).to_sparse()
    with pytest.raises(RuntimeError, match="does not support sparse gradients"):
        CRESSO5([p]).step()


def test_params_without_grad_are_skipped():
    p = torch.nn.Parameter(torch.ones(4, 4))
    opt = CRESSO5([p], cuda_ops="required")
    opt.step()
    assert len(opt.state) == 0


def test_library_loads_and_exports_every_declared_symbol():
    lib_path = ROOT / "cresso_amd" / "libcresso_hip.so"
    if not lib_path.exists():
        pytest.skip("library not built (python -m cresso_amd.build)")
    header = (ROOT / "include" / "cresso_hip.h").read_text()
    declared = set(re.findall(r"^\s*(?:[\w\*]+\s+)+\**(cresso_\w+)\s*\(", header, flags=re.M))
    assert {"cresso_hip_abi_version", "cresso_hip_last_error", "cresso_scalar_plan_step"} <= declared
    lib = ctypes.CDLL(str(lib_path))
    for name in sorted(declared):
        assert hasattr(lib, name), name
    lib = _native.load()
    assert lib.cresso_hip_abi_version() == _native.ABI_VERSION


def test_plan_creation_rejects_bad_descriptors_without_gpu():
    lib_path = ROOT / "cresso_amd" / "libcresso_hip.so"
    if not lib_path.exists():
        pytest.skip("library not built")
    lib = _native.load()
    d = (_native.ScalarDesc * 1)()
    d[0].ndim = 2
    d[0].shape[0], d[0].shape[1] = 4, 4
    d[0].numel = 15  # inconsistent with the shape
    h = _native.Hyper()
    h.drive_clip = 4.0
    assert not lib.cresso_scalar_plan_create(d, 1, ctypes.byref(h))
    assert b"numel" in lib.cresso_hip_last_error()


def test_unit_drive_update_rejects_dtype_before_any_launch():
    # an unsupported param dtype is refused by the host checks, so the call
    # returns before touching the (here fake) device pointers or any GPU
    lib_path = ROOT / "cresso_amd" / "libcresso_hip.so"
    if not lib_path.exists():
        pytest.skip("library not built")
    lib = _native.load()
    fake = ctypes.c_void_p(1 << 20)
    h = _native.Hyper()
    h.drive_clip = 4.0
    rc = lib.cresso_drive_update(fake, _native.DTYPE_CODE[torch.float64], fake, fake, fake, None, None, fake, fake,
                                 16, 1, 1, ctypes.byref(h), fake, 1 << 20, None)
    assert rc == _native.CRESSO_E_UNSUPPORTED
    assert b"not supported" in lib.cresso_hip_last_error()


def test_hash_c_oracle_matches_numpy_oracle():
    so = ROOT / "oracle" / "_build" / "libcresso_hash_oracle.so"
    if not so.exists():
        pytest.skip("oracle C restatement not built (make -C oracle)")
    import numpy as np
    lib = ctypes.CDLL(str(so))
    lib.cresso_oracle_hash_bins.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
    lib.cresso_oracle_hash_counts.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
    for n, bins, salt in [(5000, 64, 0), (5000, 37, 3), (100003, 256, 1), (777, 7, 9)]:
        out = np.empty(n, dtype=np.int32)
        lib.cresso_oracle_hash_bins(n, bins, salt, out.ctypes.data)
        np.testing.assert_array_equal(out, O.hash_index_np(n, bins, salt).astype(np.int32))
        cnt = np.empty(bins, dtype=np.int64)
        lib.cresso_oracle_hash_counts(n, bins, salt, cnt.ctypes.data)
        np.testing.assert_array_equal(cnt, np.bincount(out, minlength=bins))


def test_hash_bigint_brute_force_on_small_n():
    # Textbook restatement with Python big ints: wrap to signed 64 bits after
    # every step, arithmetic shift on the signed value, floor-mod.
    def wrap(v):
        v &= (1 << 64) - 1
        return v - (1 << 64) if v >> 63 else v

    for salt in (0, 1, 5):
        s = salt + 1
        for bins in (64, 37):
            got = O.hash_index_np(300, bins, salt)
            for i in range(300):
                h = wrap(i * (1103515245 + 97 * s) + (12345 + 0x9E3779B1 * s))
                h = wrap(h ^ (h >> 16))
                h = wrap(h * (2246822519 + 1315423911 * s))
                h = wrap(h ^ (h >> 13))
                h = wrap(h * (3266489917 + 374761393 * s))
                h = wrap(h ^ (h >> 16))
                assert got[i] == h % bins


def test_host_batch_guard_cpu_behaviour():
    # the C++ steady-state helper is built with the library; on CPU tensors it
    # refuses the fast path, and bump() advances every state["step"]
    import ctypes

    hb = _native.host_batch()
    assert hb is not None, "cresso_amd/_hostbatch extension not built"
    ps = [torch.nn.Parameter(torch.zeros(4, 4)) for _ in range(3)]
    for p in ps:
        p.grad = torch.zeros(4, 4)
    guard = hb.BatchGuard(ps)
    buf = (ctypes.c_void_p * 3)()
    assert guard.gather(ps, ctypes.addressof(buf)) is False      # CPU grads: no fast path
    assert guard.gather(ps[:2], ctypes.addressof(buf)) is False  # different group
    states = [{"step": 0}, {"step": 7}, {"step": 2}]
    guard.bump(states)
    assert [s["step"] for s in states] == [1, 8, 3]
    ps[0].grad = None
    with pytest.raises(ValueError):
        hb.BatchGuard(ps)


def test_host_batch_guard_holds_references_and_refuses_replaced_params():
    # The guard keeps each planned parameter alive (so no new object can take
    # its address) and refuses the fast path once a parameter object is replaced.
    import ctypes
    import gc
    import weakref

    hb = _native.host_batch()
    assert hb is not None, "cresso_amd/_hostbatch extension not built"
    ps = [torch.nn.Parameter(torch.zeros(4, 4)) for _ in range(3)]
    for p in ps:
        p.grad = torch.zeros(4, 4)
    guard = hb.BatchGuard(ps)
    ref = weakref.ref(ps[1])
    old = ps[1]
    ps[1] = torch.nn.Parameter(torch.zeros(4, 4))
    ps[1].grad = torch.zeros(4, 4)
    del old
    gc.collect()
    assert ref() is not None          # still referenced by the guard
    buf = (ctypes.c_void_p * 3)()
    assert guard.gather(ps, ctypes.addressof(buf)) is False
    del guard
    gc.collect()
    assert ref() is None              # released with the guard


def test_spectral_lane_assignment():
    # the multi-tensor spectral step: m tensors of one shape use min(4, m)
    # distinct lanes (one workspace each), shapes spread over the lanes
    from cresso_amd.spectral import assign_lanes

    keys = ["a"] * 6 + ["b"] + ["c"] * 2 + ["d"]
    lanes = assign_lanes(keys, 4)
    assert len(lanes) == len(keys) and all(0 <= x < 4 for x in lanes)
    by = {}
    for k, x in zip(keys, lanes):
        by.setdefault(k, []).append(x)
    assert len(set(by["a"])) == 4 and len(set(by["c"])) == 2
    assert by["a"][:4] == [0, 1, 2, 3] and by["a"][4:] == [0, 1]   # round robin
    assert by["b"] == [1] and by["c"] == [2, 3] and by["d"] == [3]  # start lane moves with each new key
    assert assign_lanes(["x", "y"], 1) == [0, 0]
    assert assign_lanes([], 4) == []


def test_spectral_batch_units_and_chunks():
    # the multi-tensor spectral step's units: same plan, dtypes, hard channel
    # and hash state batch together; a batch holds at most BATCH_BYTES of
    # per-tensor scratch, larger groups are cut into near-equal chunks
    from cresso_amd import _native
    from cresso_amd.spectral import SpectralEngine, lane_scratch_bytes

    eng = SpectralEngine.__new__(SpectralEngine)   # no library needed for the grouping
    eng.BATCH, eng.BATCH_BYTES = True, 3 * lane_scratch_bytes(100)

    def desc(numel, hard=1, hash_on=True, pdt=_native.F32):
        d = _native.SpectralDesc()
        d.numel, d.hard, d.param_dtype, d.grad_dtype = numel, hard, pdt, pdt
        d.hash_energy = 4096 if hash_on else None
        return d

    prepared = [("a", 8, desc(100)) for _ in range(7)] + [("b", 8, desc(50))] + [("a", 8, desc(100, hard=0))] \
        + [("a", 8, desc(100, pdt=_native.BF16))] + [("c", 8, desc(10)), ("c", 8, desc(10, hash_on=False))]
    sts = [{"i": i} for i in range(len(prepared))]
    units = eng._units(prepared, sts)
    got = [(u[0], [s["i"] for s in u[4]]) for u in units]
    # seven "a" tensors at three per batch: chunks of 3, 3, 1 (ceil(7 / ceil(7/3)) = 3)
    assert got[:3] == [(("a", True, 3), [0, 1, 2]), (("a", True, 3), [3, 4, 5]), (("a", True, 3), [6])]
    assert [g[1] for g in got[3:]] == [[7], [8], [9], [10], [11]]
    assert all(not u[0][1] for u in units[3:])
    eng.BATCH = False
    assert [len(u[4]) for u in eng._units(prepared, sts)] == [1] * len(prepared)


def test_load_state_dict_keeps_same_plan_workspaces():
    """A spectral workspace depends only on its plan key (shape, freqs,
    hash_bins, hash_tables, work dtype): load_state_dict keeps those the
    loaded state still uses and frees the rest (no GPU needed: the workspaces
    here are stand-in objects in the engine's table)."""
    lib_path = ROOT / "cresso_amd" / "libcresso_hip.so"
    if not lib_path.exists():
        pytest.skip("library not built")
    from cresso_amd.spectral import SpectralEngine

    p = torch.nn.Parameter(torch.zeros(64, 48))
    q = torch.nn.Parameter(torch.zeros(32, 40))
    opt = CRESSO5([p, q], cuda_ops="required", rank=8, hash_bins=64, hash_tables=2)
    group = opt.param_groups[0]
    for t in (p, q):
        opt.state[t] = opt._init_spectral(t, group)
    eng = SpectralEngine()
    opt._spectral_engine = eng
    kp = eng.plan_key(p, opt.state[p], group)
    kq = eng.plan_key(q, opt.state[q], group)
    stale = (kp[0], (7, 7)) + kp[2:]
    keep_p, keep_q, drop = object(), object(), object()
    eng.ws = {(kp, False, 0): keep_p, (kq, True, 2): keep_q, (stale, False, 1): drop}
    sd = opt.state_dict()
    opt.load_state_dict(sd)
    assert eng.ws == {(kp, False, 0): keep_p, (kq, True, 2): keep_q}
    # a loaded state with other freqs for p no longer uses p's plan
    sd2 = opt.state_dict()
    sd2["state"][0]["freqs"] = sd2["state"][0]["freqs"].flip(0).clone()
    opt.load_state_dict(sd2)
    assert set(eng.ws) == {(kq, True, 2)}


def test_spectral_plan_rank_limits_without_gpu():
    # plan creation is host work: ranks up to 32 plan on the fp32 and fp64
    # work dtypes (ranks above 16 take the general sweeps); a refusal carries
    # the library's message instead of a fallback
    lib_path = ROOT / "cresso_amd" / "libcresso_hip.so"
    if not lib_path.exists():
        pytest.skip("library not built")
    from cresso_amd.modes import mode_list

    lib = _native.load()
    shape = (1024, 512)

    def create(rank, work):
        freqs = [f for m in mode_list(rank, 2, 7) for f in m]
        return lib.cresso_spectral_plan_create_ex((ctypes.c_int64 * 8)(*shape), 2,
                                                  (ctypes.c_int64 * len(freqs))(*freqs), rank, 64, 2, work)

    for rank in (17, 24, 32):
        plan = create(rank, _native.F32)
        assert plan, lib.cresso_hip_last_error()
        assert lib.cresso_spectral_workspace_bytes(ctypes.c_void_p(plan)) > 0
        lib.cresso_spectral_plan_destroy(ctypes.c_void_p(plan))
    plan = create(24, _native.F64)
    assert plan, lib.cresso_hip_last_error()
    lib.cresso_spectral_plan_destroy(ctypes.c_void_p(plan))
    assert not create(33, _native.F32)
    assert b"rank 33" in lib.cresso_hip_last_error()
