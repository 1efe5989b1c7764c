"""Host orchestration of the spectral/hash route.

The library keeps no state of its own: plans live here, keyed by
(device, shape, freqs, hash_bins, hash_tables), together with their device
workspace (carrier tables, cached coordinate-hash bins, scratch).

A step of several spectral tensors (`step_many`) first batches the tensors
that share a plan (and dtypes, hard channel and hash state): one batched C
call steps a batch, every launch covering all its tensors, with the plan's
tables held once and per-step scratch (about 4 bytes per element plus a few
KB) once per tensor.  A batch holds at most BATCH_BYTES of such scratch;
larger groups are cut into that many chunks.  The units of work (batches and
single tensors) are spread over up to LANES side streams (default priority),
so that one unit's small finish kernels and partly filled sweeps overlap
with another's work.  Every lane has its own workspace per unit kind: units
that share a workspace run one after another on that lane's stream, so its
per-step scratch is never used concurrently.  The side streams wait for the
caller's stream before the first launch and the caller's stream waits for
all of them after the last, so the step is ordered like any other work on
the caller's stream.  A single spectral tensor runs on the caller's stream
directly.

Device memory held: per (plan, lane) a workspace of the plan's tables (about
(2 + 4) bytes per element at two tables of <= 256 bins) and its scratch;
the optimizer's load_state_dict keeps those whose plan the loaded state still
uses (`retain`) and frees the others; `reset()` frees them all.
"""

from __future__ import annotations

import ctypes
from typing import Dict, List, Sequence, Tuple

import torch

from . import _native

# (param dtype, grad dtype) pairs of the library's spectral step; the force is
# the grad converted to the work dtype, as in cresso_v5.py:907-912: fp32 for
# fp32/bf16/fp16 params, fp64 for fp64 params, whose state is fp64 too and
# whose plans carry the fp64 work dtype (cresso_v5.py:119-124).
_DTYPE_PAIRS = {(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
                (torch.float32, torch.bfloat16), (torch.float32, torch.float16), (torch.float64, torch.float64)}

_VEC_KEYS = ("q_cos", "q_sin", "p_cos", "p_sin", "metric_cos", "metric_sin", "metric_p_cos", "metric_p_sin",
             "calcium_cos", "calcium_sin", "mode_confidence")


def assign_lanes(keys: Sequence[tuple], lanes: int) -> List[int]:
    """Lane of each tensor of a multi-tensor step, given its plan key.

    The m tensors of one key take min(lanes, m) distinct lanes, round robin
    from a start lane that moves on with every new key (so single tensors of
    different shapes spread over the lanes).  Each (key, lane) pair is one
    workspace, used by its tensors one after another on that lane's stream.
    """
    count: Dict[tuple, int] = {}
    for k in keys:
        count[k] = count.get(k, 0) + 1
    seen: Dict[tuple, int] = {}
    base: Dict[tuple, int] = {}
    out = []
    for k in keys:
        if k not in base:
            base[k] = len(base) % lanes
        j = seen.get(k, 0)
        seen[k] = j + 1
        out.append((base[k] + j % min(lanes, count[k])) % lanes)
    return out


class _Workspace:
    """A plan with its device workspace: for one tensor (count=None) or for
    batches of up to `count` tensors."""

    def __init__(self, lib, shape, freqs_host: Tuple[int, ...], rank: int, bins: int, tables: int, group: dict,
                 device: torch.device, count=None, work: int = _native.F32):
        self.lib = lib
        self.count = count
        nd = len(shape)
        shp = (ctypes.c_int64 * 8)(*shape)
        fr = (ctypes.c_int64 * max(1, len(freqs_host)))(*freqs_host)
        plan = lib.cresso_spectral_plan_create_ex(shp, nd, fr, rank, bins, tables, work)
        if not plan:
            _native.check(-1, "spectral route plan")
        self.plan = ctypes.c_void_p(plan)
        hyper = _native.hyper_from_group(group)
        stream = ctypes.c_void_p(_native.stream_handle(device))
        if count is None:
            nbytes = int(lib.cresso_spectral_workspace_bytes(self.plan))
            self.buf = torch.empty(nbytes, dtype=torch.uint8, device=device)
            rc = lib.cresso_spectral_workspace_init(self.plan, ctypes.c_void_p(self.buf.data_ptr()),
                                                    ctypes.c_size_t(nbytes), ctypes.byref(hyper), stream)
        else:
            nbytes = int(lib.cresso_spectral_batched_workspace_bytes(self.plan, count))
            self.buf = torch.empty(nbytes, dtype=torch.uint8, device=device)
            rc = lib.cresso_spectral_batched_workspace_init(self.plan, count, ctypes.c_void_p(self.buf.data_ptr()),
                                                            ctypes.c_size_t(nbytes), ctypes.byref(hyper), stream)
        _native.check(rc, "spectral workspace init")

    def __del__(self):
        plan = getattr(self, "plan", None)
        if plan is not None and plan.value:
            try:
                self.lib.cresso_spectral_plan_destroy(plan)
            except Exception:
                pass


def lane_scratch_bytes(numel: int) -> int:
    """Per-tensor scratch of a batched step, for sizing chunks: the tangent
    field (4 bytes per element) dominates; the rest is a few KB per tensor
    plus small per-row and per-column sums."""
    return 4 * numel + (1 << 16)


class SpectralEngine:
    READY = True
    LANES = 4                 # side streams of a multi-tensor step
    BATCH = True              # batch same-plan tensors into one launch per kernel
    BATCH_BYTES = 512 << 20   # per-tensor scratch held by one batch (C4: 3 % faster than 256 MiB, as fast as 1 GiB)

    def __init__(self):
        self.lib = _native.load()
        self.ws: Dict[tuple, _Workspace] = {}   # (plan key, unit kind, lane) -> workspace
        self.side: Dict[torch.device, List[torch.cuda.Stream]] = {}
        self.freq_cache: Dict[int, Tuple[int, ...]] = {}

    def reset(self) -> None:
        """Forget cached frequency lists and free every workspace."""
        self.freq_cache.clear()
        self.ws.clear()

    def retain(self, keys) -> None:
        """Forget cached frequency lists; free the workspaces whose plan key is
        not in `keys` (a workspace depends on its plan key only)."""
        self.freq_cache.clear()
        for wkey in [k for k in self.ws if k[0] not in keys]:
            del self.ws[wkey]

    def plan_key(self, param: torch.Tensor, st: dict, group: dict) -> tuple:
        """The plan key of a spectral tensor: (device, shape, freqs, hash_bins, hash_tables, work dtype)."""
        work = _native.F64 if param.dtype == torch.float64 else _native.F32
        return (param.device, tuple(int(d) for d in param.shape), self._freqs(st), int(group["hash_bins"]),
                int(group["hash_tables"]), work)

    def _freqs(self, st: dict) -> Tuple[int, ...]:
        fr = st["freqs"]
        key = id(fr)
        got = self.freq_cache.get(key)
        if got is None or got[0] is not fr:
            host = tuple(int(v) for v in fr.detach().to("cpu", torch.long).reshape(-1).tolist())
            got = (fr, host)
            self.freq_cache[key] = got
        return got[1]

    def _workspace(self, key: tuple, lane: int, rank: int, group: dict, count=None) -> _Workspace:
        wkey = (key, count is not None, lane)
        ws = self.ws.get(wkey)
        if ws is None or (count is not None and ws.count < count):
            device, shape, freqs, bins, tables, work = key
            ws = None
            self.ws.pop(wkey, None)
            ws = _Workspace(self.lib, shape, freqs, rank, bins, tables, group, device, count, work)
            self.ws[wkey] = ws
        return ws

    def _prepare(self, param: torch.Tensor, grad: torch.Tensor, st: dict, group: dict):
        """Validate one tensor's state and build its descriptor; -> (key, rank, desc)."""
        if (param.dtype, grad.dtype) not in _DTYPE_PAIRS:
            raise RuntimeError(f"CRESSO5 spectral route on MI355X supports fp64/fp32/bf16/fp16 params with grads of "
                               f"the same dtype, and fp32 params with bf16/fp16 grads (got {param.dtype} / {grad.dtype})")
        sdt = torch.float64 if param.dtype == torch.float64 else torch.float32
        for k in ("force_rms", "drive_energy", "surprise", "action", "omega") + _VEC_KEYS:
            if st[k].dtype != sdt:
                raise RuntimeError(f"CRESSO5 spectral state {k} has dtype {st[k].dtype}, expected {sdt}")
        rank = int(st["omega"].numel())
        bins, tables = int(group["hash_bins"]), int(group["hash_tables"])
        key = self.plan_key(param, st, group)
        shape = key[1]
        cut = int(group["thin_matrix_hard_cutoff"])
        thin = param.ndim == 2 and cut > 0 and min(shape) <= cut
        hard = param.numel() >= int(group["hard_channel_min_size"]) and not thin
        d = _native.SpectralDesc()
        d.param = param.data_ptr()
        d.grad = grad.data_ptr()
        d.param_dtype = _native.DTYPE_CODE[param.dtype]
        d.grad_dtype = _native.DTYPE_CODE[grad.dtype]
        d.numel = param.numel()
        d.force_rms = st["force_rms"].data_ptr()
        d.drive_energy = st["drive_energy"].data_ptr()
        d.surprise = st["surprise"].data_ptr()
        d.action = st["action"].data_ptr()
        d.omega = st["omega"].data_ptr()
        for k in _VEC_KEYS:
            setattr(d, k, st[k].data_ptr())
        if hard and bins > 0 and "hash_energy" in st:
            for k in ("hash_energy", "hash_impulse", "hash_refractory"):
                if tuple(st[k].shape) != (tables, bins) or st[k].dtype != sdt:
                    raise RuntimeError(f"CRESSO5 spectral state {k} has shape {tuple(st[k].shape)}, expected "
                                       f"({tables}, {bins}) {sdt} (hash_bins/hash_tables changed after init?)")
            d.hash_energy = st["hash_energy"].data_ptr()
            d.hash_impulse = st["hash_impulse"].data_ptr()
            d.hash_refractory = st["hash_refractory"].data_ptr()
        d.step = int(st["step"]) + 1
        d.hard = 1 if hard else 0
        return key, rank, d

    def _launch(self, ws: _Workspace, d, hyper, stream: int) -> None:
        _native.check(self.lib.cresso_spectral_step(ws.plan, ctypes.byref(d), ctypes.c_void_p(ws.buf.data_ptr()),
                                                    ctypes.c_size_t(ws.buf.numel()), ctypes.byref(hyper),
                                                    ctypes.c_void_p(stream)), "spectral route step")

    def _launch_batch(self, ws: _Workspace, descs: list, hyper, stream: int) -> None:
        arr = (_native.SpectralDesc * len(descs))(*descs)
        _native.check(self.lib.cresso_spectral_step_batched(ws.plan, arr, len(descs), ctypes.c_void_p(ws.buf.data_ptr()),
                                                            ctypes.c_size_t(ws.buf.numel()), ctypes.byref(hyper),
                                                            ctypes.c_void_p(stream)), "spectral route batched step")

    def step(self, param: torch.Tensor, grad: torch.Tensor, st: dict, group: dict) -> None:
        """One tensor on the caller's stream."""
        key, rank, d = self._prepare(param, grad, st, group)
        ws = self._workspace(key, 0, rank, group)
        st["step"] += 1
        self._launch(ws, d, _native.hyper_from_group(group), _native.stream_handle(param.device))

    def _streams(self, device: torch.device, n: int) -> List[torch.cuda.Stream]:
        have = self.side.setdefault(device, [])
        while len(have) < n:
            have.append(torch.cuda.Stream(device=device))   # default priority
        return have[:n]

    def _units(self, prepared: list, sts: list) -> list:
        """Cut a step's tensors into units: (unit key, plan key, rank, [desc], [state]).
        Tensors batch when they share the plan, dtypes, hard channel and hash
        state; fp64 tensors step one at a time (fp64 plans are not batched)."""
        groups: Dict[tuple, list] = {}
        for i, (key, rank, d) in enumerate(prepared):
            bkey = (key, d.param_dtype, d.grad_dtype, d.hard, bool(d.hash_energy))
            alone = not self.BATCH or d.param_dtype == _native.F64
            groups.setdefault((bkey, i) if alone else bkey, []).append(i)
        units = []
        for bkey, idx in groups.items():
            key, rank, _ = prepared[idx[0]]
            if len(idx) == 1:
                units.append(((key, False), key, rank, [prepared[idx[0]][2]], [sts[idx[0]]]))
                continue
            per = lane_scratch_bytes(prepared[idx[0]][2].numel)
            chunks = -(-len(idx) * per // self.BATCH_BYTES)
            m = -(-len(idx) // chunks)
            for c in range(0, len(idx), m):
                sel = idx[c:c + m]
                units.append(((key, True, m), key, rank, [prepared[i][2] for i in sel], [sts[i] for i in sel]))
        return units

    def step_many(self, items: Sequence[Tuple[torch.Tensor, torch.Tensor, dict]], group: dict) -> None:
        """Every spectral tensor of a param group: (param, grad, state) each."""
        if len(items) == 1:
            self.step(*items[0], group)
            return
        by_dev: Dict[torch.device, list] = {}
        for it in items:
            by_dev.setdefault(it[0].device, []).append(it)
        hyper = _native.hyper_from_group(group)
        for device, its in by_dev.items():
            # descriptors and workspaces first: a workspace created now is
            # initialised on the caller's stream, before the lanes fork from it
            prepared = [self._prepare(p, g, st, group) for p, g, st in its]
            units = self._units(prepared, [st for _, _, st in its])
            nl = min(self.LANES, len(units))
            lanes = assign_lanes([u[0][:2] for u in units], nl)
            plan = []
            for (ukey, key, rank, descs, sts), lane in zip(units, lanes):
                count = ukey[2] if ukey[1] else None
                plan.append((self._workspace(key, lane, rank, group, count), descs, sts, lane))
            cur = torch.cuda.current_stream(device)
            side = self._streams(device, nl)
            for s in side:
                s.wait_stream(cur)
            for ws, descs, sts, lane in plan:
                for st in sts:
                    st["step"] += 1
                if ws.count is None:
                    self._launch(ws, descs[0], hyper, int(side[lane].cuda_stream))
                else:
                    self._launch_batch(ws, descs, hyper, int(side[lane].cuda_stream))
            for s in side:
                cur.wait_stream(s)
