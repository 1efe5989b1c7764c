"""CRESSO5 optimizer front end for MI355X.

Same constructor, validation messages, routing, persistent state layout and
``step()``/``state_dict()`` contract as the reference optimizer
(/root/reference/cresso_v5.py:612-1585).  All math runs in libcresso_hip.so
(gfx950 HIP kernels); this module only routes tensors, owns the state
tensors and calls the C ABI.  There is no PyTorch/CPU fallback: when the
library cannot run, ``step()`` raises.
"""

from __future__ import annotations

import ctypes
import math
from typing import Dict, Iterable, List, Optional, Sequence, Tuple

import torch
from torch import Tensor
from torch.optim import Optimizer

from . import _native
from .modes import freqs_tensor, omega_tensor

__all__ = ["CRESSO5", "CRESSO", "count_optimizer_state_elements", "theoretical_state_elements"]

# (name, lower, upper) of every float hyperparameter, cresso_v5.py:682-725
_FLOAT_BOUNDS = (
    ("lr", 0.0, None), ("weight_decay", 0.0, None), ("energy_power", 0.25, None), ("dt", 0.0, 1.0),
    ("impulse_friction", 0.0, None), ("contact_gain", 0.0, None), ("restoring", 0.0, None), ("cubic", 0.0, None),
    ("metric_dt", 0.0, 1.0), ("metric_friction", 0.0, None), ("metric_coupling", 0.0, None),
    ("local_sharpness", 0.0, None), ("instant_metric_coupling", 0.0, None), ("instant_metric_power", 0.25, None),
    ("root_channel_mix", 0.0, 1.0), ("echo_mix", 0.0, 1.0), ("transport_mix", 0.0, 1.0), ("hash_decay", 0.0, 1.0),
    ("hash_impulse_decay", 0.0, 1.0), ("hash_metric_coupling", 0.0, None), ("hash_drive_mix", 0.0, 1.0),
    ("direct_force_mix", 0.0, 1.0), ("residual_feedback_mix", 0.0, 1.0), ("micro_decay", 0.0, 1.0),
    ("micro_impulse_decay", 0.0, 1.0), ("micro_drive_mix", 0.0, 1.0), ("reservoir_decay", 0.0, 1.0),
    ("refractory_decay", 0.0, 1.0), ("refractory_gain", 0.0, None), ("confidence_decay", 0.0, 1.0),
    ("confidence_gain", 0.0, None), ("surprise_gain", 0.0, None), ("surprise_decay", 0.0, 1.0),
    ("prediction_mix", 0.0, 1.0), ("novelty_mix", 0.0, 1.0), ("surprise_brake", 0.0, None),
    ("target_update_rms", 0.0, None), ("min_gain", 0.0, None), ("max_gain", 0.0, None), ("drive_clip", 0.1, None),
    ("spike_mix", 0.0, 1.0), ("eps", 0.0, None),
)
_INT_NONNEG = (("rank", "rank must be non-negative"), ("max_frequency", "max_frequency must be non-negative"),
               ("hash_bins", "hash_bins must be non-negative"))

_SCALAR_KEYS = ("q", "impulse", "metric_q", "metric_impulse", "force_rms", "drive_energy", "surprise", "action")
# state order of a micro-route descriptor (route 1): dense fields, then the scalars
_MICRO_KEYS = ("micro_energy", "micro_impulse", "micro_refractory", "force_rms", "drive_energy", "surprise", "action")
_SPECTRAL_VEC_KEYS = ("q_cos", "q_sin", "p_cos", "p_sin", "metric_cos", "metric_sin", "metric_p_cos", "metric_p_sin",
                      "calcium_cos", "calcium_sin", "mode_confidence")


def _check_scalar(name: str, value, lower, upper) -> None:
    if not isinstance(value, (int, float)) or not math.isfinite(float(value)):
        raise ValueError(f"{name} must be a finite scalar, got {value!r}")
    if lower is not None and value < lower:
        raise ValueError(f"{name} must be >= {lower}, got {value}")
    if upper is not None and value > upper:
        raise ValueError(f"{name} must be <= {upper}, got {value}")


def _state_dtype(dtype: torch.dtype) -> torch.dtype:
    return torch.float64 if dtype == torch.float64 else torch.float32


def _normalize_route(route: str) -> str:
    r = str(route).lower()
    if r not in ("scalar", "spectral"):
        raise ValueError("thin_matrix_route must be one of 'scalar' or 'spectral'")
    return r


def _lora_thin(dims: Sequence[int], max_width: int, min_aspect: float) -> bool:
    if len(dims) != 2 or int(max_width) <= 0:
        return False
    lo, hi = min(dims), max(dims)
    return lo > 0 and lo <= int(max_width) and hi / lo >= float(min_aspect)


def _thin_scalar(dims, route="scalar", max_width=64, min_aspect=4.0) -> bool:
    return _normalize_route(route) == "scalar" and _lora_thin(tuple(int(d) for d in dims), max_width, min_aspect)


def count_optimizer_state_elements(optimizer: Optimizer) -> int:
    """Total elements of every tensor in optimizer.state (cresso_v5.py:529-535)."""
    return int(sum(v.numel() for st in optimizer.state.values() for v in st.values() if torch.is_tensor(v)))


def theoretical_state_elements(shape: Sequence[int], rank: int, spectral: bool = True, hash_bins: int = 128,
                               hash_tables: int = 2, micro_field_max_size: int = 0, hard_channel_min_size: int = 16,
                               thin_matrix_hard_cutoff: int = 8, thin_matrix_max_width: int = 64,
                               thin_matrix_min_aspect: float = 4.0, thin_matrix_route: str = "scalar") -> int:
    """Persistent-state size contract (cresso_v5.py:573-609)."""
    dims = tuple(int(d) for d in shape)
    n = math.prod(dims) if dims else 1
    if int(micro_field_max_size) > 0 and dims and n <= int(micro_field_max_size):
        return 3 * n + 4
    if spectral and not _thin_scalar(dims, thin_matrix_route, thin_matrix_max_width, thin_matrix_min_aspect):
        thin = len(dims) == 2 and int(thin_matrix_hard_cutoff) > 0 and min(dims) <= int(thin_matrix_hard_cutoff)
        hard = n >= int(hard_channel_min_size) and not thin
        return int(rank) * len(dims) + 12 * int(rank) + (3 * int(hash_bins) * int(hash_tables) if hard else 0) + 4
    return 8


class _ScalarBatch:
    """Cached plan of the scalar-route and micro-route tensors of one param
    group on one device (one library plan; micro tensors carry route 1)."""

    def __init__(self, params: List[Tensor], grads: List[Tensor], states: List[dict], group: dict,
                 device: torch.device):
        lib = _native.load()
        self.lib = lib
        self.params = params
        self.states = states
        self.device = device
        self.pptrs = [p.data_ptr() for p in params]
        self.gdtypes = [g.dtype for g in grads]   # the plan's descriptors fix the grad dtype
        self.hyper_key = self.key_of(group)
        descs = (_native.ScalarDesc * len(params))()
        for i, (p, g, st) in enumerate(zip(params, grads, states)):
            d = descs[i]
            d.param = p.data_ptr()
            d.grad = g.data_ptr()
            micro = "micro_energy" in st
            for j, k in enumerate(_MICRO_KEYS if micro else _SCALAR_KEYS):
                d.state[j] = st[k].data_ptr()
            d.route = _native.ROUTE_MICRO if micro else _native.ROUTE_SCALAR
            for a, s in enumerate(p.shape):
                d.shape[a] = int(s)
            d.numel = p.numel()
            d.ndim = p.ndim
            d.param_dtype = _native.DTYPE_CODE[p.dtype]
            d.grad_dtype = _native.DTYPE_CODE[g.dtype]
            d.step = int(st["step"])
        self.descs = descs
        hyper = _native.hyper_from_group(group)
        plan = lib.cresso_scalar_plan_create(descs, len(params), ctypes.byref(hyper))
        if not plan:
            _native.check(-1, "scalar route plan")
        self.plan = ctypes.c_void_p(plan)
        nbytes = int(lib.cresso_scalar_plan_bytes(self.plan))
        self.table = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
        stream = _native.stream_handle(device)
        _native.check(lib.cresso_scalar_plan_upload(self.plan, ctypes.c_void_p(self.table.data_ptr()),
                                                    ctypes.c_size_t(self.table.numel()), ctypes.c_void_p(stream)),
                      "scalar route upload")
        self.gptr_type = ctypes.c_void_p * len(params)
        # steady-state host bookkeeping in C++ when the helper is built
        self.gbuf = self.gptr_type()
        self.guard = None
        hb = _native.host_batch()
        if hb is not None and all(p.grad is not None for p in params):   # (not for contiguous copies)
            try:
                self.guard = hb.BatchGuard(list(params))
            except (ValueError, RuntimeError):
                self.guard = None

    @staticmethod
    def key_of(group: dict):
        return tuple(group[k] for k in _native.HYPER_DOUBLES if k != "lr") + (group["warmup_steps"], group["maximize"])

    def matches(self, params: List[Tensor], gdtypes: List[torch.dtype], group: dict) -> bool:
        return (len(params) == len(self.params) and all(a is b for a, b in zip(params, self.params))
                and [p.data_ptr() for p in params] == self.pptrs and self.key_of(group) == self.hyper_key
                and gdtypes == self.gdtypes)

    @staticmethod
    def grads_ready(params: List[Tensor]) -> bool:
        """Every grad can be passed by pointer as it is (dense, contiguous, the
        parameter's shape and device)."""
        return all(not p.grad.is_sparse and p.grad.is_contiguous() and p.grad.shape == p.shape
                   and p.grad.device == p.device for p in params)

    def run(self, group: dict, gptrs: Optional[List[int]]) -> None:
        """One step; gptrs None: the grad pointers are already in self.gbuf."""
        hyper = _native.hyper_from_group(group)
        arr = self.gbuf if gptrs is None else self.gptr_type(*gptrs)
        stream = _native.stream_handle(self.device)
        _native.check(self.lib.cresso_scalar_plan_step(self.plan, ctypes.c_void_p(self.table.data_ptr()), arr,
                                                       ctypes.byref(hyper), ctypes.c_void_p(stream)),
                      "scalar route step")
        if self.guard is not None:
            self.guard.bump(self.states)
        else:
            for st in self.states:
                st["step"] += 1

    def fast_step(self, group: dict) -> bool:
        """Steady state in C++: same params and storage, fresh grads of the
        planned dtype; False (nothing launched) when anything changed."""
        if self.guard is None or self.key_of(group) != self.hyper_key:
            return False
        if not self.guard.gather(group["params"], ctypes.addressof(self.gbuf)):
            return False
        self.run(group, None)
        return True

    def __del__(self):
        plan = getattr(self, "plan", None)
        if plan is not None and plan.value:
            try:
                self.lib.cresso_scalar_plan_destroy(plan)
            except Exception:
                pass


class CRESSO5(Optimizer):
    """Contact-Refractory Axial-Spectral Optimizer on MI355X.

    Persistent state per tensor is O(rank*ndim + rank + hash_tables*hash_bins)
    on the spectral route and 8 scalars on the scalar route, exactly as in the
    reference.  ``cuda_ops`` keeps its name for drop-in compatibility: on ROCm
    ``torch.cuda`` is HIP.
    """

    def __init__(self, params: Iterable[Tensor], lr: float = 2.0e-3, rank: int = 8, max_frequency: int = 5,
                 weight_decay: float = 0.0, energy_power: float = 1.20, dt: float = 0.15,
                 impulse_friction: float = 0.18, contact_gain: float = 0.16, restoring: float = 0.62,
                 cubic: float = 0.006, metric_dt: float = 0.09, metric_friction: float = 0.22,
                 metric_coupling: float = 0.36, local_sharpness: float = 0.0, instant_metric_coupling: float = 0.55,
                 instant_metric_power: float = 1.0, root_channel_mix: float = 0.16, echo_mix: float = 0.06,
                 transport_mix: float = 0.18, hash_bins: int = 128, hash_tables: int = 2, hash_decay: float = 0.92,
                 hash_impulse_decay: float = 0.78, hash_metric_coupling: float = 0.42, hash_drive_mix: float = 0.22,
                 direct_force_mix: float = 0.18, residual_feedback_mix: float = 0.06, micro_field_max_size: int = 0,
                 micro_decay: float = 0.94, micro_impulse_decay: float = 0.82, micro_drive_mix: float = 0.35,
                 reservoir_decay: float = 0.95, refractory_decay: float = 0.90, refractory_gain: float = 0.55,
                 confidence_decay: float = 0.92, confidence_gain: float = 0.50, surprise_gain: float = 0.18,
                 surprise_decay: float = 0.95, prediction_mix: float = 0.16, novelty_mix: float = 0.04,
                 warmup_steps: int = 10, surprise_brake: float = 0.18, target_update_rms: float = 1.0,
                 min_gain: float = 0.04, max_gain: float = 6.0, drive_clip: float = 4.0, spike_mix: float = 0.25,
                 min_spectral_size: int = 1024, basis_cache_limit_elements: int = 2_000_000,
                 cuda_ops: str | bool = "auto", hard_channel_min_size: int = 16, thin_matrix_hard_cutoff: int = 8,
                 thin_matrix_max_width: int = 64, thin_matrix_min_aspect: float = 4.0,
                 thin_matrix_route: str = "scalar", maximize: bool = False, eps: float = 1e-8) -> None:
        args = dict(locals())
        for name, lo, hi in _FLOAT_BOUNDS:
            _check_scalar(name, args[name], lo, hi)
        for name, msg in _INT_NONNEG:
            if int(args[name]) < 0:
                raise ValueError(msg)
        if int(hash_tables) < 1:
            raise ValueError("hash_tables must be >= 1")
        if int(min_spectral_size) < 1:
            raise ValueError("min_spectral_size must be >= 1")
        for name in ("micro_field_max_size", "basis_cache_limit_elements", "hard_channel_min_size",
                     "thin_matrix_hard_cutoff", "thin_matrix_max_width"):
            if int(args[name]) < 0:
                raise ValueError(f"{name} must be >= 0")
        _check_scalar("thin_matrix_min_aspect", thin_matrix_min_aspect, 1.0, None)
        if int(warmup_steps) < 0:
            raise ValueError("warmup_steps must be non-negative")
        if min_gain > max_gain:
            raise ValueError("min_gain must be <= max_gain")
        route = _normalize_route(thin_matrix_route)
        mode = ("auto" if cuda_ops else "off") if isinstance(cuda_ops, bool) else str(cuda_ops).lower()
        if mode not in ("auto", "required", "off"):
            raise ValueError("cuda_ops must be one of 'auto', 'required', or 'off'")
        defaults = {}
        for name, _, _ in _FLOAT_BOUNDS:
            defaults[name] = float(args[name])
        for name in ("rank", "max_frequency", "hash_bins", "hash_tables", "micro_field_max_size", "warmup_steps",
                     "min_spectral_size", "basis_cache_limit_elements", "hard_channel_min_size",
                     "thin_matrix_hard_cutoff", "thin_matrix_max_width"):
            defaults[name] = int(args[name])
        defaults.update(cuda_ops=mode, thin_matrix_min_aspect=float(thin_matrix_min_aspect), thin_matrix_route=route,
                        maximize=bool(maximize))
        super().__init__(params, defaults)
        self._batches: Dict[Tuple[int, str], _ScalarBatch] = {}
        self._group_other: Dict[int, bool] = {}
        self._spectral_engine = None

    # ------------------------------------------------------------------ routing
    @staticmethod
    def _route(param: Tensor, group: dict) -> str:
        """'micro' | 'spectral' | 'scalar' (cresso_v5.py:839-855)."""
        if int(group["micro_field_max_size"]) > 0 and param.ndim > 0 and param.numel() <= int(group["micro_field_max_size"]):
            return "micro"
        if param.numel() >= int(group["min_spectral_size"]) and int(group["rank"]) > 0 and param.ndim > 0 and not _thin_scalar(
                tuple(param.shape), group["thin_matrix_route"], group["thin_matrix_max_width"],
                group["thin_matrix_min_aspect"]):
            return "spectral"
        return "scalar"

    def _use_spectral_route(self, param: Tensor, group: dict) -> bool:
        return self._route(param, group) == "spectral"

    # --------------------------------------------------------------- state init
    def _init_common(self, state: dict, device, dtype) -> None:
        state["step"] = 0
        state["force_rms"] = torch.zeros((), device=device, dtype=dtype)
        state["drive_energy"] = torch.ones((), device=device, dtype=dtype)
        state["surprise"] = torch.zeros((), device=device, dtype=dtype)
        state["action"] = torch.zeros((), device=device, dtype=dtype)

    def _step_empty(self, param: Tensor, group: dict) -> None:
        """A parameter with no elements (the scalar or micro route: the
        spectral route needs min_spectral_size >= 1 elements): nothing to
        update.  The reference's step takes its means over no elements, so the
        state entries computed from them become NaN: every floating scalar of
        the scalar route; the three reservoirs of the micro route, whose
        action the micro step does not touch (cresso_v5.py:1355-1432, 1434-1585)."""
        micro = self._route(param, group) == "micro"
        st = self.state[param]
        if len(st) == 0:
            st = self._init_micro(param) if micro else self._init_scalar(param)
        st["step"] = int(st["step"]) + 1
        keep = {"action"} if micro else set()
        for k, v in st.items():
            if torch.is_tensor(v) and v.is_floating_point() and v.numel() > 0 and k not in keep:
                v.fill_(float("nan"))

    def _init_scalar(self, param: Tensor) -> dict:
        st = self.state[param]
        dtype = _state_dtype(param.dtype)
        self._init_common(st, param.device, dtype)
        for k in ("q", "impulse", "metric_q", "metric_impulse"):
            st[k] = torch.zeros((), device=param.device, dtype=dtype)
        return st

    def _init_micro(self, param: Tensor) -> dict:
        """cresso_v5.py:893-898: common scalars plus three dense fields."""
        st = self.state[param]
        dtype = _state_dtype(param.dtype)
        self._init_common(st, param.device, dtype)
        st["micro_energy"] = torch.ones_like(param.detach(), dtype=dtype, memory_format=torch.contiguous_format)
        st["micro_impulse"] = torch.zeros_like(param.detach(), dtype=dtype, memory_format=torch.contiguous_format)
        st["micro_refractory"] = torch.zeros_like(param.detach(), dtype=dtype, memory_format=torch.contiguous_format)
        return st

    def _init_spectral(self, param: Tensor, group: dict) -> dict:
        st = self.state[param]
        dtype = _state_dtype(param.dtype)
        self._init_common(st, param.device, dtype)
        rank = int(group["rank"])
        freqs = freqs_tensor(rank, param.ndim, int(group["max_frequency"]), param.device)
        st["freqs"] = freqs
        st["omega"] = omega_tensor(freqs).to(device=param.device, dtype=dtype)
        for k in _SPECTRAL_VEC_KEYS:
            st[k] = torch.zeros(rank, device=param.device, dtype=dtype)
        bins, tables = int(group["hash_bins"]), int(group["hash_tables"])
        cut = int(group["thin_matrix_hard_cutoff"])
        thin = param.ndim == 2 and cut > 0 and min(param.shape) <= cut
        if bins > 0 and param.numel() >= int(group["hard_channel_min_size"]) and not thin:
            st["hash_energy"] = torch.ones(tables, bins, device=param.device, dtype=dtype)
            st["hash_impulse"] = torch.zeros(tables, bins, device=param.device, dtype=dtype)
            st["hash_refractory"] = torch.zeros(tables, bins, device=param.device, dtype=dtype)
        return st

    # --------------------------------------------------------------------- step
    @torch.no_grad()
    def step(self, closure: Optional[callable] = None):  # type: ignore[override]
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        for gi, group in enumerate(self.param_groups):
            self._step_group(gi, group)
        return loss

    def _fast_scalar(self, gi: int, group: dict) -> bool:
        """Steady-state path: the group is exactly the cached scalar batch and
        only the grad tensors are new (autograd allocates them every step)."""
        batch = self._batches.get((gi, "scalar"))
        if batch is None or self._group_other.get(gi, True):
            return False
        if batch.guard is not None:
            return batch.fast_step(group)
        try:
            gptrs = [p.grad.data_ptr() for p in batch.params]
        except (AttributeError, RuntimeError):
            return False
        if (not batch.matches(group["params"], [p.grad.dtype for p in batch.params], group)
                or not batch.grads_ready(batch.params)):
            return False
        batch.run(group, gptrs)
        return True

    def _step_group(self, gi: int, group: dict) -> None:
        if self._fast_scalar(gi, group):
            return
        mode = str(group.get("cuda_ops", "auto"))
        scalar_ps: List[Tensor] = []   # the scalar/micro tensors stepped (contiguous)
        scalar_gs: List[Tensor] = []   # their grads (contiguous)
        scalar_st: List[dict] = []     # their states (keyed by the parameter)
        spectral_items = []
        copies = []                    # (parameter, contiguous copy) of non-contiguous parameters
        other = False
        for p in group["params"]:
            if p.grad is None or not torch.is_floating_point(p):
                other = True
                continue
            grad = p.grad
            if grad.is_sparse:
                raise RuntimeError("CRESSO5 does not support sparse gradients")
            if mode == "required" and not p.is_cuda:
                raise RuntimeError("CRESSO5 cuda_ops='required' requires every optimized parameter to be a CUDA parameter")
            if mode == "off":
                raise RuntimeError("CRESSO5 cuda_ops='off' selects the reference PyTorch path, which this MI355X build "
                                   "does not ship; use cuda_ops='auto' or 'required'")
            if not p.is_cuda:
                raise RuntimeError("CRESSO5 on MI355X optimizes GPU parameters only (got a CPU parameter with "
                                   "cuda_ops='auto'); the reference's CPU PyTorch path is not part of this build")
            if grad.shape != p.shape:
                raise RuntimeError("CRESSO5 needs gradients of the parameter's shape")
            # The kernels read elements in the parameter's (row-major) order:
            # other layouts (channels-last convolution weights, transposed
            # views) step through contiguous copies on the current stream,
            # which outlive the launches that read them (the side streams join
            # back first), and the parameter takes the result back in its own
            # layout.
            if not grad.is_contiguous():
                grad = grad.contiguous()
            data = p
            if not p.is_contiguous():
                data = p.detach().contiguous()
                copies.append((p, data))
                other = True
            if p.numel() == 0:
                other = True
                self._step_empty(p, group)
                continue
            route = self._route(p, group)
            if route == "micro":
                st = self.state[p]
                if len(st) == 0:
                    st = self._init_micro(p)
                else:
                    self._check_micro_state(p, st)
                scalar_ps.append(data)
                scalar_gs.append(grad)
                scalar_st.append(st)
                continue
            if route == "spectral":
                other = True
                st = self.state[p]
                if len(st) == 0:
                    st = self._init_spectral(p, group)
                spectral_items.append((data, grad, st))
                continue
            st = self.state[p]
            if len(st) == 0:
                st = self._init_scalar(p)
            elif "q" not in st:
                raise RuntimeError("CRESSO5 scalar route: the parameter's state belongs to another route")
            elif st["q"].dtype != _state_dtype(p.dtype):
                raise RuntimeError("CRESSO5 scalar state has dtype %s, expected %s" % (st["q"].dtype, _state_dtype(p.dtype)))
            scalar_ps.append(data)
            scalar_gs.append(grad)
            scalar_st.append(st)
        if spectral_items:
            self._spectral_step(spectral_items, group)
        self._group_other[gi] = other
        if scalar_ps:
            self._step_scalar_batch(gi, group, scalar_ps, scalar_gs, scalar_st)
        else:
            self._batches.pop((gi, "scalar"), None)
        for p, data in copies:
            p.detach().copy_(data)

    def _step_scalar_batch(self, gi: int, group: dict, scalar_ps: List[Tensor], scalar_gs: List[Tensor],
                           scalar_st: List[dict]) -> None:
        devices = {p.device for p in scalar_ps}
        if len(devices) != 1:
            raise RuntimeError("CRESSO5 scalar route: all parameters of a group must be on one device")
        batch = self._batches.get((gi, "scalar"))
        if batch is None or not batch.matches(scalar_ps, [g.dtype for g in scalar_gs], group):
            self._batches[(gi, "scalar")] = None  # drop the old plan first
            batch = _ScalarBatch(scalar_ps, scalar_gs, scalar_st, group, scalar_ps[0].device)
            self._batches[(gi, "scalar")] = batch
        batch.run(group, [g.data_ptr() for g in scalar_gs])

    @staticmethod
    def _check_micro_state(p: Tensor, st: dict) -> None:
        want = _state_dtype(p.dtype)
        for k in _MICRO_KEYS:
            if k not in st:
                raise RuntimeError(f"CRESSO5 micro route: state {k!r} is missing (the state belongs to another route)")
            v = st[k]
            if v.dtype != want or v.device != p.device:
                raise RuntimeError(f"CRESSO5 micro route: state {k!r} is {v.dtype} on {v.device}, expected {want} on "
                                   f"{p.device}")
        for k in _MICRO_KEYS[:3]:
            if st[k].shape != p.shape or not st[k].is_contiguous():
                raise RuntimeError(f"CRESSO5 micro route: state {k!r} must be contiguous with the parameter's shape")

    def _spectral_step(self, items, group: dict) -> None:
        """Every spectral tensor of the group: (param, grad, state) each."""
        if self._spectral_engine is None:
            from .spectral import SpectralEngine
            self._spectral_engine = SpectralEngine()
        self._spectral_engine.step_many(items, group)

    # ------------------------------------------------------------- checkpoints
    def load_state_dict(self, state_dict: dict) -> None:
        """torch's loader casts every non-step state tensor to param.dtype
        (freqs becomes float, bf16 params get bf16 state); restore the saved
        dtypes instead: int64 freqs and fp32 (fp64 for fp64 params) state."""
        super().load_state_dict(state_dict)
        saved_ids = [pid for g in state_dict["param_groups"] for pid in g["params"]]
        params = [p for g in self.param_groups for p in g["params"]]
        for pid, p in zip(saved_ids, params):
            saved = state_dict["state"].get(pid)
            if not saved:
                continue
            st = self.state[p]
            for k, v in saved.items():
                if torch.is_tensor(v):
                    if k == "freqs":
                        st[k] = v.to(device=p.device, dtype=torch.long)
                    else:
                        st[k] = v.to(device=p.device, dtype=_state_dtype(p.dtype)).clone()
        self._batches.clear()
        if self._spectral_engine is not None:
            # workspaces are derived from (shape, freqs, hash_bins, hash_tables,
            # work dtype) only: keep those the loaded state still uses
            self._spectral_engine.retain(self._spectral_plan_keys())

    def _spectral_plan_keys(self) -> set:
        keys = set()
        for group in self.param_groups:
            for p in group["params"]:
                st = self.state.get(p)
                if st and "freqs" in st and "omega" in st:
                    keys.add(self._spectral_engine.plan_key(p, st, group))
        return keys


CRESSO = CRESSO5
