"""Host orchestration of the spectral/hash route (one C call per tensor and step).

The library keeps no state of its own: plans live here, keyed by
(device, shape, freqs, hash_bins, hash_tables), together with their device
workspace (carrier tables, cached coordinate-hash bins, scratch).  Tensors of
the same shape share one workspace; they run one after another on the same
stream, so the per-step scratch in it is never used concurrently.
"""

from __future__ import annotations

import ctypes
from typing import Dict, Tuple

import torch

from . import _native

_VEC_KEYS = ("q_cos", "q_sin", "p_cos", "p_sin", "metric_cos", "metric_sin", "metric_p_cos", "metric_p_sin",
             "calcium_cos", "calcium_sin", "mode_confidence")


class _Workspace:
    def __init__(self, lib, shape, freqs_host: Tuple[int, ...], rank: int, bins: int, tables: int, group: dict,
                 device: torch.device):
        self.lib = lib
        nd = len(shape)
        shp = (ctypes.c_int64 * 8)(*shape)
        fr = (ctypes.c_int64 * max(1, len(freqs_host)))(*freqs_host)
        plan = lib.cresso_spectral_plan_create(shp, nd, fr, rank, bins, tables)
        if not plan:
            _native.check(-1, "spectral route plan")
        self.plan = ctypes.c_void_p(plan)
        nbytes = int(lib.cresso_spectral_workspace_bytes(self.plan))
        self.buf = torch.empty(nbytes, dtype=torch.uint8, device=device)
        hyper = _native.hyper_from_group(group)
        stream = _native.stream_handle(device)
        _native.check(lib.cresso_spectral_workspace_init(self.plan, ctypes.c_void_p(self.buf.data_ptr()),
                                                         ctypes.c_size_t(nbytes), ctypes.byref(hyper),
                                                         ctypes.c_void_p(stream)), "spectral workspace init")

    def __del__(self):
        plan = getattr(self, "plan", None)
        if plan is not None and plan.value:
            try:
                self.lib.cresso_spectral_plan_destroy(plan)
            except Exception:
                pass


class SpectralEngine:
    READY = True

    def __init__(self):
        self.lib = _native.load()
        self.ws: Dict[tuple, _Workspace] = {}
        self.freq_cache: Dict[int, Tuple[int, ...]] = {}

    def reset(self) -> None:
        self.freq_cache.clear()

    def _freqs(self, st: dict) -> Tuple[int, ...]:
        fr = st["freqs"]
        key = id(fr)
        got = self.freq_cache.get(key)
        if got is None or got[0] is not fr:
            host = tuple(int(v) for v in fr.detach().to("cpu", torch.long).reshape(-1).tolist())
            got = (fr, host)
            self.freq_cache[key] = got
        return got[1]

    def step(self, param: torch.Tensor, grad: torch.Tensor, st: dict, group: dict) -> None:
        if param.dtype not in (torch.float32, torch.bfloat16, torch.float16) or grad.dtype != param.dtype:
            raise RuntimeError(f"CRESSO5 spectral route on MI355X supports fp32/bf16/fp16 params with grads of the "
                               f"same dtype (got {param.dtype} / {grad.dtype})")
        for k in ("force_rms", "omega") + _VEC_KEYS:
            if st[k].dtype != torch.float32:
                raise RuntimeError(f"CRESSO5 spectral state {k} has dtype {st[k].dtype}, expected float32")
        rank = int(st["omega"].numel())
        freqs = self._freqs(st)
        bins, tables = int(group["hash_bins"]), int(group["hash_tables"])
        shape = tuple(int(d) for d in param.shape)
        key = (param.device, shape, freqs, bins, tables)
        ws = self.ws.get(key)
        if ws is None:
            ws = _Workspace(self.lib, shape, freqs, rank, bins, tables, group, param.device)
            self.ws[key] = ws
        st["step"] += 1
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
                if tuple(st[k].shape) != (tables, bins) or st[k].dtype != torch.float32:
                    raise RuntimeError(f"CRESSO5 spectral state {k} has shape {tuple(st[k].shape)}, expected "
                                       f"({tables}, {bins}) float32 (hash_bins/hash_tables changed after init?)")
            d.hash_energy = st["hash_energy"].data_ptr()
            d.hash_impulse = st["hash_impulse"].data_ptr()
            d.hash_refractory = st["hash_refractory"].data_ptr()
        d.step = int(st["step"])
        d.hard = 1 if hard else 0
        hyper = _native.hyper_from_group(group)
        stream = _native.stream_handle(param.device)
        _native.check(self.lib.cresso_spectral_step(ws.plan, ctypes.byref(d), ctypes.c_void_p(ws.buf.data_ptr()),
                                                    ctypes.c_size_t(ws.buf.numel()), ctypes.byref(hyper),
                                                    ctypes.c_void_p(stream)), "spectral route step")
