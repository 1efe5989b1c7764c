"""ctypes binding of libcresso_hip.so (the C ABI declared in include/cresso_hip.h).

The library is the only compute path of this package: there is no PyTorch or
CPU fallback.  :func:`load` raises ``RuntimeError`` when the library is
missing or was built for another ABI.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path
from typing import Optional

import torch

LIB_NAME = "libcresso_hip.so"
ABI_VERSION = 2

F32, F64, F16, BF16 = 0, 1, 2, 3
CRESSO_OK, CRESSO_E_INVALID, CRESSO_E_HIP, CRESSO_E_UNSUPPORTED = 0, -1, -2, -3
SPECTRAL_NOALLOC_MAX_BYTES = 32 << 20   # CRESSO_SPECTRAL_NOALLOC_MAX_BYTES
DTYPE_CODE = {torch.float32: F32, torch.float64: F64, torch.float16: F16, torch.bfloat16: BF16}

# Order of the double fields of cresso_hyper (include/cresso_hip.h).
HYPER_DOUBLES = (
    "lr", "weight_decay", "energy_power", "dt", "impulse_friction", "contact_gain",
    "restoring", "cubic", "metric_dt", "metric_friction", "metric_coupling",
    "local_sharpness", "instant_metric_coupling", "instant_metric_power",
    "root_channel_mix", "echo_mix", "transport_mix", "hash_decay",
    "hash_impulse_decay", "hash_metric_coupling", "hash_drive_mix",
    "direct_force_mix", "residual_feedback_mix", "reservoir_decay",
    "refractory_decay", "refractory_gain", "confidence_decay", "confidence_gain",
    "surprise_gain", "surprise_decay", "prediction_mix", "novelty_mix",
    "surprise_brake", "target_update_rms", "min_gain", "max_gain", "drive_clip",
    "spike_mix", "eps", "micro_decay", "micro_impulse_decay", "micro_drive_mix",
)


class Hyper(ctypes.Structure):
    _fields_ = [(n, ctypes.c_double) for n in HYPER_DOUBLES] + [
        ("warmup_steps", ctypes.c_int32),
        ("maximize", ctypes.c_int32),
    ]


class ScalarDesc(ctypes.Structure):
    _fields_ = [
        ("param", ctypes.c_void_p),
        ("grad", ctypes.c_void_p),
        ("state", ctypes.c_void_p * 8),
        ("shape", ctypes.c_int64 * 8),
        ("numel", ctypes.c_int64),
        ("ndim", ctypes.c_int32),
        ("param_dtype", ctypes.c_int32),
        ("grad_dtype", ctypes.c_int32),
        ("step", ctypes.c_int32),
        ("route", ctypes.c_int32),
    ]


ROUTE_SCALAR, ROUTE_MICRO = 0, 1


class SpectralDesc(ctypes.Structure):
    _fields_ = [
        ("param", ctypes.c_void_p),
        ("grad", ctypes.c_void_p),
        ("param_dtype", ctypes.c_int32),
        ("grad_dtype", ctypes.c_int32),
        ("numel", ctypes.c_int64),
    ] + [(k, ctypes.c_void_p) for k in (
        "force_rms", "drive_energy", "surprise", "action", "omega", "q_cos", "q_sin", "p_cos", "p_sin",
        "metric_cos", "metric_sin", "metric_p_cos", "metric_p_sin", "calcium_cos", "calcium_sin", "mode_confidence",
        "hash_energy", "hash_impulse", "hash_refractory")] + [
        ("step", ctypes.c_int32),
        ("hard", ctypes.c_int32),
    ]


def hyper_from_group(group: dict) -> Hyper:
    h = Hyper()
    for n in HYPER_DOUBLES:
        setattr(h, n, float(group[n]))
    h.warmup_steps = int(group["warmup_steps"])
    h.maximize = 1 if bool(group["maximize"]) else 0
    return h


_LOCK = threading.Lock()
_LIB: Optional[ctypes.CDLL] = None
_ERR: Optional[BaseException] = None


def library_path() -> Path:
    env = os.environ.get("CRESSO_HIP_LIBRARY")
    if env:
        return Path(env)
    return Path(__file__).resolve().with_name(LIB_NAME)


def _declare(lib: ctypes.CDLL) -> None:
    c = ctypes
    lib.cresso_hip_abi_version.restype = c.c_int32
    lib.cresso_hip_abi_version.argtypes = []
    lib.cresso_hip_last_error.restype = c.c_char_p
    lib.cresso_hip_last_error.argtypes = []
    lib.cresso_scalar_plan_create.restype = c.c_void_p
    lib.cresso_scalar_plan_create.argtypes = [c.POINTER(ScalarDesc), c.c_int32, c.POINTER(Hyper)]
    lib.cresso_scalar_plan_destroy.restype = None
    lib.cresso_scalar_plan_destroy.argtypes = [c.c_void_p]
    lib.cresso_scalar_plan_bytes.restype = c.c_size_t
    lib.cresso_scalar_plan_bytes.argtypes = [c.c_void_p]
    lib.cresso_scalar_plan_upload.restype = c.c_int32
    lib.cresso_scalar_plan_upload.argtypes = [c.c_void_p, c.c_void_p, c.c_size_t, c.c_void_p]
    lib.cresso_scalar_plan_step.restype = c.c_int32
    lib.cresso_scalar_plan_step.argtypes = [c.c_void_p, c.c_void_p, c.POINTER(c.c_void_p), c.POINTER(Hyper),
                                            c.c_void_p]
    lib.cresso_spectral_plan_create.restype = c.c_void_p
    lib.cresso_spectral_plan_create.argtypes = [c.POINTER(c.c_int64), c.c_int32, c.POINTER(c.c_int64), c.c_int32,
                                                c.c_int32, c.c_int32]
    lib.cresso_spectral_plan_create_ex.restype = c.c_void_p
    lib.cresso_spectral_plan_create_ex.argtypes = [c.POINTER(c.c_int64), c.c_int32, c.POINTER(c.c_int64), c.c_int32,
                                                   c.c_int32, c.c_int32, c.c_int32]
    lib.cresso_spectral_plan_destroy.restype = None
    lib.cresso_spectral_plan_destroy.argtypes = [c.c_void_p]
    lib.cresso_spectral_workspace_bytes.restype = c.c_size_t
    lib.cresso_spectral_workspace_bytes.argtypes = [c.c_void_p]
    lib.cresso_spectral_workspace_init.restype = c.c_int32
    lib.cresso_spectral_workspace_init.argtypes = [c.c_void_p, c.c_void_p, c.c_size_t, c.POINTER(Hyper), c.c_void_p]
    lib.cresso_spectral_step.restype = c.c_int32
    lib.cresso_spectral_step.argtypes = [c.c_void_p, c.POINTER(SpectralDesc), c.c_void_p, c.c_size_t,
                                         c.POINTER(Hyper), c.c_void_p]
    lib.cresso_spectral_batched_workspace_bytes.restype = c.c_size_t
    lib.cresso_spectral_batched_workspace_bytes.argtypes = [c.c_void_p, c.c_int32]
    lib.cresso_spectral_batched_workspace_init.restype = c.c_int32
    lib.cresso_spectral_batched_workspace_init.argtypes = [c.c_void_p, c.c_int32, c.c_void_p, c.c_size_t,
                                                           c.POINTER(Hyper), c.c_void_p]
    lib.cresso_spectral_step_batched.restype = c.c_int32
    lib.cresso_spectral_step_batched.argtypes = [c.c_void_p, c.POINTER(SpectralDesc), c.c_int32, c.c_void_p,
                                                 c.c_size_t, c.POINTER(Hyper), c.c_void_p]
    lib.cresso_spectral_step_noalloc.restype = c.c_int32
    lib.cresso_spectral_step_noalloc.argtypes = [c.c_void_p, c.POINTER(SpectralDesc), c.POINTER(Hyper), c.c_void_p]
    lib.cresso_spectral_workspace_bins.restype = c.c_int32
    lib.cresso_spectral_workspace_bins.argtypes = [c.c_void_p, c.c_void_p, c.c_size_t, c.c_void_p, c.c_void_p,
                                                   c.c_void_p]
    lib.cresso_spectral_workspace_project.restype = c.c_int32
    lib.cresso_spectral_workspace_project.argtypes = [c.c_void_p, c.c_void_p, c.c_size_t, c.c_void_p, c.c_void_p,
                                                      c.c_void_p]
    lib.cresso_spectral_workspace_reconstruct.restype = c.c_int32
    lib.cresso_spectral_workspace_reconstruct.argtypes = [c.c_void_p, c.c_void_p, c.c_size_t, c.c_void_p, c.c_void_p,
                                                          c.c_void_p, c.c_void_p, c.c_void_p]
    lib.cresso_spectral_workspace_gram.restype = c.c_int32
    lib.cresso_spectral_workspace_gram.argtypes = [c.c_void_p, c.c_void_p, c.c_size_t, c.c_void_p, c.c_void_p]
    vp, i32, i64, f64 = c.c_void_p, c.c_int32, c.c_int64, c.c_double
    lib.cresso_unit_workspace_bytes.restype = c.c_size_t
    lib.cresso_unit_workspace_bytes.argtypes = [i32]
    lib.cresso_hash_reduce_mean.restype = i32
    lib.cresso_hash_reduce_mean.argtypes = [vp, i64, i32, i32, vp, vp, c.c_size_t, vp]
    lib.cresso_hash_gather.restype = i32
    lib.cresso_hash_gather.argtypes = [vp, i32, i64, i32, vp, vp]
    lib.cresso_instant_axis_metric_2d_workspace_bytes.restype = c.c_size_t
    lib.cresso_instant_axis_metric_2d_workspace_bytes.argtypes = [i64, i64]
    lib.cresso_instant_axis_metric_2d.restype = i32
    lib.cresso_instant_axis_metric_2d.argtypes = [vp, i64, i64, f64, f64, f64, vp, vp, c.c_size_t, vp]
    lib.cresso_hash_metric_update_log.restype = i32
    lib.cresso_hash_metric_update_log.argtypes = [vp, i64, vp, i32, i32, i32, f64, f64, f64, f64, vp, vp, c.c_size_t, vp]
    lib.cresso_hash_impulse_update_gather.restype = i32
    lib.cresso_hash_impulse_update_gather.argtypes = [vp, i64, vp, vp, i32, i32, f64, f64, f64, vp, vp, c.c_size_t, vp]
    lib.cresso_metric_update.restype = i32
    lib.cresso_metric_update.argtypes = [vp, vp, vp, vp, vp, vp, vp, i32, f64, f64, vp]
    lib.cresso_confidence_update.restype = i32
    lib.cresso_confidence_update.argtypes = [vp, vp, vp, vp, vp, i32, f64, f64, vp]
    lib.cresso_contact_update_pair.restype = i32
    lib.cresso_contact_update_pair.argtypes = [vp, vp, vp, vp, vp, vp, vp, i32] + [f64] * 9 + [vp]
    lib.cresso_drive_update.restype = i32
    lib.cresso_drive_update.argtypes = [vp, i32, vp, vp, vp, vp, vp, vp, vp, i64, i32, i32, c.POINTER(Hyper), vp,
                                        c.c_size_t, vp]
    lib.cresso_spectral_workspace_basis.restype = c.c_int32
    lib.cresso_spectral_workspace_basis.argtypes = [c.c_void_p, c.c_void_p, c.c_size_t, c.c_int32, c.c_void_p,
                                                    c.c_void_p, c.c_void_p]


def load() -> ctypes.CDLL:
    """Load the HIP library once per process; raise RuntimeError if it cannot be used."""
    global _LIB, _ERR
    with _LOCK:
        if _LIB is not None:
            return _LIB
        if _ERR is not None:
            raise RuntimeError(f"CRESSO5 CUDA ops failed to load: {_ERR}") from _ERR
        path = library_path()
        try:
            if not path.exists():
                raise FileNotFoundError(f"{path} not found; build it with `python -m cresso_amd.build`")
            lib = ctypes.CDLL(str(path))
            _declare(lib)
            ver = int(lib.cresso_hip_abi_version())
            if ver != ABI_VERSION:
                raise RuntimeError(f"{path} has ABI version {ver}, expected {ABI_VERSION}")
        except Exception as exc:  # remembered: later calls fail the same way
            _ERR = exc
            raise RuntimeError(f"CRESSO5 CUDA ops failed to load: {exc}") from exc
        _LIB = lib
        return lib


_HB = None
_HB_TRIED = False


def host_batch():
    """The C++ host bookkeeping helper (cresso_amd/_hostbatch*.so), or None
    when it is not built (the Python loops then do the same work)."""
    global _HB, _HB_TRIED
    if not _HB_TRIED:
        _HB_TRIED = True
        try:
            from . import _hostbatch as hb  # type: ignore[attr-defined]
            _HB = hb
        except ImportError:
            _HB = None
    return _HB


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = (_LIB.cresso_hip_last_error() or b"").decode(errors="replace") if _LIB is not None else ""
        raise RuntimeError(f"CRESSO5 {what} failed ({rc}): {msg}")


def stream_handle(device: torch.device) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)
