"""CPU restatement of CRESSO5's ``cuda_ops="off"`` step (TEST INFRASTRUCTURE ONLY).

This module is the parity oracle.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it, and only as the
checker / the timed CPU baseline.  The shipped optimizer in ``cresso_amd`` never
imports it and has no CPU fallback.

It restates, with torch CPU ops in the work dtype (fp32 for fp16/bf16/fp32
params), the algorithm of the reference's PyTorch path
(``/root/reference/cresso_v5.py``; every function cites the lines it follows).
Evaluation order of the fp32 expressions follows the reference so that the
restatement reproduces its rounding (golden fixtures pin it; see
``tests/test_oracle_golden.py``).

Pinning of each part (what would catch a plausible mistake):
  * hash index / counts      -- golden vectors from the reference, a C
                                restatement (``oracle/hash_oracle.c``) and a
                                Python big-integer restatement; counts sum to n.
  * _hash_unit               -- golden vectors (through the basis fixtures) and
                                a 32-bit masked big-int recomputation.
  * frequency pack / omega   -- golden vectors for 7 (rank, ndim, F) triples.
  * basis pairs              -- golden vectors (incl. the degenerate 3-wide
                                axis case), plus invariants (zero mean, unit rms).
  * project / reconstruct    -- golden vectors; fp64 brute force dot products;
                                linearity.
  * spectral / scalar step   -- golden multi-step trajectories (params + every
                                state tensor) from the reference.
  * reservoir                -- known answers 3.0 then 4.0.
  * micro route              -- golden trajectory (one fixture).
  * unit operations          -- hash_metric_update_log, hash_impulse_update_gather,
                                metric_update, confidence_update,
                                contact_update_pair are the pieces the spectral
                                step calls, so the trajectories pin them.

One deliberate difference from the reference's PyTorch path: the alignment
gate's predicate sqrt(mean(pred^2) + eps) > sqrt(eps) (cresso_v5.py:1307,
1554) is decided in fp64, as the reference's fused kernels decide it.  In
fp32 it is a rounding tie whenever mean(pred^2) is below half an fp32 ulp of
eps, and torch's CPU result then differs between hosts (see _drive_apply).
The update of fp16/bf16 params keeps the reference's torch call
p.add_(u, alpha=-lr), whose CPU kernel rounds alpha to the param dtype.
"""

from __future__ import annotations

import math
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

Tensor = torch.Tensor

# Hyperparameter defaults of CRESSO5.__init__ (cresso_v5.py:621-681).
DEFAULTS: Dict[str, object] = dict(
    lr=2.0e-3, rank=8, max_frequency=5, weight_decay=0.0, energy_power=1.20,
    dt=0.15, impulse_friction=0.18, contact_gain=0.16, restoring=0.62,
    cubic=0.006, metric_dt=0.09, metric_friction=0.22, metric_coupling=0.36,
    local_sharpness=0.0, instant_metric_coupling=0.55, instant_metric_power=1.0,
    root_channel_mix=0.16, echo_mix=0.06, transport_mix=0.18, hash_bins=128,
    hash_tables=2, hash_decay=0.92, hash_impulse_decay=0.78,
    hash_metric_coupling=0.42, hash_drive_mix=0.22, direct_force_mix=0.18,
    residual_feedback_mix=0.06, micro_field_max_size=0, micro_decay=0.94,
    micro_impulse_decay=0.82, micro_drive_mix=0.35, reservoir_decay=0.95,
    refractory_decay=0.90, refractory_gain=0.55, confidence_decay=0.92,
    confidence_gain=0.50, surprise_gain=0.18, surprise_decay=0.95,
    prediction_mix=0.16, novelty_mix=0.04, warmup_steps=10,
    surprise_brake=0.18, target_update_rms=1.0, min_gain=0.04, max_gain=6.0,
    drive_clip=4.0, spike_mix=0.25, min_spectral_size=1024,
    basis_cache_limit_elements=2_000_000, hard_channel_min_size=16,
    thin_matrix_hard_cutoff=8, thin_matrix_max_width=64,
    thin_matrix_min_aspect=4.0, thin_matrix_route="scalar", maximize=False,
    eps=1e-8,
)


def work_dtype(dtype: torch.dtype) -> torch.dtype:
    """fp16/bf16 compute in fp32 (cresso_v5.py:119-124)."""
    return torch.float32 if dtype in (torch.float16, torch.bfloat16) else dtype


# --------------------------------------------------------------------------
# Integer / host helpers
# --------------------------------------------------------------------------

def hash_unit(n: int, salt: int = 0) -> float:
    """32-bit mixer to [0,1) (cresso_v5.py:127-135).

    The first product is *not* masked before the first xor-shift: Python ints
    are unbounded there, exactly as in the reference.
    """
    v = (n + 1) * 0x9E3779B1 + (salt + 11) * 0x85EBCA77
    v = v ^ (v >> 16)
    v = (v * 0x7FEB352D) & 0xFFFFFFFF
    v = v ^ (v >> 15)
    v = (v * 0x846CA68B) & 0xFFFFFFFF
    v = v ^ (v >> 16)
    return float(v & 0xFFFFFF) / 16777216.0


def frequency_pack(rank: int, ndim: int, max_frequency: int) -> List[Tuple[int, ...]]:
    """Deterministic mode list (cresso_v5.py:145-227) as Python tuples."""
    rank = int(rank)
    ndim = int(ndim)
    fmax = max(0, int(max_frequency))
    if rank <= 0:
        return []
    zero = tuple([0] * ndim)
    if fmax <= 0:
        return [zero] * rank
    modes = [zero]
    seen = {zero}

    def structured():
        for f in range(1, fmax + 1):                     # axis-local
            for a in range(ndim):
                yield tuple(f if i == a else 0 for i in range(ndim))
        for f in range(1, fmax + 1):                     # diagonal / anti-diagonal
            yield tuple([f] * ndim)
            if ndim > 1:
                yield tuple(f if i % 2 == 0 else max(1, fmax + 1 - f) for i in range(ndim))
        if ndim > 1:                                     # sparse pairs
            for f1 in range(1, fmax + 1):
                for f2 in range(1, fmax + 1):
                    for a in range(ndim):
                        v = [0] * ndim
                        v[a] = f1
                        v[(a + 1) % ndim] = f2
                        yield tuple(v)

    for cand in structured():
        if cand not in seen:
            modes.append(cand)
            seen.add(cand)
        if len(modes) >= rank:
            return modes[:rank]

    primes = (2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37)
    counter = 1
    tries = 0
    guard = max(64, 10 * rank * max(1, ndim))
    while len(modes) < rank:
        v = [(counter * primes[a % 12] + a * a + 3 * a + 1) % (fmax + 1) for a in range(ndim)]
        active = sum(1 for x in v if x != 0)
        if active == 0:
            v[counter % ndim] = 1 + (counter % fmax)
        elif active == 1 and ndim > 1:
            v[(counter + 1) % ndim] = 1 + ((counter // 2) % fmax)
        cand = tuple(v)
        if cand not in seen or tries >= guard:
            modes.append(cand)
            seen.add(cand)
        counter += 1
        tries += 1
    return modes[:rank]


def make_freqs(rank: int, ndim: int, max_frequency: int) -> Tensor:
    modes = frequency_pack(rank, ndim, max_frequency)
    if not modes:
        return torch.empty((0, ndim), dtype=torch.long)
    return torch.tensor(modes, dtype=torch.long)


def omega_from_freqs(freqs: Tensor) -> Tensor:
    """omega = sqrt(1 + sum f^2) in fp32 (cresso_v5.py:230-234)."""
    if freqs.numel() == 0:
        return torch.empty((0,), dtype=torch.float32)
    f = freqs.to(torch.float32)
    return 1.0 * torch.sqrt(1.0 + (f * f).sum(dim=1))


def hash_index_np(n: int, bins: int, salt: int) -> np.ndarray:
    """Coordinate hash bins over linear indices 0..n-1 (cresso_v5.py:495-516).

    int64 two's-complement wrap, arithmetic right shifts, floor-mod.
    """
    if bins <= 0:
        return np.empty((n,), dtype=np.int64)
    s = int(salt) + 1

    def w(c: int) -> np.int64:
        c &= 0xFFFFFFFFFFFFFFFF
        return np.int64(c - (1 << 64) if c >= (1 << 63) else c)

    with np.errstate(over="ignore"):
        h = np.arange(n, dtype=np.int64)
        h = h * w(1103515245 + 97 * s) + w(12345 + 0x9E3779B1 * s)
        h ^= h >> np.int64(16)
        h = h * w(2246822519 + 1315423911 * s)
        h ^= h >> np.int64(13)
        h = h * w(3266489917 + 374761393 * s)
        h ^= h >> np.int64(16)
    return np.mod(h, np.int64(bins))


def hash_index(shape: Sequence[int], bins: int, salt: int) -> Tensor:
    n = int(np.prod([int(d) for d in shape])) if len(shape) else 1
    return torch.from_numpy(hash_index_np(n, bins, salt)).view(tuple(int(d) for d in shape))


def hash_counts_np(n: int, bins: int, salt: int) -> np.ndarray:
    return np.bincount(hash_index_np(n, bins, salt), minlength=bins).astype(np.int64)


def hash_reduce_mean(x: Tensor, idx: Tensor, bins: int, accum: str = "native") -> Tensor:
    """Bin mean by sequential scatter_add in x's dtype (cresso_v5.py:519-526).

    accum="fp64" accumulates in float64 and rounds the means to x's dtype: the
    tie-breaker for tensors whose bins hold so many elements that the
    reference's own fp32 accumulation error (~sqrt(count) ulp, 3.8e-5
    relative at 262144 elements per bin) exceeds the parity tolerance.
    """
    if accum == "fp64" and x.dtype != torch.float64:
        return hash_reduce_mean(x.double(), idx, bins).to(x.dtype)
    fi = idx.reshape(-1)
    fx = x.reshape(-1)
    total = torch.zeros(int(bins), dtype=x.dtype).scatter_add_(0, fi, fx)
    count = torch.zeros(int(bins), dtype=x.dtype).scatter_add_(0, fi, torch.ones_like(fx))
    return total / count.clamp_min(1.0)


# --------------------------------------------------------------------------
# Routing and the state-size contract
# --------------------------------------------------------------------------

def lora_thin(shape: Sequence[int], max_width: int = 64, min_aspect: float = 4.0) -> bool:
    """cresso_v5.py:545-557."""
    dims = tuple(int(d) for d in shape)
    if len(dims) != 2 or int(max_width) <= 0:
        return False
    lo, hi = min(dims), max(dims)
    if lo <= 0:
        return False
    return lo <= int(max_width) and (hi / lo) >= float(min_aspect)


def thin_uses_scalar(shape, route="scalar", max_width=64, min_aspect=4.0) -> bool:
    """cresso_v5.py:538-542, 560-570."""
    r = str(route).lower()
    if r not in ("scalar", "spectral"):
        raise ValueError("thin_matrix_route must be one of 'scalar' or 'spectral'")
    return r == "scalar" and lora_thin(shape, max_width, min_aspect)


def theoretical_state_elements(shape, rank, spectral=True, hash_bins=128, hash_tables=2,
                               micro_field_max_size=0, hard_channel_min_size=16,
                               thin_matrix_hard_cutoff=8, thin_matrix_max_width=64,
                               thin_matrix_min_aspect=4.0, thin_matrix_route="scalar") -> int:
    """cresso_v5.py:573-609."""
    dims = tuple(int(d) for d in shape)
    n = int(np.prod(dims)) if dims else 1
    if int(micro_field_max_size) > 0 and n <= int(micro_field_max_size) and len(dims) > 0:
        return 3 * n + 4
    if bool(spectral) and not thin_uses_scalar(dims, thin_matrix_route, thin_matrix_max_width,
                                               thin_matrix_min_aspect):
        thin = len(dims) == 2 and int(thin_matrix_hard_cutoff) > 0 and min(dims) <= int(thin_matrix_hard_cutoff)
        hard = n >= int(hard_channel_min_size) and not thin
        return int(rank) * len(dims) + 12 * int(rank) + (3 * int(hash_bins) * int(hash_tables) if hard else 0) + 4
    return 8


# --------------------------------------------------------------------------
# Dense basis (cresso_v5.py:237-376)
# --------------------------------------------------------------------------

def axis_coord(dim: int, dtype: torch.dtype) -> Tensor:
    """u_k = (k + 1/2)/dim in the work dtype (cresso_v5.py:237-239)."""
    return (torch.arange(dim, dtype=dtype) + 0.5) / float(dim)


def _axis_view(t: Tensor, ndim: int, axis: int) -> Tensor:
    shape = [1] * ndim
    shape[axis] = t.numel()
    return t.view(shape)


def additive_phase(shape, freqs: Tensor, r: int, dtype, chirp: bool) -> Tensor:
    """Sum over axes of pi*f*u (+ chirp term), fp32 (cresso_v5.py:272-292)."""
    nd = len(shape)
    acc: Optional[Tensor] = None
    for a, dim in enumerate(shape):
        f = int(freqs[r, a]) if freqs.numel() else 0
        if f == 0 and not chirp:
            continue
        u = axis_coord(int(dim), dtype)
        part = (math.pi * float(f)) * u
        if chirp:
            c = 0.25 + 1.75 * hash_unit(r, 17 + a)
            part = part + (math.pi * c * float(max(1, f))) * (u - 0.5).pow(2)
        part = _axis_view(part, nd, a)
        acc = part if acc is None else acc + part
    if acc is None:
        return torch.zeros(tuple(shape), dtype=dtype)
    return acc.expand(tuple(shape))


def normalize_basis(x: Tensor) -> Tensor:
    """(x - mean)/max(sqrt(mean (x-mean)^2 + 1e-12), 1e-6) (cresso_v5.py:138-142)."""
    x = x - x.mean()
    rms = torch.sqrt(x.pow(2).mean() + 1e-12)
    return x / rms.clamp_min(1e-6)


def basis_pair(shape, freqs: Tensor, r: int, dtype) -> Tuple[Tensor, Tensor]:
    """Normalized (cos, sin) carrier of mode r (cresso_v5.py:295-348)."""
    shape = tuple(int(d) for d in shape)
    nd = len(shape)
    if (int(freqs[r].abs().sum()) if freqs.numel() else 0) == 0:
        return torch.ones(shape, dtype=dtype), torch.zeros(shape, dtype=dtype)
    kind = r % 4
    if kind == 1:
        cprod: Optional[Tensor] = None
        sprod: Optional[Tensor] = None
        for a, dim in enumerate(shape):
            f = int(freqs[r, a])
            if f == 0:
                continue
            ph = (math.pi * float(f)) * axis_coord(dim, dtype)
            c = _axis_view(torch.cos(ph), nd, a)
            s = _axis_view(torch.sin(ph), nd, a)
            cprod = c if cprod is None else cprod * c
            sprod = s if sprod is None else sprod * s
        return normalize_basis(cprod.expand(shape)), normalize_basis(sprod.expand(shape))
    phase = additive_phase(shape, freqs, r, dtype, chirp=(kind != 0))
    if kind != 3:
        return normalize_basis(torch.cos(phase)), normalize_basis(torch.sin(phase))
    win: Optional[Tensor] = None
    for a, dim in enumerate(shape):
        u = axis_coord(dim, dtype)
        mu = 0.15 + 0.70 * hash_unit(r, 101 + a)
        sig = 0.18 + 0.20 * hash_unit(r, 151 + a)
        w = _axis_view(torch.exp(-0.5 * ((u - mu) / sig).pow(2)), nd, a)
        win = w if win is None else win * w
    win = win.expand(shape)
    return normalize_basis(win * torch.cos(phase)), normalize_basis(win * torch.sin(phase))


def _shrink(rank: int) -> float:
    return 1.0 / math.sqrt(max(1.0, 0.7 * math.log2(rank + 1.0)))


class BasisSource:
    """Per-step basis provider: a dense list when 2*R*n fits the cache limit
    (cresso_v5.py:380-415, CPU branch), else rebuilt on every use
    (cresso_v5.py:351-376)."""

    def __init__(self, shape, freqs: Tensor, rank: int, dtype, cache_limit: int):
        self.shape = tuple(int(d) for d in shape)
        self.freqs = freqs
        self.rank = rank
        self.dtype = dtype
        n = int(np.prod(self.shape))
        self.pairs = None
        if int(cache_limit) > 0 and 2 * rank * n <= int(cache_limit):
            self.pairs = [basis_pair(self.shape, freqs, r, dtype) for r in range(rank)]

    def pair(self, r: int) -> Tuple[Tensor, Tensor]:
        if self.pairs is not None:
            return self.pairs[r]
        return basis_pair(self.shape, self.freqs, r, self.dtype)

    def project(self, x: Tensor) -> Tuple[Tensor, Tensor]:
        """(mean(x*C_r), mean(x*S_r)) per mode (cresso_v5.py:351-359, 418-443)."""
        cc = torch.empty(self.rank, dtype=x.dtype)
        sc = torch.empty(self.rank, dtype=x.dtype)
        for r in range(self.rank):
            bc, bs = self.pair(r)
            cc[r] = (x * bc).mean()
            sc[r] = (x * bs).mean()
        return cc, sc

    def reconstruct(self, cc: Tensor, sc: Tensor, gates: Optional[Tensor] = None) -> Tensor:
        """shrink * sum_r g_r (cc_r C_r + sc_r S_r), accumulated with add_(alpha)
        in mode order; a gate of exactly 0 skips the mode (cresso_v5.py:362-376)."""
        rank = int(cc.numel())
        out = torch.zeros(self.shape, dtype=self.dtype)
        if rank == 0:
            return out
        k = _shrink(rank)
        for r in range(rank):
            g = 1.0 if gates is None else float(gates[r])
            if g == 0.0:
                continue
            bc, bs = self.pair(r)
            out.add_(bc, alpha=float(cc[r]) * k * g)
            out.add_(bs, alpha=float(sc[r]) * k * g)
        return out


# --------------------------------------------------------------------------
# Field helpers
# --------------------------------------------------------------------------

def instant_axis_metric(rel: Tensor, power: float, coupling: float, eps: float) -> Tensor:
    """Per-axis marginal-density metric (cresso_v5.py:243-262)."""
    if coupling == 0.0 or rel.ndim == 0 or rel.numel() <= 1:
        return torch.ones_like(rel)
    nd = rel.ndim
    p = max(float(power), 0.25)
    dens = rel.clamp_min(eps).pow(p).clamp(max=1.0e6)
    logm: Optional[Tensor] = None
    for a in range(nd):
        others = tuple(i for i in range(nd) if i != a)
        m = dens.mean(dim=others, keepdim=True) if others else dens
        m = m / m.mean().clamp_min(eps)
        term = torch.log(m.clamp_min(eps))
        logm = term if logm is None else logm + term
    return torch.exp((float(coupling) / (nd * p)) * logm).clamp(0.08, 12.0)


def rms_normalize(x: Tensor, target, eps: float) -> Tensor:
    """x * target / max(rms(x), eps) (cresso_v5.py:265-269)."""
    rms = torch.sqrt(x.pow(2).mean() + eps)
    if torch.is_tensor(target):
        return x * (target.to(dtype=x.dtype) / rms.clamp_min(eps))
    return x * (float(target) / rms.clamp_min(eps))


def reservoir(old: Tensor, cur: Tensor, decay: float, step: int) -> Tensor:
    """In-place EMA, copy on the first step (cresso_v5.py:900-905)."""
    if step <= 1:
        old.copy_(cur.detach().to(dtype=old.dtype))
    else:
        old.mul_(float(decay)).add_(cur.detach().to(dtype=old.dtype), alpha=1.0 - float(decay))
    return old


# --------------------------------------------------------------------------
# The optimizer restatement
# --------------------------------------------------------------------------

# --------------------------------------------------------------------------
# Unit operations of the spectral step (each is one op of the reference's
# fused CUDA path, cresso_cuda.cpp:44-125; the step below calls them)
# --------------------------------------------------------------------------

def hash_metric_update_log(dsrc: Tensor, energy: Tensor, idx: Tensor, bins: int, step: int, h: dict, dtype,
                           accum: str = "native") -> Tensor:
    """One table of the hash metric (cresso_v5.py:1014-1026; the reference op
    hash_metric_update_log_cuda, cresso_cuda_kernel.cu:1515-1591): bin means of
    the density source, EMA into ``energy`` (this table's row of hash_energy,
    copied on step <= 1, in place), normalized by its mean, raised to
    coupling / max(0.25, energy_power), gathered per element, clamped to
    [0.08, 12] and logged.  -> per-element log term."""
    eps = float(h["eps"])
    cell = hash_reduce_mean(dsrc, idx, bins, accum)
    if step <= 1:
        energy.copy_(cell.to(energy.dtype))
    else:
        energy.mul_(float(h["hash_decay"])).add_(cell.to(energy.dtype), alpha=1.0 - float(h["hash_decay"]))
    hm = (energy.to(dtype) / energy.to(dtype).mean().clamp_min(eps)).clamp_min(eps)
    hmp = hm.pow(float(h["hash_metric_coupling"]) / max(0.25, float(h["energy_power"])))
    return torch.log(hmp[idx].clamp(0.08, 12.0).clamp_min(eps))


def hash_impulse_update_gather(psrc: Tensor, refractory: Tensor, impulse: Tensor, idx: Tensor, bins: int, h: dict,
                               dtype, accum: str = "native") -> Tensor:
    """One table of the hash impulse (cresso_v5.py:1153-1160; the reference op
    hash_impulse_update_gather_cuda, cresso_cuda_kernel.cu:1593-1661): bin means
    of the port source, refractory EMA of their magnitude (no first-step copy),
    gate 1/(1 + refractory_gain * refractory), impulse EMA of mean * gate (both
    rows in place), gathered per element.  -> per-element impulse."""
    cp = hash_reduce_mean(psrc, idx, bins, accum).to(impulse.dtype)
    refractory.mul_(float(h["hash_decay"])).add_(cp.abs(), alpha=1.0 - float(h["hash_decay"]))
    gate = 1.0 / (1.0 + float(h["refractory_gain"]) * refractory)
    impulse.mul_(float(h["hash_impulse_decay"])).add_(cp * gate, alpha=1.0 - float(h["hash_impulse_decay"]))
    return impulse.to(dtype)[idx]


def metric_update(mq_cos: Tensor, mq_sin: Tensor, mp_cos: Tensor, mp_sin: Tensor, port_cos: Tensor,
                  port_sin: Tensor, omega: Tensor, metric_dt: float, metric_friction: float) -> None:
    """Metric oscillator of both banks, in place (cresso_v5.py:1064-1088; the
    reference op metric_update_cuda, cresso_cuda_kernel.cu:1368-1395)."""
    for mq, mp, port in ((mq_cos, mp_cos, port_cos), (mq_sin, mp_sin, port_sin)):
        mp.mul_(max(0.0, 1.0 - metric_dt * metric_friction))
        mp.add_(port - (omega * omega) * mq, alpha=metric_dt)
        mq.add_(mp, alpha=metric_dt)
        mq.clamp_(-3.0, 3.0)


def confidence_update(conf: Tensor, pcp: Tensor, psp: Tensor, qc: Tensor, qs: Tensor, decay: float,
                      eps: float) -> None:
    """Mode confidence, in place (cresso_v5.py:1199-1202 and the PyTorch branch
    that follows; the reference op confidence_update_cuda,
    cresso_cuda_kernel.cu:1397-1421).  Uses the pre-contact q."""
    pe = torch.sqrt(pcp.pow(2) + psp.pow(2) + eps)
    support = (pcp * qc + psp * qs) / (pe * torch.sqrt(qc.pow(2) + qs.pow(2) + eps) + eps)
    conf.mul_(decay).add_(support.clamp(-1.0, 1.0), alpha=1.0 - decay)
    conf.clamp_(-4.0, 4.0)


def contact_update_pair(q: Tensor, pm: Tensor, port: Tensor, omega: Tensor, calcium: Tensor, action: Tensor,
                        surprise: Tensor, h: dict) -> Tensor:
    """Contact oscillator of one (cos | sin) bank, in place
    (cresso_v5.py:914-943; the reference op contact_update_pair_cuda,
    cresso_cuda_kernel.cu:1423-1498).  -> the updated action (same tensor)."""
    rank = int(q.numel())
    dt = float(h["dt"])
    rd = float(h["refractory_decay"])
    calcium.mul_(rd).add_(port.abs(), alpha=1.0 - rd)
    gate = 1.0 / (1.0 + float(h["refractory_gain"]) * calcium)
    sur = surprise.to(q.dtype)
    plast = 1.0 + float(h["surprise_gain"]) * sur / (1.0 + sur)
    brake = 1.0 / (1.0 + float(h["surprise_brake"]) * sur)
    gp = port * gate * plast * brake
    energy = 0.5 * (pm.pow(2).mean() + ((omega * q).pow(2)).mean()) if rank > 0 else torch.zeros_like(action)
    power = (gp * pm).mean() if rank > 0 else torch.zeros_like(action)
    action.mul_(0.985).add_((power - energy).to(action.dtype), alpha=dt)
    fr = float(h["impulse_friction"]) + float(h["contact_gain"]) * torch.tanh(action.abs()).to(pm.dtype)
    pm.mul_(torch.clamp(1.0 - dt * fr, min=0.0))
    pm.add_(gp - float(h["restoring"]) * (omega * omega) * q - float(h["cubic"]) * q.pow(3), alpha=dt)
    q.add_(pm, alpha=dt)
    q.clamp_(-8.0, 8.0)
    return action


class OracleCRESSO5:
    """CRESSO5 with ``cuda_ops="off"`` on CPU tensors.

    ``params`` are CPU tensors (leaf tensors with ``.grad`` set, or plain
    tensors with ``grads`` passed to :meth:`step`).  ``state[i]`` is the state
    dict of params[i] with the reference's keys, shapes and dtypes
    (cresso_v5.py:857-898).
    """

    def __init__(self, params: Sequence[Tensor], hash_accum: str = "native", **kwargs):
        """hash_accum: "native" (the reference's fp32 scatter_add, default) or
        "fp64" (the tie-breaker described at hash_reduce_mean)."""
        unknown = set(kwargs) - set(DEFAULTS) - {"cuda_ops"}
        if unknown:
            raise TypeError(f"unknown hyperparameters {sorted(unknown)}")
        self.hash_accum = hash_accum
        self.h = dict(DEFAULTS)
        self.h.update({k: v for k, v in kwargs.items() if k != "cuda_ops"})
        self.params = list(params)
        self.state: List[dict] = [dict() for _ in self.params]

    # -- routing (cresso_v5.py:839-855) --
    def route(self, p: Tensor) -> str:
        h = self.h
        if int(h["micro_field_max_size"]) > 0 and p.ndim > 0 and p.numel() <= int(h["micro_field_max_size"]):
            return "micro"
        if p.numel() >= int(h["min_spectral_size"]) and int(h["rank"]) > 0 and p.ndim > 0 and not thin_uses_scalar(
                tuple(p.shape), h["thin_matrix_route"], h["thin_matrix_max_width"], h["thin_matrix_min_aspect"]):
            return "spectral"
        return "scalar"

    @torch.no_grad()
    def step(self, grads: Optional[Sequence[Tensor]] = None) -> None:
        for i, p in enumerate(self.params):
            g = grads[i] if grads is not None else p.grad
            if g is None or not torch.is_floating_point(p):
                continue
            g = g.detach()
            if self.h["maximize"]:
                g = -g
            r = self.route(p)
            if r == "micro":
                self._micro(p, g, self.state[i])
            elif r == "spectral":
                self._spectral(p, g, self.state[i])
            else:
                self._scalar(p, g, self.state[i])

    # -- state init (cresso_v5.py:857-898) --
    @staticmethod
    def _common(st: dict, dtype) -> None:
        st["step"] = 0
        st["force_rms"] = torch.zeros((), dtype=dtype)
        st["drive_energy"] = torch.ones((), dtype=dtype)
        st["surprise"] = torch.zeros((), dtype=dtype)
        st["action"] = torch.zeros((), dtype=dtype)

    def _init_spectral(self, p: Tensor, st: dict, dtype) -> None:
        h = self.h
        self._common(st, dtype)
        rank = int(h["rank"])
        freqs = make_freqs(rank, p.ndim, int(h["max_frequency"]))
        st["freqs"] = freqs
        st["omega"] = omega_from_freqs(freqs).to(dtype=dtype)
        for k in ("q_cos", "q_sin", "p_cos", "p_sin", "metric_cos", "metric_sin", "metric_p_cos",
                  "metric_p_sin", "calcium_cos", "calcium_sin", "mode_confidence"):
            st[k] = torch.zeros(rank, dtype=dtype)
        bins, tables = int(h["hash_bins"]), int(h["hash_tables"])
        cut = int(h["thin_matrix_hard_cutoff"])
        thin = p.ndim == 2 and cut > 0 and min(p.shape) <= cut
        if bins > 0 and p.numel() >= int(h["hard_channel_min_size"]) and not thin:
            st["hash_energy"] = torch.ones(tables, bins, dtype=dtype)
            st["hash_impulse"] = torch.zeros(tables, bins, dtype=dtype)
            st["hash_refractory"] = torch.zeros(tables, bins, dtype=dtype)

    def _force(self, p: Tensor, g: Tensor, dtype) -> Tensor:
        f = g.to(dtype=dtype)
        wd = float(self.h["weight_decay"])
        if wd != 0.0:
            f = f + wd * p.detach().to(dtype=dtype)
        return f

    def _contact(self, q, pm, port, omega, calcium, action, surprise, rank) -> Tensor:
        """Contact oscillator for one (cos|sin) bank (cresso_v5.py:914-943)."""
        return contact_update_pair(q, pm, port, omega, calcium, action, surprise, self.h)

    def _spectral(self, p: Tensor, g: Tensor, st: dict) -> None:
        """Spectral/hash large-tensor route (cresso_v5.py:945-1353, PyTorch branch)."""
        h = self.h
        dtype = work_dtype(p.dtype)
        if len(st) == 0:
            self._init_spectral(p, st, work_dtype(dtype))
        st["step"] += 1
        step = int(st["step"])
        eps = float(h["eps"])
        shape = tuple(p.shape)

        force = self._force(p, g, dtype)
        now = torch.sqrt(force.pow(2).mean() + eps)
        st["force_rms"] = reservoir(st["force_rms"], now, h["reservoir_decay"], step)
        scale = st["force_rms"].to(dtype).clamp_min(eps)

        freqs = st["freqs"]
        rank = int(st["omega"].numel())
        omega = st["omega"].to(dtype=st["q_cos"].dtype)
        basis = BasisSource(shape, freqs, rank, dtype, int(h["basis_cache_limit_elements"]))
        cut = int(h["thin_matrix_hard_cutoff"])
        thin = p.ndim == 2 and cut > 0 and min(shape) <= cut
        hard = p.numel() >= int(h["hard_channel_min_size"]) and not thin

        rel = (force.abs() / scale + eps).clamp(max=1.0e4)
        bins = int(h["hash_bins"])
        tables = int(h["hash_tables"])
        hash_idx: Optional[List[Tensor]] = None
        hash_metric = 1.0
        hash_pred = 0.0
        dsrc: Optional[Tensor] = None
        if hard and bins > 0 and "hash_energy" in st:
            hash_idx = []
            dsrc = rel.pow(float(h["energy_power"]))
            logsum: Optional[Tensor] = None
            for t in range(tables):
                idx = hash_index(shape, bins, t)
                hash_idx.append(idx)
                term = hash_metric_update_log(dsrc, st["hash_energy"][t], idx, bins, step, h, dtype, self.hash_accum)
                logsum = term if logsum is None else logsum + term
            hash_metric = torch.exp(logsum / float(tables)).clamp(0.08, 12.0)
        if dsrc is None:
            dsrc = rel.pow(float(h["energy_power"]))
        dens = torch.log1p(dsrc)
        dens = dens / dens.mean().clamp_min(eps) - 1.0
        mcp, msp = basis.project(dens)
        mcp = mcp.to(st["metric_cos"].dtype)
        msp = msp.to(st["metric_sin"].dtype)
        metric_update(st["metric_cos"], st["metric_sin"], st["metric_p_cos"], st["metric_p_sin"], mcp, msp, omega,
                      float(h["metric_dt"]), float(h["metric_friction"]))

        logm = basis.reconstruct(st["metric_cos"].to(dtype), st["metric_sin"].to(dtype)).clamp(-3.0, 3.0)
        metric = torch.exp(float(h["metric_coupling"]) * logm).clamp(0.06, 16.0)
        ls = float(h["local_sharpness"])
        local = (1.0 + ls * torch.sqrt(rel.clamp(max=100.0))).clamp(1.0, 8.0) if ls != 0.0 else 1.0
        icoup = float(h["instant_metric_coupling"]) if hard else 0.0
        inst = instant_axis_metric(rel, float(h["instant_metric_power"]), icoup, eps)
        tangent = (force / (scale * metric * local * inst * hash_metric + eps)).clamp(-1.0e4, 1.0e4)

        qc, qs, conf = st["q_cos"], st["q_sin"], st["mode_confidence"]
        gates = torch.sigmoid(float(h["confidence_gain"]) * conf).to(dtype)
        pred = basis.reconstruct(qc.to(dtype), qs.to(dtype), gates)
        err = tangent - pred
        sur_now = torch.sqrt(err.pow(2).mean() + eps)
        st["surprise"] = reservoir(st["surprise"], sur_now, h["surprise_decay"], step)
        surprise = st["surprise"]

        psrc = err + float(h["transport_mix"]) * tangent
        pcp, psp = basis.project(psrc)
        pcp = pcp.to(qc.dtype)
        psp = psp.to(qs.dtype)

        if hash_idx is not None and "hash_impulse" in st:
            acc: Optional[Tensor] = None
            for t, idx in enumerate(hash_idx):
                got = hash_impulse_update_gather(psrc, st["hash_refractory"][t], st["hash_impulse"][t], idx, bins, h,
                                                 dtype, self.hash_accum)
                acc = got if acc is None else acc + got
            hash_pred = acc / float(len(hash_idx))

        confidence_update(conf, pcp, psp, qc, qs, float(h["confidence_decay"]), eps)

        action = st["action"]
        action = self._contact(qc, st["p_cos"], pcp, omega, st["calcium_cos"], action, surprise, rank)
        st["action"] = self._contact(qs, st["p_sin"], psp, omega, st["calcium_sin"], action, surprise, rank)

        gates = torch.sigmoid(float(h["confidence_gain"]) * conf).to(dtype)
        pred = basis.reconstruct(qc.to(dtype), qs.to(dtype), gates)
        err = tangent - pred
        echo_raw: Optional[Tensor] = None
        if hard and float(h["echo_mix"]) != 0.0:
            ec, es = basis.project(tangent)
            echo_raw = basis.reconstruct(ec, es)
        self._drive_apply(p, st, tangent, pred, err, echo_raw, hash_pred, hard, step, dtype, spectral=True)

    def _drive_apply(self, p, st, tangent, pred, err, echo_raw, hash_pred, hard, step, dtype, spectral):
        """Drive shaping, drive-energy reservoir and update.

        Spectral: cresso_v5.py:1303-1353.  Scalar: cresso_v5.py:1550-1582
        (root mix always on, no echo/hash terms, direct force via rms_normalize).
        """
        h = self.h
        eps = float(h["eps"])
        frms = torch.sqrt(tangent.pow(2).mean() + eps)
        prms = torch.sqrt(pred.pow(2).mean() + eps)
        align = ((tangent * pred).mean() / (frms * prms + eps)).clamp(-1.0, 1.0)
        # The gate's predicate prms > sqrt(eps) (cresso_v5.py:1307, 1554) is
        # decided in fp64, as the reference's fused kernels decide it
        # (cresso_cuda_kernel.cu:2080-2085, 2703-2708).  Evaluated in fp32 it
        # is a rounding tie whenever mean(pred^2) is below half an fp32 ulp of
        # eps (a nonzero but tiny prediction, e.g. C3 tensors whose force RMS
        # is eps-dominated), and torch's CPU result then differs between hosts
        # (observed: True on the GPU box's EPYC host, False in this container,
        # for the same inputs).
        pm2 = float(pred.double().pow(2).mean())
        agate = torch.where(torch.tensor(math.sqrt(pm2 + eps) > math.sqrt(eps)),
                            ((align + 1.0) * 0.5).clamp(0.0, 1.0), torch.zeros((), dtype=dtype))
        ws = int(h["warmup_steps"])
        warm = 1.0 if ws == 0 else (1.0 - math.exp(-step / max(1, ws)))
        sur = st["surprise"].to(dtype)
        if spectral:
            mix = float(h["prediction_mix"]) * warm * agate * (1.0 / (1.0 + sur))
        else:
            mix = float(h["prediction_mix"]) * warm * agate / (1.0 + sur)
        clip = float(h["drive_clip"])
        bnd = torch.tanh(tangent / clip) * clip
        rat = tangent / (1.0 + tangent.abs() / clip)
        root = tangent.sign() * torch.sqrt(tangent.abs().clamp(max=clip * clip) + eps)
        root = rms_normalize(root, torch.sqrt(rat.pow(2).mean() + eps), eps)
        spike = float(h["spike_mix"]) / (1.0 + sur)
        base = (1.0 - spike) * rat + spike * bnd
        if spectral:
            rmix = (float(h["root_channel_mix"]) if hard else 0.0) / (1.0 + 0.5 * sur)
        else:
            rmix = float(h["root_channel_mix"]) / (1.0 + 0.5 * sur)
        shaped = (1.0 - rmix) * base + rmix * root
        nov = torch.tanh(err / (clip * (1.0 + st["surprise"].to(dtype)))) * clip
        dmix = float(h["direct_force_mix"]) / (1.0 + 0.35 * sur)
        if spectral:
            srms = torch.sqrt(shaped.pow(2).mean() + eps)
            echo = rms_normalize(echo_raw, srms, eps) if (hard and float(h["echo_mix"]) != 0.0) else 0.0
            if torch.is_tensor(hash_pred):
                hash_pred = rms_normalize(hash_pred, srms, eps)
            direct = tangent * (srms / frms.clamp_min(eps))
        else:
            direct = rms_normalize(tangent, torch.sqrt(shaped.pow(2).mean() + eps), eps)
        core = (1.0 - dmix) * shaped + dmix * direct
        resmix = float(h["residual_feedback_mix"]) / (1.0 + sur)
        resid = rms_normalize(err, torch.sqrt(core.pow(2).mean() + eps), eps)
        if spectral:
            drive = ((1.0 - mix) * core + mix * pred + float(h["novelty_mix"]) * nov + resmix * resid
                     + (float(h["echo_mix"]) if hard else 0.0) * echo
                     + (float(h["hash_drive_mix"]) if hard else 0.0) * hash_pred)
        else:
            drive = (1.0 - mix) * core + mix * pred + float(h["novelty_mix"]) * nov + resmix * resid
        de_now = drive.pow(2).mean().to(st["drive_energy"].dtype)
        st["drive_energy"] = reservoir(st["drive_energy"], de_now, h["reservoir_decay"], step)
        gain = (float(h["target_update_rms"]) / torch.sqrt(st["drive_energy"].to(dtype) + eps)).clamp(
            float(h["min_gain"]), float(h["max_gain"]))
        self.last_update = drive * gain   # the fp32 update before its cast (inspection by tests)
        p.add_(self.last_update.to(dtype=p.dtype), alpha=-float(h["lr"]))

    def _scalar(self, p: Tensor, g: Tensor, st: dict) -> None:
        """Scalar contact route (cresso_v5.py:1434-1582, PyTorch branch)."""
        h = self.h
        dtype = work_dtype(p.dtype)
        if len(st) == 0:
            self._common(st, work_dtype(dtype))
            for k in ("q", "impulse", "metric_q", "metric_impulse"):
                st[k] = torch.zeros((), dtype=work_dtype(dtype))
        st["step"] += 1
        step = int(st["step"])
        eps = float(h["eps"])

        force = self._force(p, g, dtype)
        now = torch.sqrt(force.pow(2).mean() + eps)
        st["force_rms"] = reservoir(st["force_rms"], now, h["reservoir_decay"], step)
        scale = st["force_rms"].to(dtype).clamp_min(eps)

        dens = torch.log1p((force.abs() / scale + eps).pow(float(h["energy_power"]))).mean()
        mq, mp = st["metric_q"], st["metric_impulse"]
        mport = (dens - mq.to(dtype).tanh()).to(mq.dtype)
        mdt = float(h["metric_dt"])
        mp.mul_(max(0.0, 1.0 - mdt * float(h["metric_friction"])))
        mp.add_(mport - mq, alpha=mdt)
        mq.add_(mp, alpha=mdt)
        mq.clamp_(-3.0, 3.0)
        metric = torch.exp(float(h["metric_coupling"]) * mq.to(dtype)).clamp(0.06, 16.0)
        rel = (force.abs() / scale + eps).clamp(max=1.0e4)
        ls = float(h["local_sharpness"])
        local = (1.0 + ls * torch.sqrt(rel.clamp(max=100.0))).clamp(1.0, 8.0) if ls != 0.0 else 1.0
        inst = instant_axis_metric(rel, float(h["instant_metric_power"]), float(h["instant_metric_coupling"]), eps)
        tangent = (force / (scale * metric * local * inst + eps)).clamp(-1.0e4, 1.0e4)

        q, imp = st["q"], st["impulse"]
        pred = q.to(dtype).expand_as(tangent)
        err = tangent - pred
        sur_now = torch.sqrt(err.pow(2).mean() + eps)
        st["surprise"] = reservoir(st["surprise"], sur_now, h["surprise_decay"], step)
        port = err.mean().to(q.dtype)
        dt = float(h["dt"])
        sur = st["surprise"].to(q.dtype)
        plast = 1.0 + float(h["surprise_gain"]) * sur / (1.0 + sur)
        brake = 1.0 / (1.0 + float(h["surprise_brake"]) * sur)
        action = st["action"]
        energy = 0.5 * (imp.pow(2) + q.pow(2))
        action.mul_(0.985).add_((port * imp - energy).to(action.dtype), alpha=dt)
        fr = float(h["impulse_friction"]) + float(h["contact_gain"]) * torch.tanh(action.abs()).to(imp.dtype)
        imp.mul_(torch.clamp(1.0 - dt * fr, min=0.0))
        imp.add_(plast * brake * port - float(h["restoring"]) * q - float(h["cubic"]) * q.pow(3), alpha=dt)
        q.add_(imp, alpha=dt)
        q.clamp_(-8.0, 8.0)

        pred = q.to(dtype).expand_as(tangent)
        err = tangent - pred
        self._drive_apply(p, st, tangent, pred, err, None, 0.0, True, step, dtype, spectral=False)

    def _micro(self, p: Tensor, g: Tensor, st: dict) -> None:
        """Dense micro-field route for small tensors (cresso_v5.py:1355-1432)."""
        h = self.h
        dtype = work_dtype(p.dtype)
        if len(st) == 0:
            self._common(st, work_dtype(dtype))
            st["micro_energy"] = torch.ones_like(p.detach(), dtype=work_dtype(dtype))
            st["micro_impulse"] = torch.zeros_like(p.detach(), dtype=work_dtype(dtype))
            st["micro_refractory"] = torch.zeros_like(p.detach(), dtype=work_dtype(dtype))
        st["step"] += 1
        step = int(st["step"])
        eps = float(h["eps"])
        force = self._force(p, g, dtype)
        now = torch.sqrt(force.pow(2).mean() + eps)
        st["force_rms"] = reservoir(st["force_rms"], now, h["reservoir_decay"], step)
        scale = st["force_rms"].to(dtype).clamp_min(eps)
        rel = (force.abs() / scale + eps).clamp(max=1.0e4)
        e, imp, ref = st["micro_energy"], st["micro_impulse"], st["micro_refractory"]
        dsrc = rel.pow(float(h["energy_power"]))
        if step <= 1:
            e.copy_(dsrc.to(e.dtype))
        else:
            e.mul_(float(h["micro_decay"])).add_(dsrc.to(e.dtype), alpha=1.0 - float(h["micro_decay"]))
        metric = (e.to(dtype) / e.to(dtype).mean().clamp_min(eps)).pow(
            float(h["hash_metric_coupling"]) / max(0.25, float(h["energy_power"]))).clamp(0.08, 12.0)
        inst = instant_axis_metric(rel, float(h["instant_metric_power"]),
                                   min(0.35, float(h["instant_metric_coupling"])), eps)
        tangent = (force / (scale * metric * inst + eps)).clamp(-1.0e4, 1.0e4)
        ref.mul_(float(h["refractory_decay"])).add_(tangent.abs().to(ref.dtype), alpha=1.0 - float(h["refractory_decay"]))
        gate = 1.0 / (1.0 + float(h["refractory_gain"]) * ref.to(dtype))
        imp.mul_(float(h["micro_impulse_decay"])).add_((tangent * gate).to(imp.dtype),
                                                       alpha=1.0 - float(h["micro_impulse_decay"]))
        pred = imp.to(dtype)
        err = tangent - pred
        sur_now = torch.sqrt(err.pow(2).mean() + eps)
        st["surprise"] = reservoir(st["surprise"], sur_now, h["surprise_decay"], step)
        clip = float(h["drive_clip"])
        bnd = torch.tanh(tangent / clip) * clip
        rat = tangent / (1.0 + tangent.abs() / clip)
        sur = st["surprise"].to(dtype)
        spike = float(h["spike_mix"]) / (1.0 + sur)
        shaped = (1.0 - spike) * rat + spike * bnd
        target = torch.sqrt(shaped.pow(2).mean() + eps)
        pnorm = rms_normalize(pred, target, eps)
        dmix = float(h["direct_force_mix"]) / (1.0 + 0.35 * sur)
        mmix = float(h["micro_drive_mix"]) / (1.0 + 0.25 * sur)
        resmix = float(h["residual_feedback_mix"]) / (1.0 + sur)
        direct = rms_normalize(tangent, torch.sqrt(shaped.pow(2).mean() + eps), eps)
        resid = rms_normalize(err, torch.sqrt(shaped.pow(2).mean() + eps), eps)
        cw = (1.0 - dmix - 0.5 * mmix).clamp(0.0, 1.0)
        drive = cw * shaped + dmix * direct + mmix * pnorm + resmix * resid
        de_now = drive.pow(2).mean().to(st["drive_energy"].dtype)
        st["drive_energy"] = reservoir(st["drive_energy"], de_now, h["reservoir_decay"], step)
        gain = (float(h["target_update_rms"]) / torch.sqrt(st["drive_energy"].to(dtype) + eps)).clamp(
            float(h["min_gain"]), float(h["max_gain"]))
        self.last_update = drive * gain   # the fp32 update before its cast (inspection by tests)
        p.add_(self.last_update.to(dtype=p.dtype), alpha=-float(h["lr"]))
