"""Deterministic spectral mode tables of CRESSO5 (host-side, integer logic).

These define the persistent ``freqs``/``omega`` state and the per-mode
constants of the carriers.  They follow /root/reference/cresso_v5.py:127-135
(_hash_unit), 145-227 (_make_multiscale_frequencies) and 230-234
(_omega_from_freqs); the enumeration order and the duplicate guard of the
hashed tail are part of the state contract, so they are kept exactly.
"""

from __future__ import annotations

from typing import List, Tuple

import torch

_PRIMES = (2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37)


def hash_unit(n: int, salt: int = 0) -> float:
    """Mixer to [0, 1) on Python ints; the first product is not masked."""
    v = (n + 1) * 0x9E3779B1 + (salt + 11) * 0x85EBCA77
    v ^= v >> 16
    v = (v * 0x7FEB352D) % (1 << 32)
    v ^= v >> 15
    v = (v * 0x846CA68B) % (1 << 32)
    v ^= v >> 16
    return (v % (1 << 24)) / float(1 << 24)


def _axis_modes(ndim: int, fmax: int):
    for f in range(1, fmax + 1):
        for a in range(ndim):
            yield tuple(f if i == a else 0 for i in range(ndim))


def _diagonal_modes(ndim: int, fmax: int):
    for f in range(1, fmax + 1):
        yield (f,) * ndim
        if ndim > 1:
            yield tuple(f if i % 2 == 0 else max(1, fmax + 1 - f) for i in range(ndim))


def _pair_modes(ndim: int, fmax: int):
    if ndim < 2:
        return
    for f1 in range(1, fmax + 1):
        for f2 in range(1, fmax + 1):
            for a in range(ndim):
                v = [0] * ndim
                v[a] = f1
                v[(a + 1) % ndim] = f2
                yield tuple(v)


def mode_list(rank: int, ndim: int, max_frequency: int) -> List[Tuple[int, ...]]:
    """Zero mode, axis-local, (anti-)diagonal, sparse pairs, then a hashed tail."""
    rank, ndim, fmax = int(rank), int(ndim), max(0, int(max_frequency))
    if rank <= 0:
        return []
    zero = (0,) * ndim
    if fmax == 0:
        return [zero] * rank
    out = [zero]
    seen = {zero}
    for gen in (_axis_modes, _diagonal_modes, _pair_modes):
        for m in gen(ndim, fmax):
            if m not in seen:
                seen.add(m)
                out.append(m)
            if len(out) >= rank:
                return out[:rank]
    n, tries = 1, 0
    guard = max(64, 10 * rank * max(1, ndim))
    while len(out) < rank:
        v = [(n * _PRIMES[a % len(_PRIMES)] + a * a + 3 * a + 1) % (fmax + 1) for a in range(ndim)]
        nz = sum(1 for x in v if x)
        if nz == 0:
            v[n % ndim] = 1 + n % fmax
        elif nz == 1 and ndim > 1:
            v[(n + 1) % ndim] = 1 + (n // 2) % fmax
        m = tuple(v)
        if m not in seen or tries >= guard:
            seen.add(m)
            out.append(m)
        n += 1
        tries += 1
    return out[:rank]


def freqs_tensor(rank: int, ndim: int, max_frequency: int, device) -> torch.Tensor:
    modes = mode_list(rank, ndim, max_frequency)
    if not modes:
        return torch.empty((0, ndim), dtype=torch.long, device=device)
    return torch.tensor(modes, dtype=torch.long, device=device)


def omega_tensor(freqs: torch.Tensor) -> torch.Tensor:
    """omega_r = sqrt(1 + sum_a f_ra^2), fp32 (cresso_v5.py:230-234).

    Evaluated on the host, where the fp32 square root is correctly rounded
    (as CUDA's default sqrtf is); the device square root torch uses on ROCm
    can be one ulp off (sqrt(37) was), and an fp64 plan widens omega
    from this fp32 value, so that ulp would show at fp64 precision. The
    result is returned on the device of ``freqs``.
    """
    if freqs.numel() == 0:
        return torch.empty((0,), dtype=torch.float32, device=freqs.device)
    f = freqs.detach().to("cpu", torch.float32)
    return torch.sqrt(1.0 + (f * f).sum(dim=1)).to(freqs.device)
