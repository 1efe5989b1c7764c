"""Write golden input/output vectors of the reference's cuda_ops="off" path.

Runs in the build container only (the reference is never shipped):

    python tests/golden/make_golden.py [/root/reference]          # every fixture
    python tests/golden/make_golden.py [/root/reference] --dtypes  # only trajectories_f16_f64.npz

It loads ``cresso_v5.py`` by path exactly as the reference's own tests do and
records, as plain arrays in ``tests/golden/*.npz``:
  * frequency packs and omegas for several (rank, ndim, max_frequency);
  * hash bin indices (small n) and bin counts (up to 4096*4096);
  * dense normalized basis pairs (2D, 1D, 3D and the degenerate 3-wide 4D case);
  * project / reconstruct outputs;
  * multi-step optimizer trajectories (params + every state tensor per step)
    for the spectral, scalar and micro routes, fp32 and bf16
    (trajectories.npz), fp16 and fp64 (trajectories_f16_f64.npz).
Nothing but arrays and JSON-encoded hyperparameters is written.
"""

from __future__ import annotations

import importlib.util
import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ARGS = [a for a in sys.argv[1:] if not a.startswith("--")]
REF = Path(ARGS[0]) if ARGS else Path("/root/reference")


def load_reference():
    spec = importlib.util.spec_from_file_location("cresso_v5_reference", REF / "cresso_v5.py")
    mod = importlib.util.module_from_spec(spec)
    assert spec is not None and spec.loader is not None
    spec.loader.exec_module(mod)
    return mod


def to_np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        t = t.float()
    return t.numpy().copy()


def sample_index(n: int, k: int = 4096, seed: int = 7) -> np.ndarray:
    rs = np.random.RandomState(seed)
    return np.sort(rs.choice(n, size=min(n, k), replace=False)).astype(np.int64)


def make_inputs(shape, dtype, steps, seed, grad_std=1.0, param_std=1.0, spike=False):
    """Seeded inputs; tests/golden_inputs.py regenerates the same sequence."""
    gen = torch.Generator().manual_seed(seed)
    p0 = (param_std * torch.randn(shape, generator=gen, dtype=torch.float32)).to(dtype)
    grads = []
    for _ in range(steps):
        g = grad_std * torch.randn(shape, generator=gen, dtype=torch.float32)
        if spike:
            mask = torch.rand(shape, generator=gen) < 0.01
            g = torch.where(mask, g * 50.0, g)
        grads.append(g.to(dtype))
    return p0, grads


def run_trajectory(ref, name, shape, dtype, kwargs, steps, seed, grad_std=1.0, param_std=1.0,
                   spike=False):
    p0, grads = make_inputs(shape, dtype, steps, seed, grad_std, param_std, spike)
    store_dense = int(np.prod(shape)) <= 20000
    param = torch.nn.Parameter(p0.clone())
    opt = ref.CRESSO5([param], cuda_ops="off", **kwargs)
    out = {"meta": np.array(json.dumps(dict(name=name, shape=list(shape), dtype=str(dtype).replace("torch.", ""),
                                                kwargs=kwargs, steps=steps, seed=seed, grad_std=grad_std,
                                                param_std=param_std, spike=spike)))}
    n = int(np.prod(shape))
    idx = sample_index(n)
    if store_dense:
        out["param0"] = to_np(p0)
    out["param0_sum"] = np.array(float(p0.double().sum()))
    out["sample_index"] = idx
    for k, g in enumerate(grads):
        if store_dense:
            out[f"grad{k}"] = to_np(g)
        out[f"grad{k}_sum"] = np.array(float(g.double().sum()))
        param.grad = g.clone()
        opt.step()
        pflat = param.detach().reshape(-1)
        if pflat.dtype in (torch.bfloat16, torch.float16):
            pflat = pflat.float()
        if store_dense:
            out[f"step{k}/param"] = to_np(param)
        out[f"step{k}/param_sample"] = to_np(pflat[torch.from_numpy(idx)])
        out[f"step{k}/param_sum"] = np.array(float(pflat.double().sum()))
        out[f"step{k}/param_sumsq"] = np.array(float((pflat.double() ** 2).sum()))
        for key, val in opt.state[param].items():
            if torch.is_tensor(val):
                out[f"step{k}/state/{key}"] = to_np(val)
            else:
                out[f"step{k}/state/{key}"] = np.array(val)
    return out


# fp16 and fp64 params: the fp16 update step (alpha rounded to the param
# dtype by torch's add_) and every fp64 state and field (the fp64 work dtype,
# cresso_v5.py:119-124) on the spectral, scalar and micro routes
OPS_KWARGS = dict(lr=2.0e-3, rank=8, max_frequency=5, min_spectral_size=1, hard_channel_min_size=1,
                  thin_matrix_hard_cutoff=0, hash_bins=37, hash_tables=2, basis_cache_limit_elements=0)
DTYPE_CASES = [
    ("spectral_31x37_f16", (31, 37), torch.float16, dict(OPS_KWARGS, lr=1e-3), 3, 8643, 0.05, 0.05, False),
    ("spectral_64x48_f16", (64, 48), torch.float16,
     dict(lr=2e-3, rank=8, max_frequency=5, hash_bins=64, hash_tables=2), 4, 31, 1e-2, 0.02, True),
    ("spectral_31x37_f64", (31, 37), torch.float64, OPS_KWARGS, 5, 9013, 1.0, 1.0, False),
    ("spectral_64x48_f64", (64, 48), torch.float64,
     dict(lr=2e-3, rank=8, max_frequency=5, hash_bins=64, hash_tables=2), 6, 32, 1e-3, 0.02, True),
    ("spectral_1d_2048_f64", (2048,), torch.float64,
     dict(rank=8, max_frequency=5, hash_bins=64, hash_tables=2), 4, 33, 1e-2, 0.02, False),
    ("spectral_3d_6x10x12_f64", (6, 10, 12), torch.float64,
     dict(rank=16, max_frequency=7, hash_bins=256, hash_tables=4, min_spectral_size=1), 4, 34, 1e-3, 0.02, False),
    ("spectral_4d_8x6x3x3_f64", (8, 6, 3, 3), torch.float64,
     dict(rank=16, max_frequency=7, hash_bins=256, hash_tables=4, min_spectral_size=1), 3, 35, 1e-3, 0.02, False),
    ("spectral_40x30_variants_f64", (40, 30), torch.float64,
     dict(rank=8, max_frequency=5, hash_bins=64, hash_tables=3, weight_decay=0.01, maximize=True,
          local_sharpness=0.3, min_spectral_size=1, warmup_steps=0), 4, 36, 1e-2, 0.05, False),
    ("scalar_128x16_f64", (128, 16), torch.float64,
     dict(lr=2e-3, rank=4, thin_matrix_route="scalar", thin_matrix_max_width=64, min_spectral_size=1), 8, 2469,
     1.0, 1.0, False),
    ("scalar_4096x16_f64", (4096, 16), torch.float64, dict(rank=4, hash_bins=64, hash_tables=2), 4, 37, 1e-4, 0.02,
     False),
    ("scalar_64x16_f16", (64, 16), torch.float16,
     dict(lr=1e-3, rank=4, thin_matrix_route="scalar", thin_matrix_max_width=64, min_spectral_size=1), 3, 3580,
     0.05, 0.05, False),
    ("micro_12x10_f64", (12, 10), torch.float64, dict(micro_field_max_size=256, rank=4), 4, 38, 1e-2, 0.1, False),
]


def write_trajectories(ref, cases, fname):
    tz = {}
    for name, shape, dtype, kwargs, steps, seed, gstd, pstd, spike in cases:
        tr = run_trajectory(ref, name, shape, dtype, kwargs, steps, seed, gstd, pstd, spike)
        for k, v in tr.items():
            tz[f"{name}/{k}"] = v
        print("trajectory", name, flush=True)
    np.savez_compressed(HERE / fname, **tz)


def main() -> None:
    torch.set_num_threads(max(1, torch.get_num_threads()))
    ref = load_reference()
    write_trajectories(ref, DTYPE_CASES, "trajectories_f16_f64.npz")
    if "--dtypes" in sys.argv:
        return

    # ---------------- frequencies / omega / hash_unit ----------------
    fz = {}
    for rank, ndim, fmax in [(8, 2, 5), (16, 2, 7), (16, 4, 7), (16, 3, 7), (8, 1, 5), (4, 2, 3),
                             (12, 3, 2), (4, 2, 0), (20, 1, 3), (40, 2, 2), (30, 1, 5), (6, 5, 1)]:
        fr = ref._make_multiscale_frequencies(rank, ndim, fmax, torch.device("cpu"))
        fz[f"freqs_{rank}_{ndim}_{fmax}"] = to_np(fr)
        fz[f"omega_{rank}_{ndim}_{fmax}"] = to_np(ref._omega_from_freqs(fr))
    fz["hash_unit"] = np.array([[n, s, ref._hash_unit(n, s)] for n in range(0, 40) for s in
                                (0, 17, 18, 101, 152, 160)], dtype=np.float64)
    np.savez_compressed(HERE / "freqs.npz", **fz)

    # ---------------- hash indices / counts ----------------
    hz = {}
    for shape, bins, salt in [((23, 29), 37, 2), ((64, 48), 64, 0), ((64, 48), 64, 1), ((1000,), 7, 5),
                              ((5000,), 256, 3), ((31, 37), 37, 0), ((31, 37), 37, 1)]:
        key = f"idx_{'x'.join(map(str, shape))}_{bins}_{salt}"
        hz[key] = to_np(ref._hash_index_tensor(shape, bins, torch.device("cpu"), salt=salt)).astype(np.int32)
    for n_shape, bins, salts in [((4096, 4096), 64, (0, 1)), ((2048, 2048), 64, (0, 1)),
                                 ((8192, 8192), 256, (0, 1, 2, 3)), ((4096, 16), 64, (0, 1)),
                                 ((512, 256, 3, 3), 256, (0, 1, 2, 3)), ((64, 512, 512), 256, (0, 1, 2, 3))]:
        for salt in salts:
            idx = ref._hash_index_tensor(n_shape, bins, torch.device("cpu"), salt=salt).reshape(-1)
            key = f"counts_{'x'.join(map(str, n_shape))}_{bins}_{salt}"
            hz[key] = np.bincount(idx.numpy(), minlength=bins).astype(np.int64)
            # position-weighted checksum: catches permutations that keep the counts
            w = (torch.arange(idx.numel(), dtype=torch.int64) % 1000003)
            hz[key.replace("counts_", "wsum_")] = np.array(int((idx * w).sum()), dtype=np.int64)
            del idx, w
    np.savez_compressed(HERE / "hash.npz", **hz)

    # ---------------- dense basis / project / reconstruct ----------------
    bz = {}
    for shape, rank, fmax in [((17, 19), 8, 5), ((64,), 8, 5), ((8, 6, 3, 3), 16, 7), ((5, 7, 9), 16, 7),
                              ((12, 40), 16, 7), ((3, 200), 8, 5)]:
        tag = "x".join(map(str, shape))
        fr = ref._make_multiscale_frequencies(rank, len(shape), fmax, torch.device("cpu"))
        for r in range(rank):
            c, s = ref._basis_pair(shape, fr, r, torch.float32)
            bz[f"basis_{tag}_{rank}_{fmax}/c{r}"] = to_np(c)
            bz[f"basis_{tag}_{rank}_{fmax}/s{r}"] = to_np(s)
        gen = torch.Generator().manual_seed(1234)
        x = torch.randn(shape, generator=gen)
        cc, sc = ref._project(x, fr, rank)
        gates = torch.sigmoid(torch.linspace(-2.0, 2.0, rank))
        bz[f"proj_{tag}_{rank}_{fmax}/x"] = to_np(x)
        bz[f"proj_{tag}_{rank}_{fmax}/cos"] = to_np(cc)
        bz[f"proj_{tag}_{rank}_{fmax}/sin"] = to_np(sc)
        bz[f"proj_{tag}_{rank}_{fmax}/gates"] = to_np(gates)
        bz[f"proj_{tag}_{rank}_{fmax}/recon_gated"] = to_np(ref._reconstruct(cc, sc, fr, shape, torch.float32, gates=gates))
        bz[f"proj_{tag}_{rank}_{fmax}/recon"] = to_np(ref._reconstruct(cc, sc, fr, shape, torch.float32))
        rel = (x.abs() + 1e-8).clamp(max=1e4)
        bz[f"proj_{tag}_{rank}_{fmax}/instant"] = to_np(ref._instant_axis_metric(rel, 1.0, 0.55, 1e-8))
    np.savez_compressed(HERE / "basis.npz", **bz)

    # ---------------- optimizer trajectories ----------------
    ops_kwargs = dict(lr=2.0e-3, rank=8, max_frequency=5, min_spectral_size=1, hard_channel_min_size=1,
                      thin_matrix_hard_cutoff=0, hash_bins=37, hash_tables=2, basis_cache_limit_elements=0)
    cases = [
        ("spectral_31x37_f32", (31, 37), torch.float32, ops_kwargs, 6, 9012, 1.0, 1.0, False),
        ("spectral_31x37_cached_f32", (31, 37), torch.float32,
         dict(ops_kwargs, basis_cache_limit_elements=2_000_000), 3, 9012, 1.0, 1.0, False),
        ("spectral_64x48_f32", (64, 48), torch.float32,
         dict(lr=2e-3, rank=8, max_frequency=5, hash_bins=64, hash_tables=2), 6, 11, 1e-3, 0.02, True),
        ("spectral_1d_2048_f32", (2048,), torch.float32,
         dict(rank=8, max_frequency=5, hash_bins=64, hash_tables=2), 5, 12, 1e-2, 0.02, False),
        ("spectral_4d_8x6x3x3_f32", (8, 6, 3, 3), torch.float32,
         dict(rank=16, max_frequency=7, hash_bins=256, hash_tables=4, min_spectral_size=1), 4, 13, 1e-3, 0.02, False),
        ("spectral_3d_6x10x12_f32", (6, 10, 12), torch.float32,
         dict(rank=16, max_frequency=7, hash_bins=256, hash_tables=4, min_spectral_size=1), 4, 14, 1e-3, 0.02, False),
        ("spectral_31x37_bf16", (31, 37), torch.bfloat16,
         dict(ops_kwargs, lr=1e-3), 3, 8642, 0.05, 0.05, False),
        ("spectral_40x30_variants_f32", (40, 30), torch.float32,
         dict(rank=8, max_frequency=5, hash_bins=64, hash_tables=3, weight_decay=0.01, maximize=True,
              local_sharpness=0.3, min_spectral_size=1, warmup_steps=0), 4, 15, 1e-2, 0.05, False),
        ("spectral_thin_200x6_f32", (200, 6), torch.float32,
         dict(rank=4, max_frequency=3, hash_bins=64, thin_matrix_route="spectral"), 3, 16, 1e-2, 0.05, False),
        ("spectral_128x128_r4_f32", (128, 128), torch.float32,
         dict(rank=4, max_frequency=3, hash_bins=16, hash_tables=1, min_spectral_size=1, hard_channel_min_size=1,
              thin_matrix_hard_cutoff=0, basis_cache_limit_elements=0), 4, 17, 1.0, 1.0, False),
        ("scalar_128x16_f32", (128, 16), torch.float32,
         dict(lr=2e-3, rank=4, thin_matrix_route="scalar", thin_matrix_max_width=64, min_spectral_size=1), 10, 2468, 1.0, 1.0, False),
        ("scalar_16x300_f32", (16, 300), torch.float32, dict(rank=4), 6, 21, 1e-3, 0.02, False),
        ("scalar_4096x16_f32", (4096, 16), torch.float32, dict(rank=4, hash_bins=64, hash_tables=2), 5, 22, 1e-4, 0.02, False),
        ("scalar_64x16_bf16", (64, 16), torch.bfloat16,
         dict(lr=1e-3, rank=4, thin_matrix_route="scalar", thin_matrix_max_width=64, min_spectral_size=1), 3, 3579, 0.05, 0.05, False),
        ("scalar_1d_100_f32", (100,), torch.float32, dict(rank=8), 4, 23, 1e-2, 0.1, False),
        ("scalar_3d_4x5x6_f32", (4, 5, 6), torch.float32, dict(rank=8, weight_decay=0.02), 4, 24, 1e-2, 0.1, False),
        ("scalar_0d_f32", (), torch.float32, dict(rank=8), 3, 25, 1e-2, 0.1, False),
        ("scalar_tiny_eps_f32", (4096, 16), torch.float32, dict(rank=4), 3, 26, 1e-7, 0.02, False),
        ("micro_12x10_f32", (12, 10), torch.float32, dict(micro_field_max_size=256, rank=4), 4, 27, 1e-2, 0.1, False),
    ]
    write_trajectories(ref, cases, "trajectories.npz")

    # C1 of BASELINE.json: (2048,2048) fp32, grad N(0,1e-3) from seed 0, 10 steps.
    c1 = run_c1(ref)
    np.savez_compressed(HERE / "c1_2048.npz", **c1)
    print("wrote golden fixtures to", HERE)


def run_c1(ref):
    """(2048,2048) fp32, p0 = 0.02*randn then g_k = 1e-3*randn from one seed-0 generator."""
    shape = (2048, 2048)
    gen = torch.Generator().manual_seed(0)
    p0 = 0.02 * torch.randn(shape, generator=gen)
    param = torch.nn.Parameter(p0.clone())
    kwargs = dict(lr=2e-3, rank=8, max_frequency=5, hash_bins=64, hash_tables=2)
    opt = ref.CRESSO5([param], cuda_ops="off", **kwargs)
    idx = sample_index(shape[0] * shape[1])
    out = {"meta": np.array(json.dumps(dict(name="c1_2048", shape=list(shape), kwargs=kwargs, steps=10, seed=0))),
           "sample_index": idx, "param0_sum": np.array(float(p0.double().sum()))}
    for k in range(10):
        g = 1e-3 * torch.randn(shape, generator=gen)
        out[f"grad{k}_sum"] = np.array(float(g.double().sum()))
        param.grad = g
        opt.step()
        pf = param.detach().reshape(-1)
        out[f"step{k}/param_sample"] = to_np(pf[torch.from_numpy(idx)])
        out[f"step{k}/param_sum"] = np.array(float(pf.double().sum()))
        out[f"step{k}/param_sumsq"] = np.array(float((pf.double() ** 2).sum()))
        for key, val in opt.state[param].items():
            out[f"step{k}/state/{key}"] = to_np(val) if torch.is_tensor(val) else np.array(val)
        print("c1 step", k, flush=True)
    return out


if __name__ == "__main__":
    main()
