"""The CPU oracle (oracle/cresso_oracle.py) against golden vectors of the reference.

Fixtures come from tests/golden/make_golden.py (the reference's cuda_ops="off"
path run in the build container).  Both sides run torch CPU ops in the same
order, so the tolerances here are far tighter than the GPU parity tolerances.
"""

import json

import numpy as np
import pytest
import torch

from golden_inputs import _same, load, trajectory, trajectory_names
from oracle import cresso_oracle as O


def test_frequency_pack_and_omega_match_reference():
    z = load("freqs")
    keys = [k for k in z if k.startswith("freqs_")]
    assert len(keys) >= 10
    for k in keys:
        rank, ndim, fmax = map(int, k.split("_")[1:])
        got = O.make_freqs(rank, ndim, fmax).numpy()
        np.testing.assert_array_equal(got.reshape(z[k].shape), z[k], err_msg=k)
        om = O.omega_from_freqs(O.make_freqs(rank, ndim, fmax)).numpy()
        np.testing.assert_array_equal(om, z[k.replace("freqs_", "omega_")], err_msg=k)


def test_hashed_tail_1d_has_duplicates():
    # (8,1,5): axis-local 1..5 then the hashed tail re-emits existing modes.
    assert [m[0] for m in O.frequency_pack(8, 1, 5)] == [0, 1, 2, 3, 4, 5, 1, 3]


def test_hash_unit_matches_reference():
    tab = load("freqs")["hash_unit"]
    for n, s, v in tab:
        assert O.hash_unit(int(n), int(s)) == v


def test_hash_unit_is_32bit_masked_mixer():
    # Independent recomputation with explicit 32-bit masking after the first
    # (unmasked) product: the result only depends on the low 24 bits.
    for n in range(50):
        for s in (0, 17, 101, 151, 160):
            x = (n + 1) * 2654435761 + (s + 11) * 2246822519
            x ^= x >> 16
            x = (x * 2146121005) % (1 << 32)
            x ^= x >> 15
            x = (x * 2221713035) % (1 << 32)
            x ^= x >> 16
            assert O.hash_unit(n, s) == (x % (1 << 24)) / (1 << 24)


def test_hash_indices_match_reference():
    z = load("hash")
    keys = [k for k in z if k.startswith("idx_")]
    for k in keys:
        _, shp, bins, salt = k.split("_")
        shape = tuple(int(d) for d in shp.split("x"))
        got = O.hash_index(shape, int(bins), int(salt)).numpy().astype(np.int32)
        np.testing.assert_array_equal(got, z[k], err_msg=k)


@pytest.mark.parametrize("key", ["counts_4096x4096_64_0", "counts_4096x16_64_1", "counts_512x256x3x3_256_2"])
def test_hash_counts_match_reference(key):
    z = load("hash")
    _, shp, bins, salt = key.split("_")
    n = int(np.prod([int(d) for d in shp.split("x")]))
    idx = O.hash_index_np(n, int(bins), int(salt))
    np.testing.assert_array_equal(np.bincount(idx, minlength=int(bins)), z[key])
    w = np.arange(n, dtype=np.int64) % 1000003
    assert int((idx * w).sum()) == int(z[key.replace("counts_", "wsum_")])
    assert int(z[key].sum()) == n


def _basis_cases():
    z = load("basis")
    return sorted({k.split("/")[0] for k in z if k.startswith("basis_")})


@pytest.mark.parametrize("case", _basis_cases())
def test_dense_basis_matches_reference(case):
    z = load("basis")
    _, shp, rank, fmax = case.split("_")
    shape = tuple(int(d) for d in shp.split("x"))
    rank, fmax = int(rank), int(fmax)
    fr = O.make_freqs(rank, len(shape), fmax)
    for r in range(rank):
        c, s = O.basis_pair(shape, fr, r, torch.float32)
        np.testing.assert_array_equal(c.numpy(), z[f"{case}/c{r}"], err_msg=f"{case} c{r}")
        np.testing.assert_array_equal(s.numpy(), z[f"{case}/s{r}"], err_msg=f"{case} s{r}")


@pytest.mark.parametrize("case", [c.replace("basis_", "proj_") for c in _basis_cases()])
def test_project_reconstruct_instant_match_reference(case):
    z = load("basis")
    _, shp, rank, fmax = case.split("_")
    shape = tuple(int(d) for d in shp.split("x"))
    rank, fmax = int(rank), int(fmax)
    fr = O.make_freqs(rank, len(shape), fmax)
    src = O.BasisSource(shape, fr, rank, torch.float32, 0)
    x = torch.from_numpy(z[f"{case}/x"])
    cc, sc = src.project(x)
    np.testing.assert_array_equal(cc.numpy(), z[f"{case}/cos"])
    np.testing.assert_array_equal(sc.numpy(), z[f"{case}/sin"])
    gates = torch.from_numpy(z[f"{case}/gates"])
    np.testing.assert_array_equal(src.reconstruct(cc, sc, gates).numpy(), z[f"{case}/recon_gated"])
    np.testing.assert_array_equal(src.reconstruct(cc, sc).numpy(), z[f"{case}/recon"])
    rel = (x.abs() + 1e-8).clamp(max=1e4)
    np.testing.assert_array_equal(O.instant_axis_metric(rel, 1.0, 0.55, 1e-8).numpy(), z[f"{case}/instant"])


def test_projection_matches_fp64_brute_force():
    # Textbook dot product in fp64 on the same (fp32) carriers: a dropped term,
    # a transposed operand or a wrong mode index fails this.
    shape, rank = (17, 19), 8
    fr = O.make_freqs(rank, 2, 5)
    x = torch.randn(shape, generator=torch.Generator().manual_seed(3))
    src = O.BasisSource(shape, fr, rank, torch.float32, 0)
    cc, sc = src.project(x)
    for r in range(rank):
        c, s = O.basis_pair(shape, fr, r, torch.float32)
        np.testing.assert_allclose(cc[r].item(), (x.double() * c.double()).mean().item(), rtol=1e-5, atol=1e-7)
        np.testing.assert_allclose(sc[r].item(), (x.double() * s.double()).mean().item(), rtol=1e-5, atol=1e-7)


def test_reconstruct_is_linear():
    shape, rank = (12, 40), 16
    fr = O.make_freqs(rank, 2, 7)
    src = O.BasisSource(shape, fr, rank, torch.float32, 0)
    g = torch.Generator().manual_seed(5)
    a1, b1, a2, b2 = (torch.randn(rank, generator=g) for _ in range(4))
    lhs = src.reconstruct(a1 + 2.0 * a2, b1 + 2.0 * b2).double()
    rhs = src.reconstruct(a1, b1).double() + 2.0 * src.reconstruct(a2, b2).double()
    np.testing.assert_allclose(lhs.numpy(), rhs.numpy(), rtol=1e-5, atol=1e-5)


def test_normalized_basis_has_zero_mean_unit_rms():
    for shape in [(17, 19), (64,), (5, 7, 9)]:
        fr = O.make_freqs(8, len(shape), 5)
        for r in range(1, 8):
            c, s = O.basis_pair(shape, fr, r, torch.float32)
            for t in (c, s):
                t = t.double()
                if t.abs().max() == 0:
                    continue
                assert abs(t.mean().item()) < 1e-5
                assert abs(t.pow(2).mean().sqrt().item() - 1.0) < 1e-4


def test_reservoir_known_answers():
    # Known answers of the reference's own safety test: 3.0 then 4.0, same tensor.
    st = torch.tensor(1.0)
    assert O.reservoir(st, torch.tensor(3.0), 0.5, 1) is st and float(st) == 3.0
    assert O.reservoir(st, torch.tensor(5.0), 0.5, 2) is st and float(st) == 4.0


def test_state_count_contract():
    assert O.theoretical_state_elements((128, 16), rank=4) == 8
    assert O.theoretical_state_elements((128, 16), rank=4, thin_matrix_route="spectral") == 4 * 2 + 48 + 3 * 128 * 2 + 4
    assert O.theoretical_state_elements((128, 128), rank=4, hash_bins=16, hash_tables=1) == 8 + 48 + 48 + 4
    # 840 LoRA tensors, spectral route forced: 444 elements each (B=64, T=2, R=4).
    assert O.theoretical_state_elements((4096, 16), 4, hash_bins=64, thin_matrix_route="spectral") == 444


def _rtol_for(dtype):
    return 2e-6 if dtype == "float32" else 1e-5


@pytest.mark.parametrize("name", trajectory_names())
def test_trajectory_matches_reference(name):
    meta, p0, grads, steps, sidx = trajectory(name)
    opt = O.OracleCRESSO5([p0.clone()], **meta["kwargs"])
    p = opt.params[0]
    for k, g in enumerate(grads):
        opt.step([g])
        exp = steps[k]
        pf = p.detach().float().reshape(-1)
        tol = dict(rtol=_rtol_for(meta["dtype"]), atol=1e-7)
        if "param" in exp:
            np.testing.assert_allclose(p.float().numpy(), exp["param"], **tol, err_msg=f"{name} step {k} param")
        np.testing.assert_allclose(pf[torch.from_numpy(sidx)].numpy(), exp["param_sample"], **tol)
        st = opt.state[0]
        for key, v in exp.items():
            if not key.startswith("state/"):
                continue
            sk = key[len("state/"):]
            got = st[sk]
            if torch.is_tensor(got):
                np.testing.assert_allclose(got.double().numpy(), v, rtol=1e-5, atol=1e-7,
                                           err_msg=f"{name} step {k} {sk}")
            else:
                assert got == int(v)


def _dtype_tol(dtype: str):
    # fp64 runs the reference's own fp64 ops: agreement to fp64 rounding;
    # fp16 params: the same fp32 work and the same rounded update as the reference
    return dict(rtol=1e-11, atol=1e-14) if dtype == "float64" else dict(rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("name", trajectory_names("trajectories_f16_f64"))
def test_f16_f64_trajectory_matches_reference(name):
    """The oracle's fp16 and fp64 legs (the update step's rounding for fp16
    params, every fp64 state and field for fp64 params) against the
    reference's own output (tests/golden/trajectories_f16_f64.npz)."""
    meta, p0, grads, steps, sidx = trajectory(name, "trajectories_f16_f64")
    opt = O.OracleCRESSO5([p0.clone()], **meta["kwargs"])
    p = opt.params[0]
    tol = _dtype_tol(meta["dtype"])
    for k, g in enumerate(grads):
        opt.step([g])
        exp = steps[k]
        pf = p.detach().reshape(-1)
        pf = pf if pf.dtype == torch.float64 else pf.float()
        if "param" in exp:
            np.testing.assert_allclose(p.double().numpy(), exp["param"], **tol, err_msg=f"{name} step {k} param")
        np.testing.assert_allclose(pf[torch.from_numpy(sidx)].double().numpy(), exp["param_sample"], **tol)
        st = opt.state[0]
        for key, v in exp.items():
            if not key.startswith("state/"):
                continue
            sk = key[len("state/"):]
            got = st[sk]
            if torch.is_tensor(got):
                if got.is_floating_point() and meta["dtype"] == "float64":
                    assert got.dtype == torch.float64, (name, sk)
                np.testing.assert_allclose(got.double().numpy(), v, **tol, err_msg=f"{name} step {k} {sk}")
            else:
                assert got == int(v)


def test_c1_2048_trajectory_matches_reference():
    z = load("c1_2048")
    meta = json.loads(str(z["meta"]))
    shape = tuple(meta["shape"])
    gen = torch.Generator().manual_seed(0)
    p = 0.02 * torch.randn(shape, generator=gen)
    assert _same(float(p.double().sum()), float(z["param0_sum"]))
    opt = O.OracleCRESSO5([p], **meta["kwargs"])
    idx = torch.from_numpy(z["sample_index"])
    for k in range(meta["steps"]):
        g = 1e-3 * torch.randn(shape, generator=gen)
        assert _same(float(g.double().sum()), float(z[f"grad{k}_sum"]))
        opt.step([g])
        np.testing.assert_allclose(p.reshape(-1)[idx].numpy(), z[f"step{k}/param_sample"], rtol=2e-6, atol=1e-8)
        for key in z:
            if key.startswith(f"step{k}/state/"):
                sk = key.split("/")[-1]
                got = opt.state[0][sk]
                if torch.is_tensor(got):
                    np.testing.assert_allclose(got.double().numpy(), z[key], rtol=1e-5, atol=1e-7, err_msg=sk)
