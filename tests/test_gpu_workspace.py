"""GPU parity of the spectral workspace that every step consumes, checked
directly through the C ABI (cresso_spectral_workspace_bins / _basis):

* the coordinate-hash bin of every element for every table and the bin
  occupancy counts are bit-exact against the reference: full index arrays on
  small shapes (golden idx_* vectors and the oracle's numpy restatement), and
  at the BASELINE sizes (4096^2, 8192^2, conv and 3-D tensors) against the
  reference's golden counts plus a weighted index checksum
  sum_i bin(i) * (i mod 1000003), which a wrong bin anywhere changes;
* the normalized carriers C_r, S_r formed from the separable tables match the
  reference's dense fp32 basis (golden basis_* vectors).
"""

import ctypes

import numpy as np
import pytest
import torch

from golden_inputs import load
from gpu_util import announce, needs_gpu
from oracle import cresso_oracle as O

pytestmark = [pytest.mark.gpu, needs_gpu]


def _workspace(shape, rank, fmax, bins, tables):
    import cresso_amd
    from cresso_amd import _native
    from cresso_amd.modes import mode_list
    from cresso_amd.spectral import _Workspace

    dummy = torch.nn.Parameter(torch.zeros(1, device="cuda"))
    group = cresso_amd.CRESSO5([dummy], rank=rank, max_frequency=fmax, hash_bins=bins,
                               hash_tables=tables).param_groups[0]
    freqs = tuple(v for m in mode_list(rank, len(shape), fmax) for v in m)
    lib = _native.load()
    ws = _Workspace(lib, tuple(shape), freqs, rank, bins, tables, group, torch.device("cuda"))
    return lib, ws


def _bins(shape, bins, tables, rank=8, fmax=5):
    from cresso_amd import _native

    lib, ws = _workspace(shape, rank, fmax, bins, tables)
    n = int(np.prod(shape))
    out = torch.empty((tables, n), dtype=torch.int32, device="cuda")
    cnt = torch.empty((tables, bins), dtype=torch.int64, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    _native.check(lib.cresso_spectral_workspace_bins(ws.plan, ctypes.c_void_p(ws.buf.data_ptr()),
                                                     ctypes.c_size_t(ws.buf.numel()), ctypes.c_void_p(out.data_ptr()),
                                                     ctypes.c_void_p(cnt.data_ptr()), ctypes.c_void_p(stream)),
                  "workspace bins")
    torch.cuda.synchronize()
    return out, cnt


SMALL = [  # (golden key, shape, bins, salt)
    ("idx_23x29_37_2", (23, 29), 37, 2),
    ("idx_64x48_64_0", (64, 48), 64, 0),
    ("idx_64x48_64_1", (64, 48), 64, 1),
    ("idx_1000_7_5", (1000,), 7, 5),
    ("idx_5000_256_3", (5000,), 256, 3),
    ("idx_31x37_37_1", (31, 37), 37, 1),
]


@pytest.mark.parametrize("case", SMALL, ids=[c[0] for c in SMALL])
def test_workspace_bins_match_reference_indices(case):
    key, shape, bins, salt = case
    announce(f"workspace bins {key}")
    out, cnt = _bins(shape, bins, salt + 1)
    ref = load("hash")[key].reshape(-1)
    got = out[salt].cpu().numpy()
    np.testing.assert_array_equal(got, ref)
    for t in range(salt + 1):
        idx = O.hash_index_np(int(np.prod(shape)), bins, t)
        np.testing.assert_array_equal(out[t].cpu().numpy(), idx.astype(np.int32), err_msg=f"table {t}")
        np.testing.assert_array_equal(cnt[t].cpu().numpy(), np.bincount(idx, minlength=bins), err_msg=f"counts {t}")


LARGE = [  # shape, bins, tables (BASELINE C1, C2, C3, C5 tensors)
    ((2048, 2048), 64, 2),
    ((4096, 4096), 64, 2),
    ((4096, 16), 64, 2),
    ((512, 256, 3, 3), 256, 4),
    ((64, 512, 512), 256, 4),
    ((8192, 8192), 256, 4),
]


@pytest.mark.parametrize("case", LARGE, ids=["x".join(map(str, c[0])) for c in LARGE])
def test_workspace_bins_and_counts_at_baseline_sizes(case):
    shape, bins, tables = case
    tag = "x".join(map(str, shape))
    announce(f"workspace bins {tag} B={bins} T={tables}")
    out, cnt = _bins(shape, bins, tables, rank=16 if bins == 256 else 8, fmax=7 if bins == 256 else 5)
    z = load("hash")
    n = out.shape[1]
    w = torch.arange(n, device="cuda", dtype=torch.int64) % 1000003
    for t in range(tables):
        np.testing.assert_array_equal(cnt[t].cpu().numpy(), z[f"counts_{tag}_{bins}_{t}"], err_msg=f"counts t={t}")
        wsum = int((out[t].to(torch.int64) * w).sum().item())
        assert wsum == int(z[f"wsum_{tag}_{bins}_{t}"]), f"weighted index checksum, table {t}"
        assert int(cnt[t].sum().item()) == n
    del out


def _basis_cases():
    z = load("basis")
    return sorted({k.split("/")[0] for k in z if k.startswith("basis_")})


@pytest.mark.parametrize("case", _basis_cases())
def test_workspace_basis_matches_reference_dense_basis(case):
    from cresso_amd import _native

    announce(f"workspace basis {case}")
    z = load("basis")
    _, shp, rank, fmax = case.split("_")
    shape = tuple(int(d) for d in shp.split("x"))
    rank, fmax = int(rank), int(fmax)
    lib, ws = _workspace(shape, rank, fmax, 64, 2)
    n = int(np.prod(shape))
    c = torch.empty(n, dtype=torch.float32, device="cuda")
    s = torch.empty(n, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    for r in range(rank):
        _native.check(lib.cresso_spectral_workspace_basis(ws.plan, ctypes.c_void_p(ws.buf.data_ptr()),
                                                          ctypes.c_size_t(ws.buf.numel()), r,
                                                          ctypes.c_void_p(c.data_ptr()), ctypes.c_void_p(s.data_ptr()),
                                                          ctypes.c_void_p(stream)), "workspace basis")
        torch.cuda.synchronize()
        for got, key in ((c, f"{case}/c{r}"), (s, f"{case}/s{r}")):
            ref = z[key].reshape(-1).astype(np.float64)
            g = got.cpu().numpy().astype(np.float64)
            # a degenerate carrier (raw values are fp32 rounding residue of
            # cos at the fp32 phase, e.g. f = 3 on a 3-wide axis) is compared
            # like the others: the residue is cos of the rounded argument,
            # the same on both sides, and the normalization scales it up
            np.testing.assert_allclose(g, ref, rtol=1e-5, atol=2e-5, err_msg=key)


GRAM_CASES = [((17, 19), 8, 5), ((64, 48), 8, 5), ((2048,), 8, 5), ((6, 10, 12), 16, 7), ((8, 6, 3, 3), 16, 7),
              ((300, 257), 4, 3)]


@pytest.mark.parametrize("case", GRAM_CASES, ids=["x".join(map(str, c[0])) + f"_r{c[1]}" for c in GRAM_CASES])
def test_workspace_gram_matches_dense_basis(case):
    """The closed-form Gram matrix (pair sums of the separable tables) against
    the dense fp64 product of the carriers the same workspace forms."""
    from cresso_amd import _native

    shape, rank, fmax = case
    announce(f"workspace gram {shape} r{rank}")
    lib, ws = _workspace(shape, rank, fmax, 64, 2)
    n = int(np.prod(shape))
    stream = torch.cuda.current_stream().cuda_stream
    X = torch.empty((2 * rank, n), dtype=torch.float32, device="cuda")
    for r in range(rank):
        _native.check(lib.cresso_spectral_workspace_basis(ws.plan, ctypes.c_void_p(ws.buf.data_ptr()),
                                                          ctypes.c_size_t(ws.buf.numel()), r,
                                                          ctypes.c_void_p(X[2 * r].data_ptr()),
                                                          ctypes.c_void_p(X[2 * r + 1].data_ptr()),
                                                          ctypes.c_void_p(stream)), "workspace basis")
    G = torch.empty((2 * rank, 2 * rank), dtype=torch.float64, device="cuda")
    _native.check(lib.cresso_spectral_workspace_gram(ws.plan, ctypes.c_void_p(ws.buf.data_ptr()),
                                                     ctypes.c_size_t(ws.buf.numel()), ctypes.c_void_p(G.data_ptr()),
                                                     ctypes.c_void_p(stream)), "workspace gram")
    torch.cuda.synchronize()
    Xd = X.double().cpu()
    dense = (Xd @ Xd.T / n).numpy()
    got = G.cpu().numpy()
    scale = np.sqrt(np.outer(np.diag(dense), np.diag(dense))) + 1e-30
    # the dense side is built from fp32-rounded carriers: agreement to ~1e-6 of the entry scale
    assert np.abs(got - dense).max() <= 2e-6 * max(1.0, scale.max()), np.abs(got - dense).max()
    assert np.allclose(np.diag(got), np.diag(dense), rtol=2e-6, atol=1e-9)
    np.testing.assert_allclose(got, got.T, rtol=0, atol=1e-12)


def _proj_cases():
    z = load("basis")
    return sorted({k.split("/")[0] for k in z if k.startswith("proj_")})


@pytest.mark.parametrize("case", _proj_cases())
def test_workspace_project_reconstruct_match_reference(case):
    # the reference's _project / _reconstruct on its own golden vectors (the
    # field x, its projections, gates and both reconstructions), degenerate
    # carriers included
    from cresso_amd import _native

    announce(f"workspace project/reconstruct {case}")
    z = load("basis")
    _, shp, rank, fmax = case.split("_")
    shape = tuple(int(d) for d in shp.split("x"))
    rank, fmax = int(rank), int(fmax)
    lib, ws = _workspace(shape, rank, fmax, 64, 2)
    n = int(np.prod(shape))
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    wsp, wsn = ctypes.c_void_p(ws.buf.data_ptr()), ctypes.c_size_t(ws.buf.numel())
    x = torch.from_numpy(z[f"{case}/x"]).reshape(-1).cuda()
    out = torch.empty(2 * rank, dtype=torch.float64, device="cuda")
    _native.check(lib.cresso_spectral_workspace_project(ws.plan, wsp, wsn, ctypes.c_void_p(x.data_ptr()),
                                                        ctypes.c_void_p(out.data_ptr()), stream), "project")
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(rank, 2)
    np.testing.assert_allclose(got[:, 0], z[f"{case}/cos"].astype(np.float64), rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(got[:, 1], z[f"{case}/sin"].astype(np.float64), rtol=1e-4, atol=1e-6)

    def recon(cc, sc, gates):
        o = torch.empty(n, dtype=torch.float32, device="cuda")
        cc_d, sc_d = cc.float().cuda(), sc.float().cuda()
        g_d = gates.float().cuda() if gates is not None else None
        _native.check(lib.cresso_spectral_workspace_reconstruct(
            ws.plan, wsp, wsn, ctypes.c_void_p(cc_d.data_ptr()), ctypes.c_void_p(sc_d.data_ptr()),
            ctypes.c_void_p(g_d.data_ptr() if g_d is not None else 0), ctypes.c_void_p(o.data_ptr()), stream),
            "reconstruct")
        torch.cuda.synchronize()
        return o.cpu().numpy().astype(np.float64)

    cc = torch.from_numpy(z[f"{case}/cos"])
    sc = torch.from_numpy(z[f"{case}/sin"])
    gates = torch.from_numpy(z[f"{case}/gates"])
    np.testing.assert_allclose(recon(cc, sc, gates), z[f"{case}/recon_gated"].reshape(-1), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(recon(cc, sc, None), z[f"{case}/recon"].reshape(-1), rtol=1e-5, atol=1e-6)
