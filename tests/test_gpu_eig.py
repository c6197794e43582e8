"""The a10 eigensolver (oa_sym_eig_top, one-sided Jacobi on the device) against numpy's fp64
eigh and against what the mathematics fixes: the eigen-equation residual, orthonormality, the
top-k subspace (projectors, where the spectrum has a gap at k), ascending order, reading the
lower triangle only, and results that do not depend on the batch a matrix is in.  Spectra cover
clear gaps, near-degenerate and exactly repeated eigenvalues, a rank-deficient metric, a
diagonal matrix, a spread of six decades and the metric the build forms from synthetic data.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from openattention_amd import ops, prefill, synth
from tests.test_a10_pins import _group_metrics, _psd_with_spectrum, _spectrum, _u_ok, _w_ok

pytestmark = pytest.mark.gpu
DEV = "cuda"
D = 128
HKV, G = 2, 4


def _spectra(rng):
    out = {}
    out["gaps"] = _psd_with_spectrum(rng, _spectrum(rng))
    lam = np.sort(rng.uniform(0.05, 1.0, D // 2))[::-1]
    out["near_pairs"] = _psd_with_spectrum(rng, np.repeat(lam, 2) * np.tile([1.0, 1.0 + 1e-6], D // 2))
    lam = np.sort(rng.uniform(0.1, 1.0, D // 4))[::-1]
    out["repeated_x4"] = _psd_with_spectrum(rng, np.repeat(lam, 4))
    lam = np.zeros(D)
    lam[:48] = np.sort(rng.uniform(0.2, 1.0, 48))[::-1]
    out["rank48"] = _psd_with_spectrum(rng, lam)
    out["diagonal"] = np.diag(rng.permutation(np.linspace(0.01, 1.0, D)))
    out["six_decades"] = _psd_with_spectrum(rng, np.logspace(0, -6, D))
    return out


def _solve(Ms: np.ndarray, k: int):
    M = torch.from_numpy(np.ascontiguousarray(Ms, np.float32)).to(DEV)
    sweeps = torch.zeros(M.shape[0], dtype=torch.int32, device=DEV)
    ev, vec = ops.sym_eig_top(M, k, sweeps)
    torch.cuda.synchronize()
    return ev.cpu().double().numpy(), vec.cpu().double().numpy(), sweeps.cpu().numpy()


@pytest.mark.parametrize("k", [32, 16, 64])
def test_sym_eig_top_against_eigh_and_the_eigen_equation(k):
    print(f"[case] sym_eig_top k={k}", flush=True)
    rng = np.random.default_rng(5)
    cases = _spectra(rng)
    names = list(cases)
    Ms = np.stack([cases[n] for n in names])
    ev, vec, sweeps = _solve(Ms, k)
    for i, name in enumerate(names):
        M = Ms[i].astype(np.float32).astype(np.float64)
        lam, V = np.linalg.eigh(M)
        lmax = lam[-1]
        assert sweeps[i] > 0, (name, sweeps[i])                     # converged under the cap
        assert np.all(np.diff(ev[i]) >= 0), name                    # ascending
        err_ev = np.abs(ev[i] - lam[-k:]).max() / lmax
        vi = vec[i]
        resid = np.linalg.norm(M @ vi - vi * ev[i], axis=0).max() / lmax
        ortho = np.abs(vi.T @ vi - np.eye(k)).max()
        print(f"  {name}: sweeps {sweeps[i]} eig err {err_ev:.1e} resid {resid:.1e} ortho {ortho:.1e}")
        assert err_ev < 5e-5, name
        if name == "rank48" and k == 64:
            # (numerically) zero eigenvalues among the k: the null space's directions are free, so
            # only the nonzero part is checked as eigenvectors
            nz = lam[-k:] > 1e-6 * lmax
            assert np.all(ev[i][~nz] < 1e-5 * lmax)
            vi, evi = vi[:, nz], ev[i][nz]
            resid = np.linalg.norm(M @ vi - vi * evi, axis=0).max() / lmax
            ortho = np.abs(vi.T @ vi - np.eye(vi.shape[1])).max()
        assert resid < 2e-4, name
        assert ortho < 5e-5, name
        # the top-k subspace where the spectrum separates it from the rest
        if lam[-k] - lam[-k - 1] > 1e-3 * lmax:
            P, Pr = vi @ vi.T, V[:, -k:] @ V[:, -k:].T
            assert np.abs(P - Pr).max() < 1e-4, name


def test_sym_eig_top_reads_the_lower_triangle_and_is_batch_independent():
    print("[case] sym_eig_top lower triangle, batch independence", flush=True)
    rng = np.random.default_rng(9)
    base = _psd_with_spectrum(rng, _spectrum(rng)).astype(np.float32)
    junk = base.copy()
    iu = np.triu_indices(D, 1)
    junk[iu] = rng.standard_normal(len(iu[0])).astype(np.float32) * 100.0
    others = np.stack([_psd_with_spectrum(rng, _spectrum(rng)) for _ in range(5)]).astype(np.float32)
    batch = np.concatenate([base[None], others[:3], junk[None], others[3:]])
    ev, vec, _ = _solve(batch, 32)
    ev1, vec1, _ = _solve(base[None], 32)
    assert np.array_equal(ev[0], ev1[0]) and np.array_equal(vec[0], vec1[0])
    assert np.array_equal(ev[4], ev1[0]) and np.array_equal(vec[4], vec1[0])


def test_sym_eig_top_rejects_bad_arguments():
    M = torch.zeros(2, D, D, device=DEV)
    with pytest.raises(ValueError):
        ops.sym_eig_top(M, 65)
    with pytest.raises(ValueError):
        ops.sym_eig_top(M, 0)
    with pytest.raises(ValueError):
        ops.sym_eig_top(torch.zeros(2, 64, 64, device=DEV), 16)
    with pytest.raises(ValueError):
        ops.sym_eig_top(M.double(), 16)


def test_bases_on_device_are_the_top_eigenvectors_of_the_right_matrices():
    """prefill.bases with the device eigensolver on metrics whose heads' own top subspaces
    differ from their group mean's: U spans the group means' top-32 eigenvectors, W W^T is each
    metric's best rank-16 part with |W_j|^2 = lambda_j, both as the oracle's fp64 restatement."""
    print("[case] prefill.bases on the device", flush=True)
    rng = np.random.default_rng(11)
    M = _group_metrics(rng)
    Mg = M.reshape(HKV, G, D, D).mean(1)
    U, W = prefill.bases(torch.from_numpy(M).float().to(DEV), HKV, G)
    U, W = U.double().cpu().numpy(), W.float().double().cpu().numpy()
    assert _u_ok(U, Mg)
    assert _w_ok(W, M)
    Uo, _ = O.bases(M, HKV, G)
    PU, PUo = U @ np.swapaxes(U, 1, 2), Uo @ np.swapaxes(Uo, 1, 2)
    assert np.abs(PU - PUo).max() < 1e-4


def test_bases_on_device_from_the_build_metric():
    """The metric the build forms from synthetic keys and question rows (static metric rotated to
    T plus the question moment): the device eigenpairs against numpy's fp64 eigh."""
    print("[case] eigensolver on the build's metric", flush=True)
    static = synth.static_metric(1)
    _, _, _, qq, _ = synth.make_layer(1, 1, 4096, 4096, 64, "cpu")
    M = prefill.query_metric(static["M"][0], qq[0].float(), 4095, static["inv_freq"], 1.0)
    Mall = prefill.basis_matrices(M, 8, G).numpy()
    ev, vec, sweeps = _solve(Mall, 32)
    assert np.all(sweeps > 0)
    for i in range(Mall.shape[0]):
        lam, V = np.linalg.eigh(Mall[i].astype(np.float64))
        assert np.abs(ev[i] - lam[-32:]).max() < 5e-5 * lam[-1]
        P, Pr = vec[i] @ vec[i].T, V[:, -32:] @ V[:, -32:].T
        assert np.abs(P - Pr).max() < 1e-3
    print(f"  sweeps {sweeps.min()}..{sweeps.max()}")


@pytest.mark.parametrize("q_dtype", [torch.bfloat16, torch.float32])
def test_query_metric_kernel_against_host_metric_and_restatement(q_dtype):
    """oa_query_metric (question moments in fp64, trace normalisation, the blend with the
    rotated static metric's half, group means) against prefill.query_metric (host torch, pinned
    to the oracle's explicit-rotation restatement by tests/test_a10_pins.py) and against the
    oracle itself, for two sequences of one layer (row r uses head r % HQ)."""
    print(f"[case] query metric kernel {q_dtype}", flush=True)
    from tests.helpers import HKV as HKV_, G as G_
    HQ_ = HKV_ * G_
    static = synth.static_metric(1)
    B, N = 2, 4096
    _, _, _, qq, _ = synth.make_layer(1, B, N, N, 64, "cpu")
    qrows = qq.to(q_dtype)                                         # (B, HQ, Qn, D)
    T = N - 1
    M_pre, inv, sc = static["M"][0], static["inv_freq"], float(static["attention_scaling"])
    gm, M = prefill.metric_device(M_pre, qrows.reshape(B * HQ_, qrows.shape[2], D).to(DEV), T, inv, sc, G_)
    torch.cuda.synchronize()
    gm, M = gm.cpu().double().numpy(), M.cpu().double().numpy()
    for b in range(B):
        ref = prefill.query_metric(M_pre, qrows[b].float(), T, inv, sc).double().numpy()   # host torch
        got = M[b * HQ_:(b + 1) * HQ_]
        assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
        refg = ref.reshape(HKV_, G_, D, D).mean(1)
        assert np.abs(gm[b * HKV_:(b + 1) * HKV_] - refg).max() <= 1e-5 * np.abs(refg).max()
        o = O.query_metric(M_pre.double().numpy(), qrows[b].float().numpy(), T, inv.double().numpy(), sc)
        assert np.abs(got - o).max() <= 2e-5 * np.abs(o).max()
