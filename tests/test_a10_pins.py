"""a10, the metric and bases at prefill: the product's host code (openattention_amd/prefill.py,
torch) against the oracle's fp64 restatement with explicit rotation matrices and numpy's eigh
(oracle/oracle.py), and both against what the mathematics fixes: rotation-group identities,
the rank-one moment of rows that are one vector at consecutive positions, trace preservation,
the eigen-equations, Eckart-Young, the group mean, and sign invariance of the QGS scores.
Each bound is chosen so that a plausible slip (the bottom eigenvectors, a missing sqrt(lambda),
one head instead of the group mean, rows advanced the wrong way) fails it; the slips are
constructed below and shown to fail."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from openattention_amd import prefill, synth

D, HKV, G = 128, 2, 4
HQ = HKV * G
INV = synth.llama31_inv_freq()
INV64 = INV.double().numpy()


def _psd_with_spectrum(rng, lam):
    Q = np.linalg.qr(rng.standard_normal((D, D)))[0]
    return (Q * lam) @ Q.T


def _spectrum(rng, gaps=(16, 32)):
    """Decaying eigenvalues with a clear gap after the 16th and the 32nd."""
    lam = np.sort(rng.uniform(0.1, 1.0, D))[::-1].copy()
    lam[:gaps[1]] += 2.0
    lam[:gaps[0]] += 4.0
    return lam


# ------------------------------------------------------------------ rotations
def test_rope_matrix_pairs_and_group_law():
    """R_t rotates each pair (i, i + 64) by t theta_i, in the rotate_half convention:
    R e_i = cos e_i + sin e_{i+64}; R_a R_b = R_{a+b}; R_t R_t^T = s^2 I."""
    t, s = 777, 1.3
    R = O.rope_matrix(INV64, s, t)
    h = D // 2
    for i in (0, 5, 63):
        a = t * INV64[i]
        col = np.zeros(D)
        col[i], col[i + h] = np.cos(a), np.sin(a)
        assert np.allclose(R[:, i], s * col, atol=1e-12)
        col = np.zeros(D)
        col[i + h], col[i] = np.cos(a), -np.sin(a)
        assert np.allclose(R[:, i + h], s * col, atol=1e-12)
    assert np.allclose(R @ R.T, s * s * np.eye(D), atol=1e-12)
    Ra, Rb = O.rope_matrix(INV64, 1.0, 300), O.rope_matrix(INV64, 1.0, 477)
    assert np.allclose(Ra @ Rb, O.rope_matrix(INV64, 1.0, 777), atol=1e-9)
    # the product's rotation of rows equals the explicit matrix
    x = np.random.default_rng(0).standard_normal((3, D))
    c, sn = prefill.rope_trig(INV, torch.tensor([t]))
    got = s * (c * torch.from_numpy(x) + sn * prefill.rotate_half(torch.from_numpy(x)))
    assert np.allclose(got.numpy(), x @ R.T, atol=1e-9)


@pytest.mark.parametrize("p,s", [(0, 1.0), (4095, 1.0), (32767, 1.25), (131071, 1.0)])
def test_static_metric_window_mean(p, s):
    rng = np.random.default_rng(p)
    M = np.stack([_psd_with_spectrum(rng, _spectrum(rng)) for _ in range(3)])
    ref = O.static_metric_at(M, INV64, s, p)
    got = prefill.rot_avg(torch.from_numpy(M).float(), INV, s, p).double().numpy()
    assert np.abs(got - ref).max() < 2e-5 * np.abs(ref).max()
    # R_t / s is orthogonal: the trace scales by s^2; the identity maps to s^2 I
    assert np.allclose(np.trace(ref, axis1=1, axis2=2), s * s * np.trace(M, axis1=1, axis2=2))
    assert np.allclose(O.static_metric_at(np.eye(D)[None], INV64, s, p)[0], s * s * np.eye(D), atol=1e-12)
    ident = prefill.rot_avg(torch.eye(D)[None], INV, s, p)[0].double().numpy()
    assert np.allclose(ident, s * s * np.eye(D), atol=1e-6)


@pytest.mark.parametrize("T", [100, 4095, 32767])
def test_static_half_is_rot_avg_bit_for_bit(T):
    """The device build's static half (cached coefficients with rotate_half's signs folded in,
    rotate_half as a gather) equals 1/2 trace_norm(rot_avg(...)) exactly; the cached constants are
    reused for a second call and the picks' trig matches rope_trig of Qn - pick."""
    st = synth.static_metric(2)
    sc = float(st["attention_scaling"])
    for layer in range(2):
        ref = 0.5 * prefill.trace_norm(prefill.rot_avg(st["M"][layer], st["inv_freq"], sc, T, prefill.WIN))
        got = prefill.static_half(st["M"][layer], T, st["inv_freq"], sc, "cpu", 40)
        assert torch.equal(ref, got)
    a = prefill._metric_consts(T, 40, st["inv_freq"], sc, "cpu")
    assert prefill._metric_consts(T, 40, st["inv_freq"], sc, "cpu") is a
    pick = prefill.question_picks(40, "cpu")
    c, sn = prefill.rope_trig(st["inv_freq"], 40 - pick)
    assert torch.equal(a[2].long(), pick) and torch.equal(a[3], c) and torch.equal(a[4], sn)


def test_static_metric_window_mean_is_not_a_single_rotation():
    """The window mean differs from rotating by p alone (a dropped average would pass the
    trace check but not this one)."""
    rng = np.random.default_rng(3)
    M = _psd_with_spectrum(rng, _spectrum(rng))[None]
    one = O.rope_matrix(INV64, 1.0, 5000)
    single = one @ M[0] @ one.T
    got = prefill.rot_avg(torch.from_numpy(M).float(), INV, 1.0, 5000).double().numpy()[0]
    assert np.abs(got - single).max() > 1e-3 * np.abs(single).max()


# ------------------------------------------------------------------ question moment
@pytest.mark.parametrize("Qn", [1, 2, 3, 10, 64, 66, 200])
def test_question_moment_vs_explicit_rotations(Qn):
    rng = np.random.default_rng(Qn)
    q = rng.standard_normal((HQ, Qn, D)).astype(np.float32)
    ref = O.question_moment(q, INV64, 1.0)
    got = prefill.question_moment(torch.from_numpy(q), INV, 1.0).double().numpy()
    assert np.abs(got - ref).max() < 1e-5 * np.abs(ref).max()


def test_question_rows_are_advanced_to_the_decode_position():
    """Rows that are one pre-RoPE vector x at consecutive positions T - Qn + i all land on
    R_T x, so M_q = (R_T x)(R_T x)^T exactly (rank one).  Rows advanced by i - Qn, Qn - 1 - i or
    not at all fail."""
    T, Qn = 9000, 40
    x = np.random.default_rng(1).standard_normal(D)
    rows = np.stack([O.rope_matrix(INV64, 1.0, T - Qn + i) @ x for i in range(Qn)])[None]
    want = O.rope_matrix(INV64, 1.0, T) @ x
    want = np.outer(want, want)
    for Mq in (O.question_moment(rows, INV64, 1.0),
               prefill.question_moment(torch.from_numpy(rows), INV, 1.0).double().numpy()):
        assert np.abs(Mq[0] - want).max() < 1e-5 * np.abs(want).max()
    # advancing by Qn - 1 - i instead (one position short) leaves the rows off R_T x
    picks = prefill.question_picks(Qn, "cpu").numpy()
    wrong = np.zeros((D, D))
    for i in picks:
        r = O.rope_matrix(INV64, 1.0, Qn - 1 - int(i)) @ rows[0, i]
        wrong += np.outer(r, r)
    assert np.abs(wrong / len(picks) - want).max() > 1e-3 * np.abs(want).max()


def test_question_pick_rule():
    """P = min(64, max(Qn - 2, 1)) evenly spread picks over [0, Qn - 3], truncated, unique."""
    assert prefill.question_picks(1, "cpu").tolist() == [0]
    assert prefill.question_picks(3, "cpu").tolist() == [0]
    assert prefill.question_picks(10, "cpu").tolist() == list(range(8))
    p = prefill.question_picks(200, "cpu").tolist()
    assert len(p) == 64 and p[0] == 0 and p[-1] == 197 and p == sorted(set(p))


def test_query_metric_blend():
    rng = np.random.default_rng(5)
    M = np.stack([_psd_with_spectrum(rng, _spectrum(rng)) for _ in range(HQ)])
    q = rng.standard_normal((HQ, 50, D)).astype(np.float32)
    ref = O.query_metric(M, q, 8191, INV64, 1.0)
    got = prefill.query_metric(torch.from_numpy(M).float(), torch.from_numpy(q), 8191, INV, 1.0).double().numpy()
    assert np.abs(got - ref).max() < 2e-5 * np.abs(ref).max()
    assert np.allclose(np.trace(ref, axis1=1, axis2=2), 1.0)          # 1/2 + 1/2 of unit traces


# ------------------------------------------------------------------ bases
def _group_metrics(rng):
    """Per-head metrics whose own top subspaces differ from their group mean's."""
    out = []
    for _ in range(HKV):
        base = _psd_with_spectrum(rng, _spectrum(rng))
        for _ in range(G):
            out.append(base + 1.5 * _psd_with_spectrum(rng, np.sort(rng.uniform(0, 1, D))[::-1]))
    return np.stack(out)


def _top(M, r):
    ev, V = np.linalg.eigh(M)
    return ev[..., -r:], V[..., -r:]


def _u_ok(U, Mg):
    """U holds eigenvectors of Mg for its 32 largest eigenvalues."""
    lam = np.einsum("hdi,hde,hei->hi", U, Mg, U)
    top, _ = _top(Mg, 32)
    resid = np.linalg.norm(Mg @ U - U * lam[:, None, :], axis=(1, 2)) / np.linalg.norm(Mg, axis=(1, 2))
    ortho = np.abs(np.einsum("hdi,hdj->hij", U, U) - np.eye(32)).max()
    return (np.allclose(np.sort(lam, -1), np.sort(top, -1), rtol=1e-4) and resid.max() < 1e-4
            and ortho < 1e-4)


def _w_ok(W, M, tol=2e-2):
    """W W^T is M's best rank-16 approximation sum_{top 16} lambda u u^T (Eckart-Young), and
    each column carries sqrt(lambda) (|W_j|^2 = lambda_j)."""
    top, V = _top(M, 16)
    best = np.einsum("hdi,hi,hei->hde", V, top, V)
    WWt = W @ np.swapaxes(W, -1, -2)
    rel = np.linalg.norm(WWt - best, axis=(1, 2)) / np.linalg.norm(best, axis=(1, 2))
    norms = np.sort((W ** 2).sum(1), -1)
    return rel.max() < tol and np.allclose(norms, np.sort(top, -1), rtol=tol)


def test_bases_are_the_top_eigenvectors_of_the_right_matrices():
    rng = np.random.default_rng(11)
    M = _group_metrics(rng)
    Mg = M.reshape(HKV, G, D, D).mean(1)
    # the host side of the bases (which matrices, which eigenpairs, the sqrt scaling) over an
    # eigh's top-32 pairs; the device eigensolver that prefill.bases uses has its own GPU tests
    Mall = prefill.basis_matrices(torch.from_numpy(M).float(), HKV, G)
    ev, vec = torch.linalg.eigh(Mall.double())
    U, W = prefill.bases_from_eigenpairs(ev[..., -32:].float(), vec[..., -32:].float(), HKV)
    U, W = U.double().numpy(), W.float().double().numpy()
    Uo, Wo = O.bases(M, HKV, G)
    assert _u_ok(U, Mg) and _u_ok(Uo, Mg)
    assert _w_ok(W, M) and _w_ok(Wo, M, tol=1e-9)
    # the same subspaces from both restatements (projectors; signs are free)
    PU, PUo = U @ np.swapaxes(U, 1, 2), Uo @ np.swapaxes(Uo, 1, 2)
    assert np.abs(PU - PUo).max() < 1e-4
    # planted slips fail the checks
    _, Vall = np.linalg.eigh(Mg)
    assert not _u_ok(Vall[..., :32], Mg)                                   # bottom eigenvectors
    assert not _u_ok(np.linalg.eigh(M[::G])[1][..., -32:], Mg)             # head 0, not the mean
    ev, Vq = np.linalg.eigh(M)
    assert not _w_ok(Vq[..., -16:], M)                                     # no sqrt(lambda)
    assert not _w_ok(Vq[..., :16] * np.sqrt(ev[..., :16])[..., None, :], M)  # bottom 16
    assert not _w_ok(Vq[..., -16:] * ev[..., -16:][..., None, :], M)       # lambda, not sqrt


def test_qgs_scores_invariant_to_eigenvector_signs():
    """Flipping columns of U flips the codes and the query projection together: the QGS scores
    are bit for bit the same (the solver's sign choice cannot change the selection)."""
    rng = np.random.default_rng(2)
    T, Lmax = 1000, 1024
    K = (rng.standard_normal((HKV, Lmax, D))).astype(np.float32)
    Kb = (K.view(np.uint32) >> 16).astype(np.uint16)
    U = np.linalg.qr(rng.standard_normal((HKV, D, D)))[0][..., :32].astype(np.float32)
    flip = np.where(rng.random(32) < 0.5, -1.0, 1.0).astype(np.float32)
    q = (rng.standard_normal((HQ, D)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    S = []
    for Ux in (U, U * flip):
        codes, scale = O.qgs_codes(Kb, T, Ux)
        _, fexp, Z = O.qgs_prep(q, Ux, scale, G)
        S.append(O.qgs_scores(codes, Z, fexp, G, T, 0, 0))
    assert np.array_equal(S[0], S[1])
    assert not np.array_equal(O.qgs_codes(Kb, T, U)[0], O.qgs_codes(Kb, T, U * flip)[0])
