"""numpy front end of the CPU restatement (oracle/oa_oracle.c) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, as the
checker.  Each wrapper names the reference lines the C function restates.

Pinning (what fixes each function independently of the GPU code) is done in
tests/test_oracle_pins.py: brute-force integer/Fraction scores, fp64 closed forms, an exact
rational water-filling solver, libm comparisons of the deterministic elementary functions,
sorted-selection brute force for top-k / top-q, and invariants.
"""
from __future__ import annotations

import ctypes as ct
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

D, RQ, RC = 128, 32, 16


def _lib():
    global _LIB
    if _LIB is None:
        from oracle import build as _b
        if not os.path.exists(_b.LIB) or os.path.getmtime(_b.LIB) < os.path.getmtime(_b.SRC):
            _b.build()
        lib = ct.CDLL(_b.LIB)
        lib.oa_det_exp.restype = ct.c_double
        lib.oa_det_exp.argtypes = [ct.c_double]
        lib.oa_det_log.restype = ct.c_double
        lib.oa_det_log.argtypes = [ct.c_double]
        lib.oa_det_logf.restype = ct.c_float
        lib.oa_det_logf.argtypes = [ct.c_float]
        lib.oa_det_erff.restype = ct.c_float
        lib.oa_det_erff.argtypes = [ct.c_float]
        _LIB = lib
    return _LIB


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ct.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ------------------------------------------------------------------ elementary functions
def det_exp(x: float) -> float:
    return _lib().oa_det_exp(float(x))


def det_log(x: float) -> float:
    return _lib().oa_det_log(float(x))


def det_logf(x: float) -> float:
    return _lib().oa_det_logf(float(x))


def det_erff(x: float) -> float:
    return _lib().oa_det_erff(float(x))


# ------------------------------------------------------------------ decode-stage functions
def qgs_prep(q_bf16: np.ndarray, U: np.ndarray, scale: np.ndarray, G: int):
    """static_top_k.py:203-213 -> (zq (R,32) f32, fexp (R,) i32, Z (R,32) i32)"""
    q = _c(q_bf16, np.uint16)
    R = q.shape[0]
    U = _c(U, np.float32)
    scale = _c(scale, np.float32)
    zq = np.zeros((R, RQ), np.float32)
    fexp = np.zeros(R, np.int32)
    Z = np.zeros((R, RQ), np.int32)
    _lib().oa_ref_qgs_prep(_p(q), _p(U), _p(scale), ct.c_int(R), ct.c_int(G), _p(zq), _p(fexp), _p(Z))
    return zq, fexp, Z


def qgs_scores(codes: np.ndarray, Z: np.ndarray, fexp: np.ndarray, G: int, n: int, ns: int, nl: int,
               ncols: int | None = None) -> np.ndarray:
    """static_top_k.py:197-218 + sink/local masking -> S (R, ncols) f32"""
    codes = _c(codes, np.int8)
    BH, Lmax, _ = codes.shape
    Z = _c(Z, np.int32)
    fexp = _c(fexp, np.int32)
    R = Z.shape[0]
    ncols = Lmax if ncols is None else ncols
    S = np.zeros((R, ncols), np.float32)
    _lib().oa_ref_qgs_scores(_p(codes), ct.c_int(Lmax), _p(Z), _p(fexp), ct.c_int(R), ct.c_int(G),
                             ct.c_int(n), ct.c_int(ns), ct.c_int(nl), ct.c_int(ncols), _p(S))
    return S


def topk_select(S: np.ndarray, n: int, ns: int, nl: int, k: int) -> np.ndarray:
    """basic_fixed.py:48-67,354-363 + fixed/base.py:74-85 -> sel (R, ns+nl+k) i32"""
    S = _c(S, np.float32)
    R, ncols = S.shape
    sel = np.zeros((R, ns + nl + k), np.int32)
    _lib().oa_ref_topk_select(_p(S), ct.c_int(ncols), ct.c_int(R), ct.c_int(n), ct.c_int(ns),
                              ct.c_int(nl), ct.c_int(k), _p(sel))
    return sel


def errorgate(q_bf16, K_bf16, asg, sel, Sk, Sk2, nb, G: int, sc: float, sc2: float):
    """multibin.py:605-644, 734-738, 2370-2389; methods_eager.py:612-627 -> (score, n_t) (R,C) f32"""
    q = _c(q_bf16, np.uint16)
    K = _c(K_bf16, np.uint16)
    asg = _c(asg, np.int32)
    sel = _c(sel, np.int32)
    Sk, Sk2, nb = _c(Sk, np.float32), _c(Sk2, np.float32), _c(nb, np.float32)
    R, C = nb.shape
    Lmax = K.shape[1]
    score = np.zeros((R, C), np.float32)
    n_t = np.zeros((R, C), np.float32)
    _lib().oa_ref_errorgate(_p(q), _p(K), ct.c_int(Lmax), _p(asg), _p(sel), ct.c_int(sel.shape[1]),
                            _p(Sk), _p(Sk2), _p(nb), ct.c_int(R), ct.c_int(G), ct.c_int(C),
                            ct.c_float(sc), ct.c_float(sc2), _p(score), _p(n_t))
    return score, n_t


def waterfill(score, n_t, E: int) -> np.ndarray:
    """multibin.py:1385-1422 (+ order 2471-2472) -> quota (R,C) f32"""
    score, n_t = _c(score, np.float32), _c(n_t, np.float32)
    R, C = score.shape
    quota = np.zeros((R, C), np.float32)
    _lib().oa_ref_waterfill(_p(score), _p(n_t), ct.c_int(R), ct.c_int(C), ct.c_double(float(E)),
                            _p(quota))
    return quota


def topq(S, asg, sel, quota, n: int, E: int) -> np.ndarray:
    """multibin.py:2522-2558 with lower-position ties -> exp_idx (R,E) i32"""
    S = _c(S, np.float32)
    asg = _c(asg, np.int32)
    sel = _c(sel, np.int32)
    quota = _c(quota, np.float32)
    R, C = quota.shape
    exp_idx = np.zeros((R, E), np.int32)
    _lib().oa_ref_topq(_p(S), ct.c_int(S.shape[1]), _p(asg), ct.c_int(asg.shape[1]), _p(sel),
                       ct.c_int(sel.shape[1]), _p(quota), ct.c_int(R), ct.c_int(C), ct.c_int(n),
                       ct.c_int(E), _p(exp_idx))
    return exp_idx


def residual(K_bf16, V_bf16, asg, sel, exp_idx, quota, n_t, Sk, Sv, G: int):
    """multibin.py:2598-2642 (residual_stats='full') -> (kbar_r, vbar_r (R,C,D), log_n (R,C)) f64"""
    K, V = _c(K_bf16, np.uint16), _c(V_bf16, np.uint16)
    asg, sel, exp_idx = _c(asg, np.int32), _c(sel, np.int32), _c(exp_idx, np.int32)
    quota, n_t = _c(quota, np.float32), _c(n_t, np.float32)
    Sk, Sv = _c(Sk, np.float32), _c(Sv, np.float32)
    R, C = quota.shape
    kb = np.zeros((R, C, D), np.float64)
    vb = np.zeros((R, C, D), np.float64)
    ln = np.zeros((R, C), np.float64)
    _lib().oa_ref_residual(_p(K), _p(V), ct.c_int(K.shape[1]), _p(asg), _p(sel), ct.c_int(sel.shape[1]),
                           _p(exp_idx), ct.c_int(exp_idx.shape[1]), _p(quota), _p(n_t), _p(Sk), _p(Sv),
                           ct.c_int(R), ct.c_int(G), ct.c_int(C), _p(kb), _p(vb), _p(ln))
    return kb, vb, ln


def flash(q_bf16, K_bf16, V_bf16, sel, exp_idx, kbar, vbar, log_n, G: int, sm: float,
          proxy_per_kv: bool = False) -> np.ndarray:
    """multibin.py:2727-2747, methods_eager.py:708-720 (fp64) -> out (R,D) f64"""
    q, K, V = _c(q_bf16, np.uint16), _c(K_bf16, np.uint16), _c(V_bf16, np.uint16)
    sel, exp_idx = _c(sel, np.int32), _c(exp_idx, np.int32)
    kbar, vbar, log_n = _c(kbar, np.float64), _c(vbar, np.float64), _c(log_n, np.float64)
    R = q.shape[0]
    out = np.zeros((R, D), np.float64)
    _lib().oa_ref_flash(_p(q), _p(K), _p(V), ct.c_int(K.shape[1]), _p(sel), ct.c_int(sel.shape[1]),
                        _p(exp_idx), ct.c_int(exp_idx.shape[1]), _p(kbar), _p(vbar), _p(log_n),
                        ct.c_int(log_n.shape[1]), ct.c_int(1 if proxy_per_kv else 0), ct.c_int(R),
                        ct.c_int(G), ct.c_double(sm), _p(out))
    return out


def dense(q_bf16, K_bf16, V_bf16, n: int, G: int, sm: float) -> np.ndarray:
    q, K, V = _c(q_bf16, np.uint16), _c(K_bf16, np.uint16), _c(V_bf16, np.uint16)
    R = q.shape[0]
    out = np.zeros((R, D), np.float64)
    _lib().oa_ref_dense(_p(q), _p(K), _p(V), ct.c_int(K.shape[1]), ct.c_int(n), ct.c_int(R), ct.c_int(G),
                        ct.c_double(sm), _p(out))
    return out


def index_update(st: dict, pos: int, G: int, rmax: int) -> None:
    """ours_graph.py:43-90; mutates st['codes','asg','nb','Sk','Sk2','Sv','reclist','reccnt']"""
    names = ("codes", "asg", "nb", "Sk", "Sk2", "Sv", "reclist", "reccnt")
    for k in names:
        assert st[k].flags["C_CONTIGUOUS"]
    K, V = _c(st["K"], np.uint16), _c(st["V"], np.uint16)
    R, C = st["nb"].shape
    _lib().oa_ref_index_update(_p(K), _p(V), ct.c_int(K.shape[1]), ct.c_int(pos), ct.c_int(R), ct.c_int(G),
                               ct.c_int(C), _p(st["codes"]), _p(_c(st["U"], np.float32)),
                               _p(_c(st["scale"], np.float32)), _p(_c(st["W"], np.uint16)),
                               _p(_c(st["colmean"], np.float32)), _p(_c(st["cent"], np.float32)),
                               _p(st["asg"]), _p(st["nb"]), _p(st["Sk"]), _p(st["Sk2"]), _p(st["Sv"]),
                               _p(st["reclist"]), _p(st["reccnt"]), ct.c_int(rmax))


def index_downdate(st: dict, pos: int, G: int) -> None:
    """The token at pos leaves every query row's cluster statistics (multibin.py:2210-2218 tail
    validity, in the index update's fp32 terms); mutates st['nb','Sk','Sk2','Sv']"""
    for k in ("nb", "Sk", "Sk2", "Sv"):
        assert st[k].flags["C_CONTIGUOUS"] and st[k].dtype == np.float32
    K, V = _c(st["K"], np.uint16), _c(st["V"], np.uint16)
    R, C = st["nb"].shape
    asg = _c(st["asg"], np.int32)
    assert asg.shape[1] == K.shape[1]
    _lib().oa_ref_index_downdate(_p(K), _p(V), ct.c_int(K.shape[1]), ct.c_int(pos), ct.c_int(R), ct.c_int(G),
                                 ct.c_int(C), _p(asg), _p(st["nb"]), _p(st["Sk"]), _p(st["Sk2"]), _p(st["Sv"]))


# ------------------------------------------------------------------ prefill index build
def qgs_codes(K_bf16: np.ndarray, T: int, U: np.ndarray):
    """ours_fastbuild.py:256-261, static_top_k.py:174-181.  K (HKV, Lmax, 128) bf16 bits;
    U (HKV, 128, 32).  Returns codes (HKV, Lmax, 32) int8 (zero past T), scale (HKV, 32)."""
    K = _c(K_bf16, np.uint16)
    HKV, Lmax = K.shape[0], K.shape[1]
    U = _c(U, np.float32)
    codes = np.zeros((HKV, Lmax, RQ), np.int8)
    scale = np.zeros((HKV, RQ), np.float32)
    _lib().oa_ref_qgs_codes(_p(K), ct.c_int(Lmax), ct.c_int(HKV), ct.c_int(T), _p(U), _p(codes), _p(scale))
    return codes, scale


def qgc_zraw(K_bf16: np.ndarray, T: int, W_bf16: np.ndarray, G: int) -> np.ndarray:
    """bf16(k W) per query row (ours_fastbuild.py:264-275) with an exact product sum rounded once
    to fp32.  W (R, 128, 16) bf16 bits.  Returns (R, T, 16) bf16 bits."""
    K = _c(K_bf16, np.uint16)
    W = _c(W_bf16, np.uint16)
    R = W.shape[0]
    out = np.zeros((R, T, RC), np.uint16)
    _lib().oa_ref_qgc_zraw(_p(K), ct.c_int(K.shape[1]), ct.c_int(R), ct.c_int(G), ct.c_int(T), _p(W), _p(out))
    return out


def qgc_center(zraw_bf16: np.ndarray):
    """colmean (the device's fixed fp64 order) and zP = zraw - colmean (methods_eager.py:529-531).
    zraw (R, T, 16) bf16 bits.  Returns zP (R, T, 16) fp32, colmean (R, 16)."""
    zr = _c(zraw_bf16, np.uint16)
    R, T = zr.shape[0], zr.shape[1]
    zP = np.zeros((R, T, RC), np.float32)
    cm = np.zeros((R, RC), np.float32)
    _lib().oa_ref_qgc_center(_p(zr), ct.c_int(R), ct.c_int(T), _p(zP), _p(cm))
    return zP, cm


def kmeans_assign(zP: np.ndarray, cent: np.ndarray) -> np.ndarray:
    """ours_fastbuild.py:52-82 bf16 rule, ties to the lower cluster.  zP (R, T, 16); cent (R, C, 16)."""
    zP = _c(zP, np.float32)
    cent = _c(cent, np.float32)
    R, T = zP.shape[0], zP.shape[1]
    C = cent.shape[1]
    asg = np.zeros((R, T), np.int32)
    _lib().oa_ref_kmeans_assign(_p(zP), ct.c_int(R), ct.c_int(T), _p(cent), ct.c_int(C), _p(asg))
    return asg


def kmeans_update(zP: np.ndarray, asg: np.ndarray, C: int, init: np.ndarray):
    """ours_fastbuild.py:85-108: member means (fp64 sums in position order), empty -> zP[init].
    Returns cent (R, C, 16), cnt (R, C)."""
    zP = _c(zP, np.float32)
    asg = _c(asg, np.int32)
    init = _c(init, np.int32)
    R, T = zP.shape[0], zP.shape[1]
    cent = np.zeros((R, C, RC), np.float32)
    cnt = np.zeros((R, C), np.float32)
    _lib().oa_ref_kmeans_update(_p(zP), ct.c_int(R), ct.c_int(T), _p(asg), ct.c_int(C), _p(init), _p(cent), _p(cnt))
    return cent, cnt


def cluster_build(K_bf16: np.ndarray, V_bf16: np.ndarray, T: int, asg: np.ndarray, C: int, G: int):
    """ours_fastbuild.py:111-139, 293-301.  K, V (HKV, Lmax, 128) bf16 bits; asg (R, T).
    Returns nb, Sk, Sk2, Sv, mem (R, T), cstart, clen."""
    K, V = _c(K_bf16, np.uint16), _c(V_bf16, np.uint16)
    asg = _c(asg, np.int32)
    R = asg.shape[0]
    nb = np.zeros((R, C), np.float32)
    Sk, Sk2, Sv = (np.zeros((R, C, D), np.float32) for _ in range(3))
    mem = np.zeros((R, T), np.int32)
    cstart = np.zeros((R, C), np.int32)
    clen = np.zeros((R, C), np.int32)
    _lib().oa_ref_cluster_build(_p(K), _p(V), ct.c_int(K.shape[1]), ct.c_int(R), ct.c_int(G), ct.c_int(T),
                                _p(asg), ct.c_int(C), _p(nb), _p(Sk), _p(Sk2), _p(Sv), _p(mem), _p(cstart),
                                _p(clen))
    return nb, Sk, Sk2, Sv, mem, cstart, clen


# ------------------------------------------------------------------ a10: metric and bases (fp64)
# An independent restatement with explicit rotation matrices and numpy's eigh; the product's
# host code (openattention_amd/prefill.py) forms the same quantities another way, in fp32/fp64
# torch on the device.  tests/test_a10_pins.py compares the two and pins this one to the
# mathematics.
WIN, P_ROWS = 32, 64


def rope_matrix(inv_freq: np.ndarray, scaling: float, pos: int) -> np.ndarray:
    """R_pos = s (diag(cos pos theta) + diag(sin pos theta) J), theta = [inv_freq, inv_freq],
    J = [[0, -I], [I, 0]] (UTAMultiBinAttention._rope_matrix, multibin.py:1606-1615)."""
    th = np.concatenate([inv_freq, inv_freq]).astype(np.float64)
    h = th.size // 2
    J = np.zeros((2 * h, 2 * h))
    J[:h, h:] = -np.eye(h)
    J[h:, :h] = np.eye(h)
    ang = float(pos) * th
    return float(scaling) * (np.diag(np.cos(ang)) + np.diag(np.sin(ang)) @ J)


def static_metric_at(M_pre: np.ndarray, inv_freq, scaling: float, T: int, w: int = WIN) -> np.ndarray:
    """mean_{t in [T, T+w)} R_t M R_t^T by the explicit loop (multibin.py:1687-1692), fp64."""
    M = np.asarray(M_pre, np.float64)
    acc = np.zeros_like(M)
    for t in range(T, T + w):
        R = rope_matrix(inv_freq, scaling, t)
        acc += R @ M @ R.T
    return acc / w


def question_moment(qrows: np.ndarray, inv_freq, scaling: float) -> np.ndarray:
    """M_q of static_top_k.py:185-194 / multibin.py:1674-1680: the picked question rows (H, Qn,
    D), row i advanced by an explicit R_{Qn-i}, averaged outer products, fp64."""
    import torch
    Qn = qrows.shape[1]
    P = min(P_ROWS, max(Qn - 2, 1))
    picks = torch.linspace(0, max(Qn - 3, 0), P, dtype=torch.float32).long().unique().numpy()
    q = np.asarray(qrows, np.float64)
    out = np.zeros((q.shape[0], q.shape[2], q.shape[2]))
    for i in picks:
        r = q[:, i, :] @ rope_matrix(inv_freq, scaling, Qn - int(i)).T         # (H, D): R q_i
        out += r[:, :, None] * r[:, None, :]
    return out / len(picks)


def query_metric(M_pre, qrows, T: int, inv_freq, scaling: float) -> np.ndarray:
    """M = 1/2 M_st / tr(M_st) + 1/2 M_q / tr(M_q) (methods_eager.py:511-518), fp64."""
    def nt(x):
        return x / np.maximum(np.trace(x, axis1=-2, axis2=-1), 1e-12)[..., None, None]
    return 0.5 * nt(static_metric_at(M_pre, inv_freq, scaling, T)) + 0.5 * nt(question_moment(qrows, inv_freq, scaling))


def bases(M: np.ndarray, HKV: int, G: int):
    """U (HKV, D, 32): eigenvectors of the 32 largest eigenvalues of the mean of each KV
    group's G metrics (methods_eager.py:519-520, StaticTopKMasker._build share_kv,
    static_top_k.py:155-162); W (HQ, D, 16): eigenvectors of the 16 largest eigenvalues of each
    head's metric scaled by sqrt(max(lambda, 0)) (methods_eager.py:527-528,
    multibin.py:1704-1712).  numpy eigh, fp64; eigenvalues ascending."""
    Mg = M.reshape(HKV, G, *M.shape[-2:]).mean(1)
    _, Ug = np.linalg.eigh(Mg)
    ev, Uq = np.linalg.eigh(M)
    U = Ug[..., -RQ:]
    W = Uq[..., -RC:] * np.sqrt(np.maximum(ev[..., -RC:], 0.0))[..., None, :]
    return U, W


def kmeans_init(T: int, C: int, layer: int) -> np.ndarray:
    """The first C of torch.randperm(T) under the generator seeded 1234 + 31 (layer + 1)
    (multibin.py:1894-1895)."""
    import torch
    g = torch.Generator(device="cpu").manual_seed(1234 + 31 * (layer + 1))
    return torch.randperm(T, generator=g)[:C].numpy().astype(np.int32)


def build_row(st, b: int, K, V, qrows, T: int, M_pre, inv_freq, scaling: float, layer: int,
              G: int = 4, iters: int = 4) -> None:
    """CPU counterpart of openattention_amd.prefill.build_row: the restated metric and bases
    (a10, fp64 above; U stored in fp32 and W in bf16 as the state holds them) and the restated
    codes, projection, k-means and cluster statistics (a11-a13).  st: a LayerState on the CPU;
    K, V: (HKV, >=T, 128) bf16 torch tensors; qrows (HQ, Qn, 128)."""
    import torch
    HKV = K.shape[0]
    HQ = HKV * G
    C = st.C
    M = query_metric(np.asarray(M_pre, np.float64), qrows.float().numpy(), T,
                     np.asarray(inv_freq, np.float64), scaling)
    U64, W64 = bases(M, HKV, G)
    U = torch.from_numpy(U64.astype(np.float32))
    W = torch.from_numpy(W64.astype(np.float32)).to(torch.bfloat16)
    kb = K.contiguous().view(torch.int16).numpy().view(np.uint16)
    vb = V.contiguous().view(torch.int16).numpy().view(np.uint16)
    Wb = W.contiguous().view(torch.int16).numpy().view(np.uint16)
    codes, scale = qgs_codes(kb, T, U.numpy())
    zP, cm = qgc_center(qgc_zraw(kb, T, Wb, G))
    if T < C:
        raise ValueError(f"the prefix ({T} tokens) must hold at least C = {C} tokens")
    init = kmeans_init(T, C, layer)
    cent = zP[:, init].copy()
    for _ in range(iters):
        asg = kmeans_assign(zP, cent)
        cent, _cnt = kmeans_update(zP, asg, C, init)
    nb, Sk, Sk2, Sv, mem, cstart, clen = cluster_build(kb, vb, T, asg, C, G)
    r0, q0 = b * HKV, b * HQ
    st.codes[r0:r0 + HKV, :T] = torch.from_numpy(codes[:, :T])
    st.U[r0:r0 + HKV] = U
    st.scale[r0:r0 + HKV] = torch.from_numpy(scale)
    st.W[q0:q0 + HQ] = W
    st.colmean[q0:q0 + HQ] = torch.from_numpy(cm)
    st.cent[q0:q0 + HQ] = torch.from_numpy(cent)
    st.asg[q0:q0 + HQ, :T] = torch.from_numpy(asg)
    st.asg8[q0:q0 + HQ, :T] = torch.from_numpy(asg.astype(np.uint8))
    st.nb[q0:q0 + HQ] = torch.from_numpy(nb)
    st.Sk[q0:q0 + HQ] = torch.from_numpy(Sk)
    st.Sk2[q0:q0 + HQ] = torch.from_numpy(Sk2)
    st.Sv[q0:q0 + HQ] = torch.from_numpy(Sv)
    st.mem[q0:q0 + HQ, :T] = torch.from_numpy(mem)
    st.cstart[q0:q0 + HQ] = torch.from_numpy(cstart)
    st.clen[q0:q0 + HQ] = torch.from_numpy(clen)
    st.reccnt[q0:q0 + HQ] = 0


# ------------------------------------------------------------------ composition
def decode_step(st: dict, q_bf16: np.ndarray, n: int, ns: int, nl: int, k: int, E: int, G: int,
                sm: float, sm2: float, rmax: int = 256, update_index: bool = True) -> dict:
    """The deployed decode step of one layer (ours_graph.py:290-347) with multibin decision
    semantics: index update of position n-1, QGS scores, top-k, ErrorGate, water-filling,
    within-cluster top-q, residual proxies, merge softmax.  Mutates the index state in st when
    update_index is set.  Returns every intermediate."""
    Lk = st["K"].shape[1]
    if not (st["asg"].shape[1] == st["codes"].shape[1] == st["V"].shape[1] == Lk):
        raise ValueError("decode_step: K, V, asg and codes must share one Lmax (row length); got "
                         f"{Lk}, {st['V'].shape[1]}, {st['asg'].shape[1]}, {st['codes'].shape[1]}")
    if update_index:
        index_update(st, n - 1, G, rmax)
    zq, fexp, Z = qgs_prep(q_bf16, st["U"], st["scale"], G)
    S = qgs_scores(st["codes"], Z, fexp, G, n, ns, nl)
    sel = topk_select(S, n, ns, nl, k)
    score, n_t = errorgate(q_bf16, st["K"], st["asg"], sel, st["Sk"], st["Sk2"], st["nb"], G, sm, sm2)
    quota = waterfill(score, n_t, E)
    exp_idx = topq(S, st["asg"], sel, quota, n, E)
    kb, vb, ln = residual(st["K"], st["V"], st["asg"], sel, exp_idx, quota, n_t, st["Sk"], st["Sv"], G)
    out = flash(q_bf16, st["K"], st["V"], sel, exp_idx, kb, vb, ln, G, sm)
    return dict(zq=zq, fexp=fexp, Z=Z, S=S, sel=sel, score=score, n_t=n_t, quota=quota,
                exp_idx=exp_idx, kbar_r=kb, vbar_r=vb, log_n=ln, out=out)


def rows_step(st: dict, q_rows: np.ndarray, n_keys: int, ns: int, nl: int, k: int, E: int, G: int,
              sm: float, sm2: float, rows=None) -> dict:
    """A multi-row call of the estimator (UTAMultiBinAttention.custom_attention with Q query rows,
    multibin.py:2875-2970 over the masks of basic_fixed.py:180-214, 384-418 and
    static_top_k.py:221-262): query row i (q_rows[i], (R, 128) bf16 bits) sits at position
    n_keys - Q + i and, with the causal mask, attends the n_i = n_keys - Q + i + 1 keys before it:
    sink, local window [n_i - nl, n_i) and top-k over [ns, n_i - nl), sizes fixed by the call's
    key count (ns, nl, k); its tail, bins and statistics hold keys below n_i only.  The index in
    st holds all n_keys keys; row i's statistics are those of [0, n_keys) with the keys
    n_keys - 1, ..., n_i taken back (index_downdate), and the rows run from the last to the
    first.  st is not modified.  Returns {i: decode_step results of row i} for the rows asked
    (all by default)."""
    Q = q_rows.shape[0]
    want = set(range(Q)) if rows is None else set(rows)
    s = dict(st)
    for f in ("nb", "Sk", "Sk2", "Sv"):
        s[f] = st[f].copy()
    res = {}
    for i in range(Q - 1, -1, -1):
        n_i = n_keys - Q + i + 1
        if i in want:
            res[i] = decode_step(s, q_rows[i], n_i, ns, nl, k, E, G, sm, sm2, update_index=False)
        if i > 0:
            index_downdate(s, n_i - 1, G)
        if not any(j < i for j in want):
            break
    return res
