"""Per-request index build at prefill (QGS codes, QGC clusters, cluster sums, CSR lists).

Follows the deployed build (inference/methods_eager.py:505-555, inference/ours_fastbuild.py:
199-304) with the accuracy-path choices where the two differ (k-means seed 1234 + 31(l+1) of
multibin.py:1894):
  a10  M_st rotated to the decode position T and averaged over a window of w = 32 positions
       (StaticTopKMasker._rot_avg, static_top_k.py:103-131); M_q from P <= 64
       question rows, each rotated to T (static_top_k.py:185-194); M = 1/2 nt(M_st) + 1/2
       nt(M_q), nt = trace normalisation; U = top-32 eigenvectors of the group-mean M per KV
       head; W = top-16 eigenvectors * sqrt(eigenvalue) per query head, in bf16.  The rotated
       static metric in torch on the device, the question moments, blend and group means by
       oa_query_metric, the eigenpairs by oa_sym_eig_top (one-sided Jacobi).
  a11  codes: oa_qgs_codes (zc = k U, scale = max(max_t |zc| / 127, 1e-12), codes =
       clamp(rint(zc / scale), -127, 127); static_top_k.py:174-181).
  a12  oa_qgc_project (zP = bf16(k W) - colmean on the bf16 matrix cores), then 4 Lloyd
       iterations of oa_kmeans_assign (bf16 distance bf16(bf16(zP . c) - bf16(|c|^2 / 2)), ties
       to the lower cluster) and oa_kmeans_update (member means; an empty cluster keeps its
       initial point) (methods_eager.py:526-547).
  a13  oa_cluster_build: n_b, sum k, sum k^2, sum v per cluster and the CSR member lists
       (ours_fastbuild.py:293-301).
The a11-a13 stages run only on the HIP kernels (a tensor on another device raises).  The
decode stage's parity tests inject one built state into both the GPU kernels and the CPU
restatement; the build stages have their own parity tests.
"""
from __future__ import annotations

import torch

D = 128
RQ, RC = 32, 16
WIN = 32
P_ROWS = 64
ITERS = 4


def rope_trig(inv_freq: torch.Tensor, positions: torch.Tensor):
    """cos and sin of the RoPE angles t * theta_i (fp64), theta = [inv_freq, inv_freq]: the
    rotation by t positions acts on x as R_t x = s (cos * x + sin * rotate_half(x)), s the
    attention scaling (static_top_k.py:91-100 applies the same rotation to the question rows).
    positions: (P,) -> two (P, D) tensors."""
    theta = torch.cat([inv_freq, inv_freq]).to(torch.float64)
    ang = positions.to(torch.float64).unsqueeze(-1) * theta.to(positions.device)
    return ang.cos(), ang.sin()


def rotate_half(x: torch.Tensor, dim: int = -1) -> torch.Tensor:
    """J x along `dim`, J = [[0, -I], [I, 0]]: the second half, negated, then the first half.
    Along dim -2 of a matrix it is J M; along dim -1 it is M J^T."""
    a, b = x.chunk(2, dim=dim)
    return torch.cat([-b, a], dim=dim)


def rot_avg(M_pre: torch.Tensor, inv_freq: torch.Tensor, scaling: float, p: int, w: int = WIN):
    """The static metric seen from decode position p: mean over t in [p, p + w) of
    R_t M R_t^T (StaticTopKMasker._rot_avg, static_top_k.py:103-131; the explicit loop of
    multibin.py:1687-1692).

    With R_t = s (diag(c_t) + diag(s_t) J), entry (i, j) of R_t M R_t^T is
      s^2 (c_i c_j M + c_i s_j (M J^T) + s_i c_j (J M) + s_i s_j (J M J^T))_ij,
    so the window mean needs only the four window means of the trigonometric outer products,
    E[c c^T], E[c s^T], E[s c^T] = E[c s^T]^T and E[s s^T]: (w, D) x (D, w) products in fp64."""
    t = torch.arange(p, p + w, device=M_pre.device, dtype=torch.float64)
    c, sn = rope_trig(inv_freq.to(M_pre.device), t)                        # (w, D) each
    s2 = float(scaling) * float(scaling) / w
    a_cc = (c.T @ c) * s2
    a_cs = (c.T @ sn) * s2
    a_ss = (sn.T @ sn) * s2
    M = M_pre.float()
    JM = rotate_half(M, -2)
    return (a_cc.float() * M + a_cs.float() * rotate_half(M, -1) + a_cs.T.float() * JM
            + a_ss.float() * rotate_half(JM, -1))


def question_picks(Qn: int, device) -> torch.Tensor:
    """Indices of the question rows the moment uses: P = min(64, max(Qn - 2, 1)) points spread
    evenly over [0, Qn - 3], truncated to integers, duplicates dropped -- the reference's pick
    rule (static_top_k.py:188-189), with torch.linspace's fp32 points so the picks agree."""
    P = min(P_ROWS, max(Qn - 2, 1))
    return torch.linspace(0, max(Qn - 3, 0), P, device=device, dtype=torch.float32).long().unique()


def question_moment(qrows: torch.Tensor, inv_freq: torch.Tensor, scaling: float) -> torch.Tensor:
    """M_q = mean over the picked question rows of (R_{Qn-i} q_i)(R_{Qn-i} q_i)^T: row i sits at
    position T - Qn + i and is advanced by Qn - i positions to the decode position T
    (static_top_k.py:185-194).  qrows (H, Qn, D) -> (H, D, D) fp32 (rotation and products in
    fp64)."""
    Qn = qrows.shape[-2]
    pick = question_picks(Qn, qrows.device)
    q = qrows.index_select(-2, pick).to(torch.float64)                    # (H, P, D)
    c, sn = rope_trig(inv_freq.to(qrows.device), (Qn - pick).to(qrows.device))
    r = float(scaling) * (c * q + sn * rotate_half(q, -1))
    return (r.transpose(-1, -2) @ r / pick.numel()).float()


def trace_norm(x: torch.Tensor) -> torch.Tensor:
    """x / tr(x) per matrix, the trace floored at 1e-12 (the blend of methods_eager.py:518)."""
    tr = torch.diagonal(x, dim1=-2, dim2=-1).sum(-1)
    return x / tr.clamp(min=1e-12).unsqueeze(-1).unsqueeze(-1)


def query_metric(M_pre: torch.Tensor, qrows: torch.Tensor, T: int, inv_freq, scaling) -> torch.Tensor:
    """M = 1/2 nt(M_st rotated to T) + 1/2 nt(M_q)  (methods_eager.py:511-518)."""
    Mst = rot_avg(M_pre, inv_freq, scaling, T, WIN)
    Mq = question_moment(qrows, inv_freq, scaling)
    return 0.5 * trace_norm(Mst) + 0.5 * trace_norm(Mq)


def kmeans_seed(layer: int) -> int:
    """multibin.py:1894 (accuracy path); the deployed build uses 31 * (layer + 1)."""
    return 1234 + 31 * (layer + 1)


def basis_matrices(M: torch.Tensor, HKV: int, G: int) -> torch.Tensor:
    """The matrices the bases come from: the HKV group means of the per-query-head metric M
    (HQ, D, D) (methods_eager.py:519), then the HQ metrics themselves (methods_eager.py:527)."""
    return torch.cat([M.view(HKV, G, D, D).mean(1), M], 0)


def bases_from_eigenpairs(ev: torch.Tensor, vec: torch.Tensor, HKV: int):
    """U, W from the top eigenpairs of basis_matrices' output, ascending (the last columns of an
    eigh): U (HKV, D, 32) = the top-32 eigenvectors of each group mean (methods_eager.py:519-520),
    W (HQ, D, 16) bf16 = the top-16 eigenvectors * sqrt(eigenvalue) of each metric
    (methods_eager.py:527-528)."""
    U = vec[:HKV, :, -RQ:].contiguous()
    evq, Uq = ev[HKV:], vec[HKV:]
    W = (Uq[..., -RC:] * evq[..., -RC:].clamp(min=0).sqrt().unsqueeze(-2)).to(torch.bfloat16).contiguous()
    return U, W


def bases(M: torch.Tensor, HKV: int, G: int):
    """a10 bases from the per-query-head metric M (HQ, D, D) on a HIP device: the top-32
    eigenpairs of the HKV group means and the HQ metrics from one launch of the library's
    Jacobi eigensolver (oa_sym_eig_top: one workgroup per matrix, each decomposed on its own),
    then bases_from_eigenpairs.  The metric is a positive blend of second-moment matrices
    (positive semi-definite), which the solver requires."""
    from openattention_amd import ops
    ev, vec = ops.sym_eig_top(basis_matrices(M, HKV, G).contiguous(), RQ)
    return bases_from_eigenpairs(ev, vec, HKV)


def _h2d(x: torch.Tensor, dev) -> torch.Tensor:
    """x on dev; a host tensor goes through pinned memory without waiting for the stream (a
    pageable copy makes the host wait for every queued launch, and the device then idles while the
    next launches are issued)."""
    if x.device.type != "cpu" or torch.device(dev).type == "cpu":
        return x.to(dev)
    return x.pin_memory().to(dev, non_blocking=True)


_CONSTS: dict = {}


def _metric_consts(T: int, Qn: int, inv_freq: torch.Tensor, scaling: float, dev):
    """What the device metric needs that depends on T, Qn, the RoPE frequencies and the scaling
    only, formed once per such tuple and device (a host inv_freq is the key; a device one is not
    cached): rot_avg's four window-mean coefficient matrices in fp32 with rotate_half's signs
    folded in, rotate_half's index map (J x = sgn * x[perm]), the question picks and their RoPE
    cos / sin."""
    key = None
    if inv_freq.device.type == "cpu":
        key = (int(T), int(Qn), float(scaling), inv_freq.to(torch.float64).numpy().tobytes(),
               str(torch.device(dev)))
        hit = _CONSTS.get(key)
        if hit is not None:
            return hit
    invd = _h2d(inv_freq, dev)
    t = torch.arange(T, T + WIN, device=dev, dtype=torch.float64)
    c, sn = rope_trig(invd, t)                                               # (WIN, D) each
    s2 = float(scaling) * float(scaling) / WIN
    a_cc = (c.T @ c) * s2
    a_cs = (c.T @ sn) * s2
    a_ss = (sn.T @ sn) * s2
    half = D // 2
    perm = torch.cat([torch.arange(half, D, device=dev), torch.arange(0, half, device=dev)])
    sgn = torch.ones(D, device=dev, dtype=torch.float64)
    sgn[:half] = -1.0
    # a * (-m) == (-a) * m exactly, so these products are rot_avg's bit for bit
    coef = (a_cc.float(), (a_cs * sgn[None, :]).float(), (a_cs.T * sgn[:, None]).float(),
            (a_ss * sgn[:, None] * sgn[None, :]).float())
    pick = question_picks(Qn, "cpu")
    pick_d = _h2d(pick.to(torch.int32), dev)
    cq, sq = rope_trig(invd, Qn - pick_d)
    out = (coef, perm, pick_d, cq.contiguous(), sq.contiguous())
    if key is not None:
        if len(_CONSTS) >= 16:
            _CONSTS.clear()
        _CONSTS[key] = out
    return out


def static_half(M_pre: torch.Tensor, T: int, inv_freq: torch.Tensor, scaling: float, dev,
                Qn: int = 1) -> torch.Tensor:
    """1/2 trace_norm(rot_avg(M_pre, ..., T, WIN)) on dev, bit-identical to that expression:
    with the cached coefficients the rotated metric is four products of M, M[:, perm],
    M[perm, :] and M[perm][:, perm] (rotate_half as a gather), summed in rot_avg's order."""
    (A1, A2, A3, A4), perm = _metric_consts(T, Qn, inv_freq, scaling, dev)[:2]
    M = _h2d(M_pre, dev).float()
    Mr = M.index_select(-2, perm)
    raw = A1 * M + A2 * M.index_select(-1, perm) + A3 * Mr + A4 * Mr.index_select(-1, perm)
    return 0.5 * trace_norm(raw)


def metric_device(M_pre: torch.Tensor, qrows: torch.Tensor, T: int, inv_freq: torch.Tensor,
                  scaling: float, G: int, gm_out=None, m_out=None):
    """query_metric on the library's kernel for every query-head row of qrows (R, Qn, D) (R =
    KV rows * G, row r using head r % HQ of M_pre (HQ, D, D)): the rotated static metric's half
    is formed once here in torch (query_metric's arithmetic), the question moments, the blend and
    each KV row's group mean by oa_query_metric.  Returns (group means (R / G, D, D), metrics
    (R, D, D)), into gm_out / m_out when given: basis_matrices' two parts."""
    from openattention_amd import ops
    dev = qrows.device
    Qn = qrows.shape[-2]
    # the picks depend on Qn only: chosen on the host (on the device, unique() waits for the
    # queue to drain to size its output), with the other T / Qn constants, once
    _, _, pick_d, c, sn = _metric_consts(T, Qn, inv_freq, scaling, dev)
    mst = static_half(M_pre, T, inv_freq, scaling, dev, Qn).contiguous()
    return ops.query_metric(qrows, pick_d, c, sn, scaling, mst, G, gm_out, m_out)


def kmeans_init(T: int, C: int, layer: int) -> torch.Tensor:
    """Initial centroid positions: the first C of a seeded permutation of the T tokens
    (multibin.py:1894-1895; CPU generator, as the reference)."""
    if T < C:
        raise ValueError(f"the prefix ({T} tokens) must hold at least C = {C} tokens")
    g = torch.Generator(device="cpu").manual_seed(kmeans_seed(layer))
    return torch.randperm(T, generator=g)[:C]


@torch.no_grad()
def build_row(st, b: int, K: torch.Tensor, V: torch.Tensor, qrows: torch.Tensor, T: int,
              M_pre: torch.Tensor, inv_freq: torch.Tensor, scaling: float, layer: int,
              G: int = 4, marks: list | None = None) -> None:
    """Build batch row b of one layer's index into `st` (a LayerState on a HIP device).

    K, V: (HKV, >=T, D) bf16 of this batch row; qrows: (HQ, Qn, D) question rows.
    marks: if a list, (stage, event) pairs are appended, recorded on the current stream after
    each stage (per-stage timing).
    """
    def mark(name):
        if marks is not None:
            e = torch.cuda.Event(enable_timing=True)
            e.record()
            marks.append((name, e))

    from openattention_amd import ops
    dev = K.device
    if dev.type != "cuda":
        raise RuntimeError("the index build runs on the HIP kernels: K, V must be on a HIP device")
    HKV = K.shape[0]
    HQ = HKV * G
    if marks is not None:
        mark("start")
    gm, M = metric_device(M_pre, qrows, T, inv_freq, scaling, G)                  # (HKV / HQ, D, D)
    mark("metric")
    ev, vec = ops.sym_eig_top(torch.cat([gm, M], 0), RQ)
    U, W = bases_from_eigenpairs(ev, vec, HKV)
    st.U[b * HKV:(b + 1) * HKV] = U
    st.W[b * HQ:(b + 1) * HQ] = W
    mark("bases")
    _build_device(st, b * HKV, K, V, T, layer, G, mark)


@torch.no_grad()
def build_rows(st, K: torch.Tensor, V: torch.Tensor, qrows: torch.Tensor, T: int,
               M_pre: torch.Tensor, inv_freq: torch.Tensor, scaling: float, layer: int,
               G: int = 4, marks: list | None = None) -> None:
    """build_row for every batch row of one layer at once: the bases of all rows from one
    eigensolver launch (one workgroup per matrix), then each HIP stage
    over all B * HQ rows in one launch (the stages are row-parallel: one launch per stage
    instead of one per stage and row).

    K, V: (B, HKV, >=T, D) bf16, contiguous; qrows: (B, HQ, Qn, D).  Same state as build_row
    row by row."""
    def mark(name):
        if marks is not None:
            e = torch.cuda.Event(enable_timing=True)
            e.record()
            marks.append((name, e))

    from openattention_amd import ops
    dev = K.device
    if dev.type != "cuda":
        raise RuntimeError("the index build runs on the HIP kernels: K, V must be on a HIP device")
    B, HKV = K.shape[0], K.shape[1]
    HQ = HKV * G
    if not (K.is_contiguous() and V.is_contiguous() and K.shape == V.shape and K.dim() == 4):
        raise ValueError("build_rows: K and V must be contiguous (B, HKV, Lmax, D) tensors")
    if B * HKV > st.U.shape[0] or qrows.shape[0] != B or qrows.shape[1] != HQ:
        raise ValueError("build_rows: K, qrows and the state disagree on B, HKV or HQ")
    mark("start")
    # the rotated static metric depends on the layer and T only: formed once for all rows
    Mall = torch.empty(B * HKV + B * HQ, D, D, device=dev)
    metric_device(M_pre, qrows.reshape(B * HQ, qrows.shape[2], D), T, inv_freq, scaling, G,
                  Mall[:B * HKV], Mall[B * HKV:])
    mark("metric")
    ev, vec = ops.sym_eig_top(Mall, RQ)
    U, W = bases_from_eigenpairs(ev, vec, B * HKV)
    st.U[:B * HKV] = U
    st.W[:B * HQ] = W
    mark("bases")
    _build_device(st, 0, K.reshape(B * HKV, K.shape[2], D), V.reshape(B * HKV, V.shape[2], D), T,
                  layer, G, mark)


def build_layers(states, Ks, Vs, qrows, T: int, M_pre: torch.Tensor, inv_freq: torch.Tensor,
                 scaling: float, layers, G: int = 4) -> None:
    """build_rows for several layers at once: every layer's metric first, then the bases of all
    layers and rows from one eigensolver launch (at B = 1 a layer's 40 matrices would hold 40 of
    the 256 compute units; 32 layers' 1280 fill them), then each
    layer's HIP stages.  states[i], Ks[i], Vs[i], qrows[i] belong to layer layers[i]; M_pre is
    the (L, HQ, D, D) static metric of every layer."""
    if not (len(states) == len(Ks) == len(Vs) == len(qrows) == len(layers)) or not layers:
        raise ValueError("build_layers: one state, K, V, question block and layer index per layer")
    from openattention_amd import ops
    dev = Ks[0].device
    if dev.type != "cuda":
        raise RuntimeError("the index build runs on the HIP kernels: K, V must be on a HIP device")
    B, HKV = Ks[0].shape[0], Ks[0].shape[1]
    HQ = HKV * G
    nl = len(layers)
    # every layer's group means first, then every layer's head metrics (basis_matrices' order)
    Mall = torch.empty(nl * (B * HKV + B * HQ), D, D, device=dev)
    for i, (st, K, V, q, layer) in enumerate(zip(states, Ks, Vs, qrows, layers)):
        if not (K.is_contiguous() and V.is_contiguous() and K.shape == V.shape and K.dim() == 4
                and K.shape[:2] == (B, HKV)):
            raise ValueError("build_layers: K and V must be contiguous (B, HKV, Lmax, D) tensors of one shape")
        if B * HKV > st.U.shape[0] or q.shape[0] != B or q.shape[1] != HQ:
            raise ValueError("build_layers: K, qrows and the state disagree on B, HKV or HQ")
        g0, m0 = i * B * HKV, nl * B * HKV + i * B * HQ
        metric_device(M_pre[layer], q.reshape(B * HQ, q.shape[2], D), T, inv_freq, scaling, G,
                      Mall[g0:g0 + B * HKV], Mall[m0:m0 + B * HQ])
    ev, vec = ops.sym_eig_top(Mall, RQ)
    U, W = bases_from_eigenpairs(ev, vec, nl * B * HKV)
    for i, (st, K, V, layer) in enumerate(zip(states, Ks, Vs, layers)):
        st.U[:B * HKV] = U[i * B * HKV:(i + 1) * B * HKV]
        st.W[:B * HQ] = W[i * B * HQ:(i + 1) * B * HQ]
        _build_device(st, 0, K.reshape(B * HKV, K.shape[2], D), V.reshape(B * HKV, V.shape[2], D), T,
                      layer, G, lambda name: None)


def _build_device(st, r0: int, K: torch.Tensor, V: torch.Tensor, T: int, layer: int, G: int,
                  mark) -> None:
    """a11-a13 on the HIP kernels for the KV rows r0 .. r0 + K.shape[0] of st (their query-head
    rows G times as many, from G * r0), from the U and W already in st."""
    from openattention_amd import ops
    dev = K.device
    HKV = K.shape[0]
    HQ = HKV * G
    C = st.C
    q0 = r0 * G
    # a11: QGS codes and scale
    amax = torch.empty(HKV * RQ, device=dev, dtype=torch.int32)
    zc = torch.empty(HKV * T * RQ, device=dev)          # k U kept between the two passes
    ops.qgs_codes(K, T, st.U[r0:r0 + HKV], st.codes[r0:r0 + HKV], st.scale[r0:r0 + HKV], amax, zc)
    del zc
    mark("codes")
    # a12: QGC projection and k-means
    # the projection is kept as its bf16 values; the k-means kernels form zP = bf16(k W) - colmean
    # (fp32) as they read it
    zraw = torch.empty(HQ, T, RC, device=dev, dtype=torch.bfloat16)
    colmean = st.colmean[q0:q0 + HQ]
    ops.qgc_project(K, T, st.W[q0:q0 + HQ], G, zraw, colmean)
    mark("project")
    init = _h2d(kmeans_init(T, C, layer).to(torch.int32), dev)
    cent = st.cent[q0:q0 + HQ]
    cent.copy_(zraw.index_select(1, init.long()).float() - colmean[:, None, :])
    asg, asg8 = st.asg[q0:q0 + HQ], st.asg8[q0:q0 + HQ]
    mark("kmeans_init")
    for _ in range(ITERS):
        ops.kmeans_assign(zraw, colmean, T, cent, asg, asg8)
        mark("kmeans_assign")
        ops.kmeans_update(zraw, colmean, T, asg8, init, cent, st.mem[q0:q0 + HQ], st.cstart[q0:q0 + HQ],
                          st.clen[q0:q0 + HQ])
        mark("kmeans_update")
    # a13: cluster statistics; the CSR member lists are the last update's (the assignment did not
    # change after it), so they are not sorted again
    ops.cluster_sums(K, V, T, G, C, st.nb[q0:q0 + HQ], st.Sk[q0:q0 + HQ], st.Sk2[q0:q0 + HQ],
                     st.Sv[q0:q0 + HQ], st.mem[q0:q0 + HQ], st.cstart[q0:q0 + HQ], st.clen[q0:q0 + HQ])
    st.reccnt[q0:q0 + HQ] = 0
    mark("cluster_build")


class LayerState:
    """One layer's decode index for all B batch rows (rows flattened: KV rows b*HKV + h,
    query-head rows b*HQ + h)."""

    FIELDS = ("codes", "U", "scale", "W", "colmean", "cent", "asg", "asg8", "nb", "Sk", "Sk2", "Sv",
              "mem", "cstart", "clen", "reclist", "reccnt")

    def __init__(self, B: int, HKV: int, G: int, Lmax: int, C: int, rmax: int, dev):
        BH, R = B * HKV, B * HKV * G
        if C > 256:
            raise ValueError("at most 256 clusters (cluster ids are also kept as bytes)")
        self.B, self.HKV, self.G, self.Lmax, self.C, self.rmax = B, HKV, G, Lmax, C, rmax
        z = lambda *s, dt=torch.float32: torch.zeros(*s, device=dev, dtype=dt)  # noqa: E731
        self.codes = z(BH, Lmax, RQ, dt=torch.int8)
        self.U = z(BH, D, RQ)
        self.scale = z(BH, RQ)
        self.W = z(R, D, RC, dt=torch.bfloat16)
        self.colmean = z(R, RC)
        self.cent = z(R, C, RC)
        self.asg = z(R, Lmax, dt=torch.int32)
        # byte ids are streamed four at a time: rows padded to a multiple of 64 entries
        self.asg8 = z(R, -(-Lmax // 64) * 64, dt=torch.uint8)
        self.nb = z(R, C)
        self.Sk = z(R, C, D)
        self.Sk2 = z(R, C, D)
        self.Sv = z(R, C, D)
        self.mem = z(R, Lmax, dt=torch.int32)
        self.cstart = z(R, C, dt=torch.int32)
        self.clen = z(R, C, dt=torch.int32)
        self.reclist = z(R, C, max(rmax, 1), dt=torch.int32)
        self.reccnt = z(R, C, dt=torch.int32)

    def to_numpy(self) -> dict:
        return {f: getattr(self, f).detach().cpu().contiguous().numpy().copy()
                if getattr(self, f).dtype != torch.bfloat16 else
                getattr(self, f).detach().cpu().contiguous().view(torch.int16).numpy().view("uint16").copy()
                for f in self.FIELDS}

    def clone(self) -> "LayerState":
        new = LayerState.__new__(LayerState)
        new.__dict__.update({k: (v.clone() if torch.is_tensor(v) else v) for k, v in self.__dict__.items()})
        return new
