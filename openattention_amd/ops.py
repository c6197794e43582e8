"""torch-tensor front end of the gfx950 kernels.

Operator surface kept from the reference:
  ours_flash(q, k, v, sel_idx, exp_idx, kbar, vbar, log_n, nb=None)      methods_eager.py:161-172
  decode_expand_attention(q, k, v, sel_idx, exp_idx, kbar, vbar, log_n,
                          sm_scale=None, block_n=64, block_b=64, num_warps=4)
                                                                        triton_expand_decode.py:139-165
plus one function per decode stage (index_update, qgs_prep, qgs_scan, topk_select, errorgate,
waterfill, topq, residual, residual_flash, dense_decode), each a thin checked call of the C ABI
(include/openattention_amd.h) on torch's current HIP stream.  Shape, dtype, device, alignment
and stride checks happen here; the kernels trust them.  There is no CPU path: tensors must live
on a HIP device and the kernel library must be built.
"""
from __future__ import annotations

import torch

from openattention_amd import lib

HEAD_DIM = 128
RANK_Q = 32
RANK_C = 16
GROUP = 4


def _ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def _stream(dev: torch.device):
    return torch.cuda.current_stream(dev).cuda_stream


def _dev(*ts: torch.Tensor) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError("openattention_amd kernels need tensors on a HIP device "
                               f"(got {t.device}); there is no CPU fallback")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _chk(t: torch.Tensor, name: str, dtype: torch.dtype, shape: tuple | None = None,
         contiguous: bool = False) -> None:
    """dtype, exact shape (None entries: any extent; a negative entry -m: at least m) and, when
    asked, contiguity -- the layout the kernels index without further checks."""
    _need(t.dtype == dtype, f"{name}: dtype must be {dtype} (got {t.dtype})")
    if shape is not None:
        ok = t.dim() == len(shape) and all(
            want is None or (got == want if want >= 0 else got >= -want)
            for got, want in zip(t.shape, shape))
        _need(ok, f"{name}: shape {tuple(t.shape)} does not match {shape} (-m: at least m)")
    if contiguous:
        _need(t.is_contiguous(), f"{name}: must be contiguous")
    else:
        _need(t.dim() == 0 or t.stride(-1) == 1, f"{name}: last dimension must be contiguous")


def _stats(R: int, C: int, *named) -> None:
    """pooled statistics (R, C, 128) fp32, contiguous (the kernels step rows by C * 128)"""
    for t, name in named:
        _chk(t, name, torch.float32, (R, C, HEAD_DIM), contiguous=True)


def _rows_contig(t: torch.Tensor, name: str, align_elems: int = 1) -> None:
    _need(t.stride(-1) == 1, f"{name}: last dimension must be contiguous")
    for s in t.stride()[:-1]:
        _need(s % align_elems == 0, f"{name}: strides must be multiples of {align_elems} elements")
    _need(t.data_ptr() % (2 * align_elems if t.dtype == torch.bfloat16 else 4 * align_elems) == 0,
          f"{name}: base pointer misaligned")


def _contig(t: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    _need(t.dtype == dtype, f"{name}: expected {dtype}, got {t.dtype}")
    _need(t.is_contiguous(), f"{name}: must be contiguous")


# ================================================================== OpenAttention.flash
def flash_decode(q, k, v, sel_idx, exp_idx, kbar, vbar, log_n, *, proxy_per_kv: bool,
                 sm_scale: float, n_bins: int | None = None, n_split: int | None = None,
                 out: torch.Tensor | None = None, noalloc: bool = False) -> torch.Tensor:
    """Shared body of ours_flash / decode_expand_attention.  noalloc=True calls
    oa_flash_decode_noalloc (split partials in the library's fixed device array; nothing is
    allocated, so `out` must be given)."""
    dev = _dev(q, k, v, sel_idx, exp_idx, kbar, vbar, log_n)
    R, D = q.shape
    _need(D == HEAD_DIM, f"head_dim must be {HEAD_DIM}")
    _need(q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16,
          "q, k, v must be bfloat16")
    _need(k.dim() == 3 and k.shape == v.shape and k.stride() == v.stride() and k.shape[2] == D,
          "k, v must be (B*HKV, Lmax, D) with identical strides")
    BH = k.shape[0]
    _need(R % BH == 0, "rows of q must be a multiple of the KV rows of k")
    _rows_contig(q, "q", 8)
    _rows_contig(k, "k", 8)
    _rows_contig(v, "v", 8)
    _need(sel_idx.dtype == torch.int32 and exp_idx.dtype == torch.int32, "indices must be int32")
    _need(sel_idx.shape[0] == R and exp_idx.shape[0] == R, "index rows must match q")
    _need(sel_idx.stride(-1) == 1 and exp_idx.stride(-1) == 1, "index rows must be contiguous")
    NB = kbar.shape[1] if n_bins is None else int(n_bins)
    _need(0 <= NB <= kbar.shape[1], "nb out of range")
    _need(kbar.shape == vbar.shape and kbar.stride() == vbar.stride() and kbar.dtype == vbar.dtype,
          "kbar and vbar must match")
    _need(kbar.dtype in (torch.bfloat16, torch.float32), "kbar/vbar must be bf16 or fp32")
    _need(kbar.shape[0] == (BH if proxy_per_kv else R) and kbar.shape[2] == D, "kbar shape")
    _rows_contig(kbar, "kbar", 8 if kbar.dtype == torch.bfloat16 else 4)
    _need(log_n.dtype == torch.float32 and log_n.shape[0] == R and log_n.stride(-1) == 1,
          "log_n must be fp32 (R, C)")
    _need(not noalloc or out is not None, "noalloc needs a caller-provided out")
    if out is None:
        out = torch.empty_like(q)
    _need(out.shape == q.shape and out.dtype in (torch.bfloat16, torch.float32) and out.stride(1) == 1,
          "out must be (R, 128) bf16 or fp32 with contiguous rows")
    out_f32 = 1 if out.dtype == torch.float32 else 0
    T = sel_idx.shape[1] + exp_idx.shape[1] + NB
    if n_split is None:
        # few rows cannot fill the GPU: split each row's list (reference: ours_graph.py:276)
        n_split = 1 if R >= 512 else max(2, min(16, (4096 // max(R, 1)), -(-T // 32)))
    n_split = max(1, int(n_split))
    if noalloc:
        lib.call("oa_flash_decode_noalloc",
                 _ptr(q), q.stride(0), _ptr(k), _ptr(v), k.stride(0), k.stride(1),
                 _ptr(sel_idx), sel_idx.stride(0), sel_idx.shape[1],
                 _ptr(exp_idx), exp_idx.stride(0), exp_idx.shape[1],
                 _ptr(kbar), _ptr(vbar), kbar.stride(0), kbar.stride(1),
                 1 if kbar.dtype == torch.float32 else 0, 1 if proxy_per_kv else 0,
                 _ptr(log_n), log_n.stride(0), NB, _ptr(out), out.stride(0), out_f32,
                 R, BH, D, float(sm_scale), n_split, _stream(dev))
        return out
    ws = None
    if n_split > 1:
        ws = torch.empty(R * n_split * (HEAD_DIM + 2), device=dev, dtype=torch.float32)
        ws_m = ws[: R * n_split]
        ws_l = ws[R * n_split: 2 * R * n_split]
        ws_acc = ws[2 * R * n_split:]
    lib.call("oa_flash_decode",
             _ptr(q), q.stride(0), _ptr(k), _ptr(v), k.stride(0), k.stride(1),
             _ptr(sel_idx), sel_idx.stride(0), sel_idx.shape[1],
             _ptr(exp_idx), exp_idx.stride(0), exp_idx.shape[1],
             _ptr(kbar), _ptr(vbar), kbar.stride(0), kbar.stride(1),
             1 if kbar.dtype == torch.float32 else 0, 1 if proxy_per_kv else 0,
             _ptr(log_n), log_n.stride(0), NB, _ptr(out), out.stride(0), out_f32,
             R, BH, D, float(sm_scale), n_split,
             _ptr(ws_m) if ws is not None else None, _ptr(ws_l) if ws is not None else None,
             _ptr(ws_acc) if ws is not None else None, _stream(dev))
    return out


def ours_flash(q, k, v, sel_idx, exp_idx, kbar, vbar, log_n, nb=None):
    """q:(R,D) k,v:(B*HKV,Lmax,D) sel:(R,Ns) exp:(R,Ne) int32 (-1 = pad); kbar,vbar:(R,C,D);
    log_n:(R,C) natural log, -inf = no proxy.  nb overrides the proxy count (0 = P3 off).
    Same contract as inference/methods_eager.py:161-172; sm_scale = D**-0.5."""
    return flash_decode(q, k, v, sel_idx, exp_idx, kbar, vbar, log_n, proxy_per_kv=False,
                        sm_scale=HEAD_DIM ** -0.5, n_bins=nb)


def decode_expand_attention(q, k, v, sel_idx, exp_idx, kbar, vbar, log_n, sm_scale=None,
                            block_n=64, block_b=64, num_warps=4):
    """q:(BQ,D) k,v:(BH,K,D) sel_idx:(BQ,N_SEL) exp_idx:(BQ,N_EXP) kbar,vbar:(BH,NB,D)
    log_n:(BQ,NB) -> (BQ,D).  Same contract as triton_expand_decode.py:139-165; the Triton
    tuning arguments (block_n, block_b, num_warps) are accepted and ignored."""
    D = q.shape[1]
    scale = D ** -0.5 if sm_scale is None else float(sm_scale)
    return flash_decode(q, k, v, sel_idx, exp_idx, kbar, vbar, log_n, proxy_per_kv=True,
                        sm_scale=scale)


# ================================================================== decode-stage kernels
def index_update(K, V, st, n_dev: torch.Tensor, rmax: int) -> None:
    """The token at n-1 joins the index (ours_graph.py:43-90).  st: LayerState-like object
    with codes, U, scale, W, colmean, cent, asg, nb, Sk, Sk2, Sv, reclist, reccnt (one layer,
    all batch rows, flattened to rows)."""
    dev = _dev(K, V, n_dev)
    BH, Lmax, D = K.shape
    R = st.nb.shape[0]
    C = st.nb.shape[1]
    lib.call("oa_index_update", _ptr(K), _ptr(V), K.stride(0), K.stride(1), R, BH, D,
             _ptr(st.codes), st.codes.shape[1], RANK_Q, _ptr(st.U), _ptr(st.scale), _ptr(st.W),
             _ptr(st.colmean), RANK_C, _ptr(st.cent), C, _ptr(st.asg), st.asg.stride(0),
             _ptr(st.asg8), st.asg8.stride(0), _ptr(st.nb), _ptr(st.Sk), _ptr(st.Sk2), _ptr(st.Sv), _ptr(st.reclist),
             _ptr(st.reccnt), rmax, _ptr(n_dev), _stream(dev))


def index_downdate(K, V, st, n_dev: torch.Tensor) -> None:
    """The token at n-1 leaves the cluster statistics (nb, Sk, Sk2, Sv) of every query row: the
    statistics step of index_update undone, so that a causal row ending before it sees the
    statistics of the keys it attends (multibin.py:2210-2218)."""
    dev = _dev(K, V, n_dev)
    BH, Lmax, D = K.shape
    R = st.nb.shape[0]
    C = st.nb.shape[1]
    _chk(K, "K", torch.bfloat16, (BH, Lmax, HEAD_DIM))
    _need(V.shape == K.shape and V.stride() == K.stride() and V.dtype == K.dtype, "V must match K")
    _chk(st.asg, "asg", torch.int32, (R, -Lmax))
    _chk(st.nb, "nb", torch.float32, (R, C), contiguous=True)
    _stats(R, C, (st.Sk, "Sk"), (st.Sk2, "Sk2"), (st.Sv, "Sv"))
    _chk(n_dev, "n_dev", torch.int32)
    lib.call("oa_index_downdate", _ptr(K), _ptr(V), K.stride(0), K.stride(1), R, BH, D, _ptr(st.asg),
             st.asg.stride(0), _ptr(st.nb), _ptr(st.Sk), _ptr(st.Sk2), _ptr(st.Sv), C, _ptr(n_dev),
             _stream(dev))


def index_prep(K, V, st, n_dev: torch.Tensor, rmax: int, q, limbs, fexp) -> None:
    """index_update and qgs_prep in one launch (same results as the two calls)."""
    dev = _dev(K, V, n_dev, q, limbs, fexp)
    BH, Lmax, D = K.shape
    R = st.nb.shape[0]
    C = st.nb.shape[1]
    _chk(K, "K", torch.bfloat16, (BH, Lmax, HEAD_DIM))
    _need(V.shape == K.shape and V.stride() == K.stride() and V.dtype == K.dtype, "V must match K")
    _chk(st.codes, "codes", torch.int8, (BH, -Lmax, RANK_Q), contiguous=True)
    _chk(st.asg, "asg", torch.int32, (R, -Lmax))
    _chk(st.asg8, "asg8", torch.uint8, (R, -Lmax))
    _chk(st.nb, "nb", torch.float32, (R, C), contiguous=True)
    _stats(R, C, (st.Sk, "Sk"), (st.Sk2, "Sk2"), (st.Sv, "Sv"))
    _chk(q, "q", torch.bfloat16, (R, HEAD_DIM))
    _chk(n_dev, "n_dev", torch.int32)
    _chk(limbs, "limbs", torch.int8, (BH, 16, RANK_Q), contiguous=True)
    _chk(fexp, "fexp", torch.int32, (R,), contiguous=True)
    _rows_contig(q, "q")
    lib.call("oa_index_prep", _ptr(K), _ptr(V), K.stride(0), K.stride(1), R, BH, D,
             _ptr(st.codes), st.codes.shape[1], RANK_Q, _ptr(st.U), _ptr(st.scale), _ptr(st.W),
             _ptr(st.colmean), RANK_C, _ptr(st.cent), C, _ptr(st.asg), st.asg.stride(0),
             _ptr(st.asg8), st.asg8.stride(0), _ptr(st.nb), _ptr(st.Sk), _ptr(st.Sk2), _ptr(st.Sv),
             _ptr(st.reclist), _ptr(st.reccnt), rmax, _ptr(n_dev), _ptr(q), q.stride(0),
             _ptr(limbs), _ptr(fexp), _stream(dev))


def qgs_prep(q, U, scale, limbs, fexp, zq_out=None) -> None:
    dev = _dev(q, U, scale, limbs, fexp)
    R = q.shape[0]
    BH = U.shape[0]
    _rows_contig(q, "q")
    lib.call("oa_qgs_prep", _ptr(q), q.stride(0), _ptr(U), _ptr(scale), R, BH, q.shape[1], RANK_Q,
             _ptr(limbs), _ptr(fexp), _ptr(zq_out), _stream(dev))


def qgs_scan(codes, limbs, fexp, S, TM, n_dev, ns: int, nl: int) -> None:
    dev = _dev(codes, limbs, fexp, S, TM, n_dev)
    BH, Lmax, rq = codes.shape
    lib.call("oa_qgs_scan", _ptr(codes), BH, Lmax, rq, _ptr(limbs), _ptr(fexp), _ptr(S), S.stride(0),
             _ptr(TM), TM.stride(0), _ptr(n_dev), ns, nl, _stream(dev))


def topk_select(S, TM, sel, n_dev, ns: int, nl: int, k_top: int) -> None:
    dev = _dev(S, TM, sel, n_dev)
    R = S.shape[0]
    lib.call("oa_topk_select", _ptr(S), S.stride(0), _ptr(TM), TM.stride(0), R, TM.shape[1],
             _ptr(sel), sel.stride(0), _ptr(n_dev), ns, nl, k_top, _stream(dev))


def qgs_scan_heads(codes, limbs, fexp, H, TM, n_dev, ns: int, nl: int, TMn=None) -> None:
    """The scan writing 16-bit key heads of the scores (int16 tensor H, raw bits) instead of
    fp32 scores; TM (exact tile maxima) as oa_qgs_scan; TMn (optional, like TM): each tile's
    least finite score (+inf without one), the range topq_heads bins with."""
    dev = _dev(codes, limbs, fexp, H, TM, n_dev)
    if H.dtype != torch.int16:
        raise ValueError("H must be int16 (16-bit key heads)")
    BH, Lmax, rq = codes.shape
    _chk(codes, "codes", torch.int8, (BH, Lmax, RANK_Q), contiguous=True)
    _chk(H, "H", torch.int16, (GROUP * BH, -Lmax))
    _chk(TM, "TM", torch.float32, (GROUP * BH, None))
    _tile_min(TM, TMn)
    _chk(limbs, "limbs", torch.int8, (BH, 16, RANK_Q), contiguous=True)
    _chk(fexp, "fexp", torch.int32, (GROUP * BH,), contiguous=True)
    _chk(n_dev, "n_dev", torch.int32)
    lib.call("oa_qgs_scan_heads", _ptr(codes), BH, Lmax, rq, _ptr(limbs), _ptr(fexp), _ptr(H),
             H.stride(0), _ptr(TM), TM.stride(0), _ptr(TMn), _ptr(n_dev), ns, nl, _stream(dev))


def _tile_min(TM, TMn) -> None:
    """TMn, when given, is laid out as TM (same shape and row stride)."""
    if TMn is not None and (TMn.dtype != torch.float32 or TMn.shape != TM.shape
                            or TMn.stride() != TM.stride() or TMn.device != TM.device):
        raise ValueError("TMn must be a float32 tensor with TM's shape, strides and device")


def topk_select_heads(H, TM, sel, n_dev, ns: int, nl: int, k_top: int, codes, limbs, fexp) -> None:
    """Top-k over key-head rows: candidate scores recomputed exactly from the codes; the
    selected tokens' heads are set to that of -inf."""
    dev = _dev(H, TM, sel, n_dev, codes, limbs, fexp)
    R = H.shape[0]
    BH, Lmax, _ = codes.shape
    lib.call("oa_topk_select_heads", _ptr(H), H.stride(0), _ptr(TM), TM.stride(0), R, TM.shape[1],
             _ptr(sel), sel.stride(0), _ptr(n_dev), ns, nl, k_top, _ptr(codes), BH, Lmax,
             _ptr(limbs), _ptr(fexp), _stream(dev))


def errorgate(q, K, asg, sel, Sk, Sk2, nb, score, n_t, sm_scale: float) -> None:
    """wl1 cluster scores; sm_scale is the Python (double) scale, whose square is formed in
    double and rounded once, as the estimator does (multibin.py:643)."""
    dev = _dev(q, K, asg, sel, Sk, Sk2, nb, score, n_t)
    R, C = nb.shape
    BH = K.shape[0]
    lib.call("oa_errorgate", _ptr(q), q.stride(0), _ptr(K), K.stride(0), K.stride(1), R, BH,
             q.shape[1], _ptr(asg), asg.stride(0), _ptr(sel), sel.stride(0), sel.shape[1],
             _ptr(Sk), _ptr(Sk2), _ptr(nb), C, float(sm_scale), float(sm_scale) * float(sm_scale),
             _ptr(score), _ptr(n_t), _stream(dev))


def gate_fill(q, K, asg, sel, Sk, Sk2, nb, score, n_t, quota, sm_scale: float, E: int,
              qsk=None) -> None:
    """ErrorGate + water-filling (same results as errorgate then waterfill); qsk (R, C) fp32,
    when given, receives q . Sk of every cluster for residual_flash."""
    dev = _dev(q, K, asg, sel, Sk, Sk2, nb, score, n_t, quota)
    R, C = nb.shape
    BH = K.shape[0]
    _chk(q, "q", torch.bfloat16, (R, HEAD_DIM))
    _chk(K, "K", torch.bfloat16, (BH, None, HEAD_DIM))
    _chk(asg, "asg", torch.int32, (R, None))
    _chk(sel, "sel", torch.int32, (R, None))
    _stats(R, C, (Sk, "Sk"), (Sk2, "Sk2"))
    for t, name in ((nb, "nb"), (score, "score"), (n_t, "n_t"), (quota, "quota")):
        _chk(t, name, torch.float32, (R, C), contiguous=True)
    if qsk is not None and (qsk.shape != (R, C) or qsk.dtype != torch.float32 or not qsk.is_contiguous()):
        raise ValueError("qsk must be a contiguous (rows, C) float32 tensor")
    lib.call("oa_gate_fill", _ptr(q), q.stride(0), _ptr(K), K.stride(0), K.stride(1), R, BH,
             q.shape[1], _ptr(asg), asg.stride(0), _ptr(sel), sel.stride(0), sel.shape[1],
             _ptr(Sk), _ptr(Sk2), _ptr(nb), C, float(sm_scale), float(sm_scale) * float(sm_scale),
             int(E), _ptr(score), _ptr(n_t), _ptr(quota), _ptr(qsk), _stream(dev))


def topk_gate_fill(H, TM, n_dev, ns: int, nl: int, k_top: int, codes, limbs, fexp, q, K, asg, sel,
                   Sk, Sk2, nb, score, n_t, quota, sm_scale: float, E: int, qsk=None) -> None:
    """topk_select_heads then gate_fill (the same sel, marked heads, score, n_t, quota, qsk); one
    launch when the row fits the register top-k (its pooled ErrorGate computed while the top-k
    runs, then the selected tokens' correction and the fill).  sel has ns + nl + k_top columns."""
    dev = _dev(H, TM, n_dev, codes, limbs, fexp, q, K, asg, sel, Sk, Sk2, nb, score, n_t, quota)
    R, C = nb.shape
    BH, Lmax, _ = codes.shape
    _chk(H, "H", torch.int16, (R, -Lmax))
    _chk(TM, "TM", torch.float32, (R, None))
    _chk(codes, "codes", torch.int8, (BH, Lmax, RANK_Q), contiguous=True)
    _chk(limbs, "limbs", torch.int8, (BH, 16, RANK_Q), contiguous=True)
    _chk(fexp, "fexp", torch.int32, (R,), contiguous=True)
    _chk(q, "q", torch.bfloat16, (R, HEAD_DIM))
    _chk(K, "K", torch.bfloat16, (K.shape[0], None, HEAD_DIM))
    _chk(asg, "asg", torch.int32, (R, None))
    _chk(sel, "sel", torch.int32, (R, ns + nl + k_top))
    _stats(R, C, (Sk, "Sk"), (Sk2, "Sk2"))
    for t, name in ((nb, "nb"), (score, "score"), (n_t, "n_t"), (quota, "quota")):
        _chk(t, name, torch.float32, (R, C), contiguous=True)
    if qsk is not None and (qsk.shape != (R, C) or qsk.dtype != torch.float32 or not qsk.is_contiguous()):
        raise ValueError("qsk must be a contiguous (rows, C) float32 tensor")
    lib.call("oa_topk_gate_fill", _ptr(H), H.stride(0), _ptr(TM), TM.stride(0), TM.shape[1],
             _ptr(n_dev), ns, nl, k_top, _ptr(codes), Lmax, _ptr(limbs), _ptr(fexp), _ptr(q),
             q.stride(0), _ptr(K), K.stride(0), K.stride(1), R, K.shape[0], q.shape[1], _ptr(asg),
             asg.stride(0), _ptr(sel), sel.stride(0), _ptr(Sk), _ptr(Sk2), _ptr(nb), C,
             float(sm_scale), float(sm_scale) * float(sm_scale), int(E), _ptr(score), _ptr(n_t),
             _ptr(quota), _ptr(qsk), _stream(dev))


def qgs_scan_gate(codes, limbs, fexp, H, TM, n_dev, ns: int, nl: int, q, Sk, Sk2, nb, score, n_t,
                  sm_scale: float, qsk=None, TMn=None) -> None:
    """qgs_scan_heads and the pooled part of the ErrorGate in one launch: score, n_t (rows, C)
    of every cluster as if it held no selected token, and q . Sk_c into qsk."""
    dev = _dev(codes, limbs, fexp, H, TM, n_dev, q, Sk, Sk2, nb, score, n_t)
    BH, Lmax, rq = codes.shape
    R, C = nb.shape
    _chk(codes, "codes", torch.int8, (BH, Lmax, RANK_Q), contiguous=True)
    _chk(H, "H", torch.int16, (GROUP * BH, -Lmax))
    _chk(TM, "TM", torch.float32, (GROUP * BH, None))
    _tile_min(TM, TMn)
    _chk(limbs, "limbs", torch.int8, (BH, 16, RANK_Q), contiguous=True)
    _chk(fexp, "fexp", torch.int32, (GROUP * BH,), contiguous=True)
    _chk(n_dev, "n_dev", torch.int32)
    _chk(q, "q", torch.bfloat16, (R, HEAD_DIM))
    _need(R == GROUP * BH, "nb must have one row per query-head row")
    _stats(R, C, (Sk, "Sk"), (Sk2, "Sk2"))
    for t, name in ((nb, "nb"), (score, "score"), (n_t, "n_t")):
        _chk(t, name, torch.float32, (R, C), contiguous=True)
    if qsk is not None and (qsk.shape != (R, C) or qsk.dtype != torch.float32 or not qsk.is_contiguous()):
        raise ValueError("qsk must be a contiguous (rows, C) float32 tensor")
    lib.call("oa_qgs_scan_gate", _ptr(codes), BH, Lmax, rq, _ptr(limbs), _ptr(fexp), _ptr(H), H.stride(0),
             _ptr(TM), TM.stride(0), _ptr(TMn), _ptr(n_dev), ns, nl, _ptr(q), q.stride(0), _ptr(Sk), _ptr(Sk2), _ptr(nb),
             C, float(sm_scale), float(sm_scale) * float(sm_scale), _ptr(score), _ptr(n_t), _ptr(qsk),
             _stream(dev))


def topk_fix_fill(H, TM, n_dev, ns: int, nl: int, k_top: int, codes, limbs, fexp, q, K, asg, sel, Sk,
                  Sk2, nb, score, n_t, quota, sm_scale: float, E: int) -> None:
    """After qgs_scan_gate: the top-k over the heads, the ErrorGate of the clusters holding a
    selected token done again (score, n_t updated in place), the water-fill.  The same sel,
    marked heads, score, n_t and quota as topk_select_heads followed by gate_fill."""
    dev = _dev(H, TM, n_dev, codes, limbs, fexp, q, K, asg, sel, Sk, Sk2, nb, score, n_t, quota)
    R, C = nb.shape
    BH, Lmax, _ = codes.shape
    _chk(H, "H", torch.int16, (R, -Lmax))
    _chk(TM, "TM", torch.float32, (R, None))
    _chk(codes, "codes", torch.int8, (BH, Lmax, RANK_Q), contiguous=True)
    _chk(limbs, "limbs", torch.int8, (BH, 16, RANK_Q), contiguous=True)
    _chk(fexp, "fexp", torch.int32, (R,), contiguous=True)
    _chk(q, "q", torch.bfloat16, (R, HEAD_DIM))
    _chk(K, "K", torch.bfloat16, (K.shape[0], None, HEAD_DIM))
    _chk(asg, "asg", torch.int32, (R, None))
    _chk(sel, "sel", torch.int32, (R, ns + nl + k_top))
    _stats(R, C, (Sk, "Sk"), (Sk2, "Sk2"))
    for t, name in ((nb, "nb"), (score, "score"), (n_t, "n_t"), (quota, "quota")):
        _chk(t, name, torch.float32, (R, C), contiguous=True)
    lib.call("oa_topk_fix_fill", _ptr(H), H.stride(0), _ptr(TM), TM.stride(0), TM.shape[1],
             _ptr(n_dev), ns, nl, k_top, _ptr(codes), Lmax, _ptr(limbs), _ptr(fexp), _ptr(q),
             q.stride(0), _ptr(K), K.stride(0), K.stride(1), R, K.shape[0], q.shape[1], _ptr(asg),
             asg.stride(0), _ptr(sel), sel.stride(0), _ptr(Sk), _ptr(Sk2), _ptr(nb), C,
             float(sm_scale), float(sm_scale) * float(sm_scale), int(E), _ptr(score), _ptr(n_t),
             _ptr(quota), _stream(dev))


def waterfill(score, n_t, quota, E: int) -> None:
    dev = _dev(score, n_t, quota)
    R, C = score.shape
    lib.call("oa_waterfill", _ptr(score), _ptr(n_t), R, C, int(E), _ptr(quota), _stream(dev))


def topq(S, asg8, quota, exp_idx, n_dev, path: int | None = None) -> None:
    """Within-cluster top-q (exp_idx segments grouped by cluster, position order inside).
    path None: oa_topq; 0 / 1 / 2: oa_topq_path (both kernels / key-prefix only / linear-bin only,
    a row left to the key-prefix kernel then holding -2 in exp_idx[row, 0])."""
    dev = _dev(S, asg8, quota, exp_idx, n_dev)
    R, C = quota.shape
    Lmax = asg8.shape[1]
    E = exp_idx.shape[1]
    if path is None:
        lib.call("oa_topq", _ptr(S), S.stride(0), _ptr(asg8), asg8.stride(0), _ptr(quota), R, C,
                 Lmax, _ptr(exp_idx), E, _ptr(n_dev), _stream(dev))
    else:
        lib.call("oa_topq_path", _ptr(S), S.stride(0), _ptr(asg8), asg8.stride(0), _ptr(quota), R,
                 C, Lmax, _ptr(exp_idx), E, _ptr(n_dev), int(path), _stream(dev))


def topq_heads(H, asg8, quota, exp_idx, n_dev, codes, limbs, fexp, S32, path: int = 0, TM=None,
               TMn=None) -> None:
    """Within-cluster top-q over key-head rows (oa_topq_heads); S32 (fp32, rows as H) receives
    the exact scores of rows left to the key-prefix kernel.  path 2: the linear-bin kernel
    alone; path 3: every row through the key-prefix kernel.  TM, TMn (both or neither): the
    scan's tile maxima and minima, the row range taken from them (same result)."""
    dev = _dev(H, asg8, quota, exp_idx, n_dev, codes, limbs, fexp, S32)
    R, C = quota.shape
    Lmax = codes.shape[1]
    E = exp_idx.shape[1]
    _chk(H, "H", torch.int16, (R, -Lmax))
    _chk(asg8, "asg8", torch.uint8, (R, -Lmax))
    _chk(quota, "quota", torch.float32, (R, C), contiguous=True)
    _chk(exp_idx, "exp_idx", torch.int32, (R, E), contiguous=True)
    _chk(codes, "codes", torch.int8, (R // GROUP, Lmax, RANK_Q), contiguous=True)
    _chk(limbs, "limbs", torch.int8, (R // GROUP, 16, RANK_Q), contiguous=True)
    _chk(fexp, "fexp", torch.int32, (R,), contiguous=True)
    _chk(S32, "S32", torch.float32, (R, -Lmax))
    if (TM is None) != (TMn is None):
        raise ValueError("TM and TMn are given together")
    if TM is not None:
        _chk(TM, "TM", torch.float32, (R, -((Lmax + 63) // 64)))
        _tile_min(TM, TMn)
    lib.call("oa_topq_heads", _ptr(H), H.stride(0), _ptr(asg8), asg8.stride(0), _ptr(quota), R, C,
             Lmax, _ptr(exp_idx), E, _ptr(n_dev), _ptr(codes), codes.shape[0], _ptr(limbs),
             _ptr(fexp), _ptr(S32), S32.stride(0), _ptr(TM), _ptr(TMn),
             TM.stride(0) if TM is not None else 0, int(path), _stream(dev))


def residual(K, V, asg, sel, exp_idx, quota, n_t, Sk, Sv, kbar_r, vbar_r, log_n) -> None:
    dev = _dev(K, V, asg, sel, exp_idx, quota, n_t, Sk, Sv, kbar_r, vbar_r, log_n)
    R, C = quota.shape
    BH = K.shape[0]
    lib.call("oa_residual", _ptr(K), _ptr(V), K.stride(0), K.stride(1), R, BH, K.shape[2],
             _ptr(asg), asg.stride(0), _ptr(sel), sel.stride(0), sel.shape[1], _ptr(exp_idx),
             exp_idx.shape[1], _ptr(quota), _ptr(n_t), _ptr(Sk), _ptr(Sv), C, _ptr(kbar_r),
             _ptr(vbar_r), _ptr(log_n), _stream(dev))


def residual_flash(q, K, V, asg, sel, exp_idx, quota, n_t, Sk, Sv, out, sm_scale: float,
                   qsk=None) -> None:
    """Residual proxies + fused softmax; qsk (R, C) fp32 from gate_fill, when given, replaces the
    kernel's own pass over Sk (same quantity, summed in another order)."""
    dev = _dev(q, K, V, asg, sel, exp_idx, quota, n_t, Sk, Sv, out)
    R, C = quota.shape
    BH = K.shape[0]
    _chk(q, "q", torch.bfloat16, (R, HEAD_DIM))
    _chk(K, "K", torch.bfloat16, (BH, None, HEAD_DIM))
    _need(V.shape == K.shape and V.stride() == K.stride() and V.dtype == K.dtype, "V must match K")
    _chk(asg, "asg", torch.int32, (R, None))
    _chk(sel, "sel", torch.int32, (R, None))
    _chk(exp_idx, "exp_idx", torch.int32, (R, None), contiguous=True)
    for t, name in ((quota, "quota"), (n_t, "n_t")):
        _chk(t, name, torch.float32, (R, C), contiguous=True)
    _stats(R, C, (Sk, "Sk"), (Sv, "Sv"))
    if qsk is not None and (qsk.shape != (R, C) or qsk.dtype != torch.float32 or not qsk.is_contiguous()):
        raise ValueError("qsk must be a contiguous (rows, C) float32 tensor")
    _need(out.shape == (R, HEAD_DIM) and out.dtype in (torch.bfloat16, torch.float32) and out.stride(1) == 1,
          "out must be (R, 128) bf16 or fp32 with contiguous rows")
    lib.call("oa_residual_flash", _ptr(q), q.stride(0), _ptr(K), _ptr(V), K.stride(0), K.stride(1),
             R, BH, K.shape[2], _ptr(asg), asg.stride(0), _ptr(sel), sel.stride(0), sel.shape[1],
             _ptr(exp_idx), exp_idx.shape[1], _ptr(quota), _ptr(n_t), _ptr(Sk), _ptr(Sv), C,
             float(sm_scale), _ptr(out), out.stride(0), 1 if out.dtype == torch.float32 else 0,
             _ptr(qsk), _stream(dev))


# key chunks per KV row of the dense comparator: measured best both at B = 32 (8192 workgroups:
# 725 us against 980 with 256 chunks) and at B = 1 (54 us against 117: the combine walks every
# chunk)
DENSE_SPLITS = 32


def dense_decode(q, K, V, n_dev, out=None, sm_scale: float | None = None, nsplit: int | None = None,
                 ws: torch.Tensor | None = None) -> torch.Tensor:
    """Dense decode attention over [0, n) (graph_runner.py:259-312 comparator)."""
    dev = _dev(q, K, V, n_dev)
    R, D = q.shape
    BH, Lmax, _ = K.shape
    _rows_contig(q, "q", 8)
    _rows_contig(K, "K", 8)
    if nsplit is None:
        nsplit = DENSE_SPLITS
    if out is None:
        out = torch.empty_like(q)
    need = R * nsplit * (HEAD_DIM + 2)
    if ws is None or ws.numel() < need:
        ws = torch.empty(need, device=dev, dtype=torch.float32)
    scale = D ** -0.5 if sm_scale is None else sm_scale
    lib.call("oa_dense_decode", _ptr(q), q.stride(0), _ptr(K), _ptr(V), K.stride(0), K.stride(1), R,
             BH, D, Lmax, _ptr(n_dev), float(scale), nsplit, _ptr(ws[: R * nsplit]),
             _ptr(ws[R * nsplit: 2 * R * nsplit]), _ptr(ws[2 * R * nsplit: need]), _ptr(out),
             out.stride(0), _stream(dev))
    return out


# ================================================================== prefill index build
def qgs_codes(K, T: int, U, codes, scale, amax_ws, zc_ws=None) -> None:
    """a11 of one request: K (HKV, >=T, 128) bf16; U (HKV, 128, 32) fp32; codes (HKV, Lmax, 32)
    int8 (rows written up to T); scale (HKV, 32); amax_ws >= HKV*32 int32 scratch; zc_ws >= HKV*T*32
    fp32 scratch or None (then k U is formed twice; the same codes)."""
    dev = _dev(K, U, codes, scale, amax_ws)
    HKV = K.shape[0]
    _need(K.dtype == torch.bfloat16 and K.stride(-1) == 1, "K: bf16 with contiguous rows")
    _need(U.is_contiguous() and U.shape == (HKV, HEAD_DIM, RANK_Q), "U: (HKV, 128, 32) contiguous")
    _need(scale.is_contiguous() and scale.shape == (HKV, RANK_Q), "scale: (HKV, 32) contiguous")
    _need(codes.dtype == torch.int8 and codes.stride(2) == 1 and codes.stride(1) == RANK_Q,
          "codes: (HKV, Lmax, 32) int8 rows")
    _need(amax_ws.numel() >= HKV * RANK_Q, "amax_ws too small")
    _need(T <= K.shape[1] and T <= codes.shape[1], "T beyond the rows")
    if zc_ws is not None:
        _need(zc_ws.dtype == torch.float32 and zc_ws.is_contiguous() and zc_ws.numel() >= HKV * T * RANK_Q,
              "zc_ws: >= HKV*T*32 fp32, contiguous")
    lib.call("oa_qgs_codes", _ptr(K), K.stride(0), K.stride(1), HKV, T, _ptr(U), _ptr(codes),
             codes.stride(0), _ptr(scale), _ptr(amax_ws), _ptr(zc_ws), _stream(dev))


def query_metric(q, pick, cosv, sinv, scaling: float, mst_half, G: int, gm_out=None, m_out=None):
    """a10 metric of every query row of q (rows, Qn, 128) bf16 or fp32 (rows = KV rows * G):
    returns (gm_out (rows / G, 128, 128) group means, m_out (rows, 128, 128) metrics), fp32.
    pick (P,) int32 question positions; cosv, sinv (P, 128) fp64 RoPE cos / sin of each picked
    row's advance; mst_half (heads, 128, 128) fp32, used for row r as mst_half[r % heads]."""
    dev = _dev(q, pick, cosv, sinv, mst_half, gm_out, m_out)
    _need(q.dim() == 3 and q.shape[-1] == HEAD_DIM and q.stride(-1) == 1
          and q.dtype in (torch.bfloat16, torch.float32), "q: (rows, Qn, 128) bf16 or fp32, rows of dims contiguous")
    rows = q.shape[0]
    _need(rows % G == 0, "rows: a multiple of G")
    _need(pick.dtype == torch.int32 and pick.dim() == 1 and pick.is_contiguous(), "pick: (P,) int32")
    P = pick.numel()
    _need(1 <= P <= 64, "P: 1..64 picked rows")
    for t, nm in ((cosv, "cosv"), (sinv, "sinv")):
        _need(t.dtype == torch.float64 and t.shape == (P, HEAD_DIM) and t.is_contiguous(), f"{nm}: (P, 128) fp64")
    _need(mst_half.dtype == torch.float32 and mst_half.dim() == 3 and mst_half.shape[1:] == (HEAD_DIM, HEAD_DIM)
          and mst_half.is_contiguous(), "mst_half: (heads, 128, 128) fp32 contiguous")
    if gm_out is None:
        gm_out = torch.empty(rows // G, HEAD_DIM, HEAD_DIM, device=dev, dtype=torch.float32)
    if m_out is None:
        m_out = torch.empty(rows, HEAD_DIM, HEAD_DIM, device=dev, dtype=torch.float32)
    for t, n_, nm in ((gm_out, rows // G, "gm_out"), (m_out, rows, "m_out")):
        _need(t.dtype == torch.float32 and t.is_contiguous() and t.shape == (n_, HEAD_DIM, HEAD_DIM),
              f"{nm}: ({n_}, 128, 128) fp32 contiguous")
    lib.call("oa_query_metric", _ptr(q), int(q.dtype == torch.bfloat16), q.stride(0), q.stride(1), rows, G,
             _ptr(pick), P, _ptr(cosv), _ptr(sinv), float(scaling), _ptr(mst_half), mst_half.shape[0],
             _ptr(gm_out), _ptr(m_out), _stream(dev))
    return gm_out, m_out


def sym_eig_top(M, k: int, sweeps=None):
    """Top-k eigenpairs of symmetric positive semi-definite (batch, 128, 128) fp32 matrices (the
    lower triangle is read): (evals (batch, k), evecs (batch, 128, k)), ascending, the last k of
    torch.linalg.eigh's order; signs are free.  sweeps: (batch,) int32 or None, the Jacobi sweeps
    each matrix took (negative: unconverged at the cap)."""
    dev = _dev(M, sweeps)
    _need(M.dtype == torch.float32 and M.dim() == 3 and M.shape[1:] == (HEAD_DIM, HEAD_DIM)
          and M.stride(2) == 1 and M.stride(1) == HEAD_DIM
          and (M.shape[0] <= 1 or M.stride(0) >= HEAD_DIM * HEAD_DIM),
          "M: (batch, 128, 128) fp32 with contiguous matrices")
    _need(1 <= k <= 64, "k: 1..64")
    B = M.shape[0]
    m_stride = M.stride(0) if B > 1 else HEAD_DIM * HEAD_DIM
    if sweeps is not None:
        _need(sweeps.dtype == torch.int32 and sweeps.is_contiguous() and sweeps.numel() >= B,
              "sweeps: >= batch int32, contiguous")
    ev = torch.empty(B, k, device=dev, dtype=torch.float32)
    vec = torch.empty(B, HEAD_DIM, k, device=dev, dtype=torch.float32)
    if B:
        lib.call("oa_sym_eig_top", _ptr(M), m_stride, B, HEAD_DIM, k, _ptr(ev), _ptr(vec),
                 _ptr(sweeps), _stream(dev))
    return ev, vec


def qgc_project(K, T: int, W, G: int, zraw, colmean, zP=None) -> None:
    """a12 projection: zraw (HQ, T, 16) int16/bf16 = bf16(k W) (what kmeans_assign and
    kmeans_update read); colmean (HQ, 16); zP (HQ, T, 16) fp32 = bf16(k W) - colmean, or None."""
    dev = _dev(K, W, zraw, colmean)
    HQ = W.shape[0]
    _need(W.dtype == torch.bfloat16 and W.is_contiguous() and W.shape[1:] == (HEAD_DIM, RANK_C),
          "W: (HQ, 128, 16) bf16 contiguous")
    _need(K.shape[0] * G == HQ and T <= K.shape[1], "K: HQ / G rows of at least T tokens")
    _zraw(zraw, HQ, T)
    _need(colmean.is_contiguous() and colmean.shape == (HQ, RANK_C), "colmean: (HQ, 16) contiguous")
    if zP is not None:
        _need(zP.dtype == torch.float32 and zP.stride() == zraw.stride(), "zP: fp32, zraw's strides")
    ntiles = -(-T // 64)
    ws = torch.empty(HQ * ntiles * RANK_C, device=dev, dtype=torch.float64)
    lib.call("oa_qgc_project", _ptr(K), K.stride(0), K.stride(1), HQ, G, T, _ptr(W), _ptr(zP),
             zraw.stride(0), _ptr(colmean), _ptr(ws), _ptr(zraw), _stream(dev))


def _zraw(zraw, HQ: int, T: int) -> None:
    _need(zraw.element_size() == 2 and zraw.dim() == 3 and zraw.shape[0] == HQ and zraw.shape[1] >= T
          and zraw.shape[2] == RANK_C and zraw.stride(2) == 1 and zraw.stride(1) == RANK_C,
          "zraw: (HQ, >=T, 16) 16-bit rows")


def kmeans_assign(zraw, colmean, T: int, cent, asg, asg8) -> None:
    """a12 assignment into asg (HQ, >=T) int32 and asg8 (HQ, >=T) uint8 rows; zP = zraw - colmean
    formed on the fly from the bf16 projection."""
    dev = _dev(zraw, colmean, cent, asg, asg8)
    HQ, C = cent.shape[0], cent.shape[1]
    _zraw(zraw, HQ, T)
    _need(colmean.is_contiguous() and colmean.shape == (HQ, RANK_C), "colmean: (HQ, 16) contiguous")
    _need(cent.is_contiguous() and cent.shape[2] == RANK_C, "cent: (HQ, C, 16) contiguous")
    _need(asg.stride(1) == 1 and asg8.stride(1) == 1, "asg rows must be contiguous")
    lib.call("oa_kmeans_assign", _ptr(zraw), _ptr(colmean), zraw.stride(0), HQ, T, _ptr(cent), C, _ptr(asg),
             asg.stride(0), _ptr(asg8), asg8.stride(0), _stream(dev))


def kmeans_update(zraw, colmean, T: int, asg8, init, cent, mem, cstart, clen, cnt=None) -> None:
    """a12 update of cent (HQ, C, 16) in place; init (C,) int32 initial positions; zP as in
    kmeans_assign; mem (HQ, >=T), cstart, clen (HQ, C) int32 receive the assignment's member lists."""
    dev = _dev(zraw, colmean, asg8, init, cent, mem, cstart, clen)
    HQ, C = cent.shape[0], cent.shape[1]
    _zraw(zraw, HQ, T)
    _need(colmean.is_contiguous() and colmean.shape == (HQ, RANK_C), "colmean: (HQ, 16) contiguous")
    _need(init.dtype == torch.int32 and init.numel() == C, "init: (C,) int32")
    _chk(mem, "mem", torch.int32, (HQ, -T))
    _chk(cstart, "cstart", torch.int32, (HQ, C), contiguous=True)
    _chk(clen, "clen", torch.int32, (HQ, C), contiguous=True)
    lib.call("oa_kmeans_update", _ptr(zraw), _ptr(colmean), zraw.stride(0), HQ, T, _ptr(asg8), asg8.stride(0),
             C, _ptr(init), _ptr(cent), _ptr(cnt), _ptr(mem), mem.stride(0), _ptr(cstart), _ptr(clen),
             _stream(dev))


def cluster_sums(K, V, T: int, G: int, C: int, nb, Sk, Sk2, Sv, mem, cstart, clen) -> None:
    """a13 over member lists already built (kmeans_update's for the assignment it was given):
    nb = clen, Sk/Sk2/Sv as cluster_build, which would sort that assignment again."""
    dev = _dev(K, V, nb, Sk, Sk2, Sv, mem, cstart, clen)
    HQ = nb.shape[0]
    _need(K.stride() == V.stride() and K.stride(-1) == 1, "K, V: same strides, contiguous rows")
    _need(K.shape[0] * G == HQ and T <= K.shape[1], "K: HQ / G rows of at least T tokens")
    for t, nm in ((nb, "nb"), (Sk, "Sk"), (Sk2, "Sk2"), (Sv, "Sv"), (cstart, "cstart"), (clen, "clen")):
        _need(t.is_contiguous(), f"{nm} must be contiguous")
    _need(mem.dtype == torch.int32 and mem.stride(-1) == 1 and cstart.dtype == torch.int32
          and clen.dtype == torch.int32, "mem, cstart, clen: int32")
    lib.call("oa_cluster_sums", _ptr(K), _ptr(V), K.stride(0), K.stride(1), HQ, G, T, C, _ptr(nb),
             _ptr(Sk), _ptr(Sk2), _ptr(Sv), _ptr(mem), mem.stride(0), _ptr(cstart), _ptr(clen),
             _stream(dev))


def cluster_build(K, V, T: int, G: int, asg8, C: int, nb, Sk, Sk2, Sv, mem, cstart, clen) -> None:
    """a13: nb (HQ, C), Sk/Sk2/Sv (HQ, C, 128), mem (HQ, >=T), cstart/clen (HQ, C)."""
    dev = _dev(K, V, asg8, nb, Sk, Sk2, Sv, mem, cstart, clen)
    HQ = nb.shape[0]
    _need(K.stride() == V.stride() and K.stride(-1) == 1, "K, V: same strides, contiguous rows")
    _need(K.shape[0] * G == HQ and T <= K.shape[1], "K: HQ / G rows of at least T tokens")
    for t, nm in ((nb, "nb"), (Sk, "Sk"), (Sk2, "Sk2"), (Sv, "Sv"), (cstart, "cstart"), (clen, "clen")):
        _need(t.is_contiguous(), f"{nm} must be contiguous")
    lib.call("oa_cluster_build", _ptr(K), _ptr(V), K.stride(0), K.stride(1), HQ, G, T, _ptr(asg8),
             asg8.stride(0), C, _ptr(nb), _ptr(Sk), _ptr(Sk2), _ptr(Sv), _ptr(mem), mem.stride(0),
             _ptr(cstart), _ptr(clen), _stream(dev))
