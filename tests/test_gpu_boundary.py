"""The drop-in boundary on the GPU, driven the way the reference drives it.

  attn_hook (graph_runner.py:469-482): the prefill branch writes each batch row's K, V into the
      cache, returns dense causal attention and builds the row's index through OursHIP.build
      (question rows = the last C.qlen[b] prefill rows); the decode branch appends the new K, V
      at the device-side C.kv_idx and runs the sparse step, captured in a hipGraph and replayed.
  UTAMultiBinHIP.custom_attention (multibin.py:2875-2970): a question-chunk call (Q >= 8)
      builds the index, Q = 1 calls decode, the protocol's errors are raised.

Both are compared with the CPU restatement: selection, quotas and expanded sets bit-exact,
outputs within the bf16 bar; the dense prefill rows against an fp32 CPU attention.
"""
import types

import numpy as np
import pytest
import torch

from oracle import oracle as O
from openattention_amd import method as M
from openattention_amd import synth
from openattention_amd.multibin import UTAMultiBinHIP
from openattention_amd.prefill import LayerState, build_row, build_rows
from tests.helpers import D, G, HKV, HQ, SC, SC2, bf16_np, seq_state_np

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF16_TOL = 2e-2
RMAX = M.RMAX


def rel_rows(got, ref):
    return np.linalg.norm(got - ref, axis=-1) / np.maximum(np.linalg.norm(ref, axis=-1), 1e-30)


def causal_ref(q, k, v, scale):
    """fp32 CPU attention: q (HQ, Q, D) at the last Q positions of k, v (HKV, K, D)."""
    q, k, v = q.float().cpu(), k.float().cpu(), v.float().cpu()
    Q, K = q.shape[1], k.shape[1]
    kk = k.repeat_interleave(q.shape[0] // k.shape[0], 0)
    vv = v.repeat_interleave(q.shape[0] // k.shape[0], 0)
    s = torch.matmul(q, kk.transpose(1, 2)) * scale
    last = K - Q + torch.arange(Q)
    s.masked_fill_(torch.arange(K)[None, :] > last[:, None], float("-inf"))
    return torch.matmul(torch.softmax(s, -1), vv).numpy()


def _check_step(res_sel, res_quota, res_exp, res_out, pre, q_rows, n, bud, E, tag):
    ns, nl, k = bud.counts(n)
    ref = O.decode_step(pre, q_rows, n, ns, nl, k, E, G, np.float32(SC), np.float32(SC2), rmax=RMAX)
    assert np.array_equal(res_sel, ref["sel"]), f"{tag}: sel"
    assert np.array_equal(res_quota, ref["quota"]), f"{tag}: quota"
    assert np.array_equal(res_exp, ref["exp_idx"]), f"{tag}: exp_idx"
    rel = rel_rows(res_out, ref["out"])
    print(f"  {tag}: out rel err max {rel.max():.2e}", flush=True)
    assert rel.max() < BF16_TOL


def test_attn_hook_prefill_then_graph_decode():
    print("[case] attn_hook prefill + captured decode", flush=True)
    B, N, Qn = 2, 2048, 64
    T = N - 1
    Lmax = N + 64
    K, V, q, qq, _ = synth.make_layer(1, B, N, Lmax, 64, DEV)
    static = synth.static_metric(1, dev="cpu")
    m = M.OursHIP(types.SimpleNamespace(rho=0.01), B, Lmax, DEV, n_layers=1, static=static, ctx_len=N)
    C = M.C
    C.K = [torch.zeros_like(K)]
    C.V = [torch.zeros_like(V)]
    C.qlen = [Qn] * B
    C.method = m
    module = types.SimpleNamespace(layer_idx=0)
    # ---- prefill: one call per batch row; the last Qn rows of the prompt are the question
    g = torch.Generator(device=DEV).manual_seed(3)
    C.phase = "prefill"
    ref_state = LayerState(B, HKV, G, Lmax, m.Cn, RMAX, DEV)
    for b in range(B):
        qpre = (torch.randn(1, HQ, T, D, device=DEV, generator=g)).to(torch.bfloat16)
        qpre[0, :, T - Qn:] = qq[b]
        C.brow = b
        out, none = M.attn_hook(module, qpre, K[b:b + 1, :, :T], V[b:b + 1, :, :T], None, scaling=SC)
        torch.cuda.synchronize()
        assert none is None and out.shape == (1, T, HQ, D)
        rows = np.r_[0:8, T - 72:T]
        want = causal_ref(qpre[0][:, rows], K[b, :, :T], V[b, :, :T], SC)
        # rows 0..7 see only the first keys: restate them on their own prefix
        want[:, :8] = causal_ref(qpre[0][:, :8], K[b, :, :8], V[b, :, :8], SC)
        got = out[0].transpose(0, 1)[:, rows].float().cpu().numpy()
        rel = rel_rows(got, want)
        print(f"  prefill row b={b}: rel err max {rel.max():.2e}", flush=True)
        assert rel.max() < BF16_TOL
        build_row(ref_state, b, K[b], V[b], qq[b], T, static["M"][0], static["inv_freq"], 1.0, 0, G)
    torch.cuda.synchronize()
    assert torch.equal(C.K[0][:, :, :T], K[:, :, :T]) and torch.equal(C.V[0][:, :, :T], V[:, :, :T])
    got_st, want_st = m.st[0].to_numpy(), ref_state.to_numpy()
    for f in LayerState.FIELDS:
        assert np.array_equal(got_st[f], want_st[f]), f"hook build: {f}"
    # ---- decode at n = N through the hook, captured once and replayed
    C.phase = "decode"
    C.n = N
    C.n_dev = torch.tensor([N], device=DEV, dtype=torch.int32)
    C.n0_dev = torch.tensor([T], device=DEV, dtype=torch.int32)
    C.kv_idx = torch.tensor([N - 1], device=DEV, dtype=torch.long)
    knew, vnew = K[:, :, N - 1:N].contiguous(), V[:, :, N - 1:N].contiguous()
    pre = {b: seq_state_np(m.st[0], K, V, b) for b in range(B)}      # K, V hold the new row
    base = m.st[0].clone()

    def reset():
        for f in LayerState.FIELDS:
            getattr(m.st[0], f).copy_(getattr(base, f))

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        M.attn_hook(module, q, knew, vnew, None)                    # warm-up
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    reset()
    C.K[0][:, :, N - 1] = 0
    C.V[0][:, :, N - 1] = 0
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        out, _ = M.attn_hook(module, q, knew, vnew, None)
    torch.cuda.synchronize()
    assert not bool(C.K[0][:, :, N - 1].any()), "capture must not run the step"
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(C.K[0][:, :, N - 1], K[:, :, N - 1])
    assert out.shape == (B, 1, HQ, D)
    got = out[:, 0].float().reshape(-1, D).cpu().numpy()
    sel, quota, ex = m.last_sel.cpu().numpy(), m.quota.cpu().numpy(), m.exp_idx.cpu().numpy()[:, :m.E]
    for b in range(B):
        r = slice(b * HQ, (b + 1) * HQ)
        _check_step(sel[r], quota[r], ex[r], got[r], pre[b], bf16_np(q[b].reshape(-1, D)), N, m.bud, m.E,
                    f"hook decode b={b}")


def hf_causal_mask(B: int, Q: int, K: int, dtype=torch.bfloat16) -> torch.Tensor:
    """HF's additive causal mask of Q rows ending at key K - 1: 0 where row i may attend
    (j <= K - Q + i), the dtype's minimum elsewhere."""
    i = torch.arange(Q).view(Q, 1)
    j = torch.arange(K).view(1, K)
    m = torch.zeros(B, 1, Q, K, dtype=dtype)
    m.masked_fill_(j > (K - Q) + i, torch.finfo(dtype).min)
    return m.to(DEV)


def _check_rows(rows, out, pre, q_rows, n_keys, bud, E, b, tol, tag):
    """The recorded rows (i, sel, quota, exp_idx) of sequence b and its output rows
    out (HQ, Q, D) against the restatement's multi-row call on the pre-call state."""
    ns, nl, k = bud.counts(n_keys)
    ref = O.rows_step(pre, q_rows, n_keys, ns, nl, k, E, G, np.float32(SC), np.float32(SC2))
    r = slice(b * HQ, (b + 1) * HQ)
    worst = 0.0
    for i, sel, quota, ex in rows:
        assert np.array_equal(sel.cpu().numpy()[r], ref[i]["sel"]), f"{tag} row {i}: sel"
        assert np.array_equal(quota.cpu().numpy()[r], ref[i]["quota"]), f"{tag} row {i}: quota"
        assert np.array_equal(ex.cpu().numpy()[r, :E], ref[i]["exp_idx"]), f"{tag} row {i}: exp_idx"
        rel = rel_rows(out[:, i].float().cpu().numpy(), ref[i]["out"])
        worst = max(worst, float(rel.max()))
    print(f"  {tag}: {len(rows)} rows bit-exact selection, out rel err max {worst:.2e}", flush=True)
    assert worst < tol


@pytest.mark.parametrize("B,N,out_dtype", [(2, 4096, torch.bfloat16), (2, 4096, torch.float32),
                                           (1, 32768, torch.bfloat16)])
def test_custom_attention_question_rows_then_multirow_then_decode(B, N, out_dtype):
    """The accuracy-path surface as the reference drives it (multibin.py:2875-2970):
      * a 64-row question chunk with HF's causal mask builds the index (the state equal to
        build_rows') and every question row gets the estimator's output: row i attends the keys
        before K - 64 + i + 1 (sink, its own local window, top-k, ErrorGate, water-fill, top-q,
        residual proxies, fused softmax); each row's sel, quotas and expanded set equal the
        restatement's multi-row call bit for bit, outputs within 2e-2 (bf16) / 1e-3 (fp32 rows);
      * a 3-row call over 3 appended keys (the index extended first), the same way;
      * two one-row decode calls against the restatement's decode step;
      * the protocol errors: no sparse_meta_data / layer_idx, a decode-sized call before the
        question chunk, a multi-row call without the causal mask or with a padding mask."""
    print(f"[case] custom_attention B={B} N={N} out={out_dtype}", flush=True)
    Qn = 64
    T = N - 1
    Lmax = N + 64
    tol = BF16_TOL if out_dtype == torch.bfloat16 else 1e-3
    K, V, q, qq, _ = synth.make_layer(1 if N == 4096 else 3, B, N, Lmax, 64 if N == 4096 else 256, DEV)
    static = synth.static_metric(1, dev="cpu")
    att = UTAMultiBinHIP(rho=0.01, static=static, ctx_len=N if N != 32768 else 32768, out_dtype=out_dtype,
                         record_rows=True)
    meta = {}
    module = types.SimpleNamespace(layer_idx=0)
    # protocol errors
    with pytest.raises(ValueError, match="sparse_meta_data"):
        att.custom_attention(module, q, K[:, :, :N], V[:, :, :N], None, SC, 0.0, layer_idx=0)
    with pytest.raises(ValueError, match="layer_idx"):
        att.custom_attention(module, q, K[:, :, :N], V[:, :, :N], None, SC, 0.0, sparse_meta_data=meta)
    with pytest.raises(ValueError, match="question chunk"):
        att.custom_attention(module, q, K[:, :, :N], V[:, :, :N], None, SC, 0.0, sparse_meta_data=meta,
                             layer_idx=0)
    # ---- the question chunk: rows at positions T - 64 .. T - 1 of T keys
    keys, values = K[:, :, :T].contiguous(), V[:, :, :T].contiguous()
    out, none = att.custom_attention(module, qq, keys, values, hf_causal_mask(B, Qn, T), SC, 0.0,
                                     sparse_meta_data=meta, layer_idx=0)
    torch.cuda.synchronize()
    assert none is None and out.shape == (B, Qn, HQ, D) and out.dtype == out_dtype
    ref_state = LayerState(B, HKV, G, att_state(meta).Lmax, att_state(meta).C, RMAX, DEV)
    build_rows(ref_state, keys, values, qq, T, static["M"][0], static["inv_freq"], 1.0, 0, G)
    torch.cuda.synchronize()
    got_st, want_st = att_state(meta).to_numpy(), ref_state.to_numpy()
    for f in LayerState.FIELDS:
        assert np.array_equal(got_st[f], want_st[f]), f"question-chunk build: {f}"
    ent = meta["oa_hip"][0]
    m = ent["m"]
    assert len(ent["rows"]) == Qn
    for b in range(B):
        pre = seq_state_np(att_state(meta), K, V, b)
        _check_rows(ent["rows"], out[b].transpose(0, 1), pre, bf16_np(qq[b].transpose(0, 1)), T, m.bud,
                    m.E, b, tol, f"question rows b={b}")
    # ---- a 3-row call over 3 appended keys
    gen = torch.Generator(device=DEV).manual_seed(11)
    for p in range(T, T + 3):
        K[:, :, p] = (K[:, :, 100 + p % 7].float() + 0.3 * torch.randn(B, HKV, D, device=DEV, generator=gen)
                      ).to(torch.bfloat16)
        V[:, :, p] = torch.randn(B, HKV, D, device=DEV, generator=gen).to(torch.bfloat16)
    n3 = T + 3
    keys, values = K[:, :, :n3].contiguous(), V[:, :, :n3].contiguous()
    q3 = qq[:, :, 5:8].contiguous()
    with pytest.raises(NotImplementedError, match="causal mask"):
        att.custom_attention(module, q3, keys, values, None, SC, 0.0, sparse_meta_data=meta, layer_idx=0)
    pad = hf_causal_mask(B, 3, n3)
    pad[:, :, :, 10] = torch.finfo(torch.bfloat16).min
    with pytest.raises(NotImplementedError, match="padding"):
        att.custom_attention(module, q3, keys, values, pad, SC, 0.0, sparse_meta_data=meta, layer_idx=0)
    pres = {b: seq_state_np(att_state(meta), K, V, b) for b in range(B)}
    for b in range(B):
        for p in range(T, n3):
            O.index_update(pres[b], p, G, RMAX)
    out3, _ = att.custom_attention(module, q3, keys, values, hf_causal_mask(B, 3, n3), SC, 0.0,
                                   sparse_meta_data=meta, layer_idx=0)
    torch.cuda.synchronize()
    assert out3.shape == (B, 3, HQ, D) and len(ent["rows"]) == 3
    for b in range(B):
        _check_rows(ent["rows"], out3[b].transpose(0, 1), pres[b], bf16_np(q3[b].transpose(0, 1)), n3, m.bud,
                    m.E, b, tol, f"3-row call b={b}")
    # the multi-row call left the index holding all n3 keys with their full statistics
    for b in range(B):
        now = seq_state_np(att_state(meta), K, V, b)
        for f in ("nb", "Sk", "Sk2", "Sv", "asg", "codes"):
            assert np.array_equal(now[f], pres[b][f]), f"state after the 3-row call: {f}"
    # ---- two one-row decode calls (each key fresh), each against the restatement
    for step in range(2):
        n = n3 + 1 + step
        K[:, :, n - 1] = (K[:, :, 100].float() + 0.3 * torch.randn(B, HKV, D, device=DEV, generator=gen)
                          ).to(torch.bfloat16)
        V[:, :, n - 1] = torch.randn(B, HKV, D, device=DEV, generator=gen).to(torch.bfloat16)
        keys, values = K[:, :, :n].contiguous(), V[:, :, :n].contiguous()
        pre = {b: seq_state_np(att_state(meta), K, V, b) for b in range(B)}
        out, _ = att.custom_attention(module, q, keys, values, None, SC, 0.0, sparse_meta_data=meta,
                                      layer_idx=0)
        torch.cuda.synchronize()
        assert out.shape == (B, 1, HQ, D)
        got = out[:, 0].float().reshape(-1, D).cpu().numpy()
        sel, quota, ex = m.last_sel.cpu().numpy(), m.quota.cpu().numpy(), m.exp_idx.cpu().numpy()[:, :m.E]
        for b in range(B):
            r = slice(b * HQ, (b + 1) * HQ)
            ns, nl, k = m.bud.counts(n)
            ref = O.decode_step(pre[b], bf16_np(q[b].reshape(-1, D)), n, ns, nl, k, m.E, G, np.float32(SC),
                                np.float32(SC2), rmax=RMAX)
            assert np.array_equal(sel[r], ref["sel"]) and np.array_equal(quota[r], ref["quota"])
            assert np.array_equal(ex[r], ref["exp_idx"])
            rel = rel_rows(got[r], ref["out"])
            print(f"  decode step {step} b={b}: out rel err max {rel.max():.2e}", flush=True)
            assert rel.max() < tol


def test_custom_attention_full_mask_rows_are_dense():
    """When a masker returns the full mask (K <= local + Q: a 64-row chunk over 64 keys), the
    reference returns true attention (multibin.py:2916-2920): every row equals fp32 causal
    attention within the bf16 bar."""
    print("[case] custom_attention full mask", flush=True)
    B, T, Qn = 1, 64, 64
    K, V, q, qq, _ = synth.make_layer(1, B, T, T + 16, 8, DEV)
    att = UTAMultiBinHIP(rho=0.01, static=synth.static_metric(1, dev="cpu"), ctx_len=4096)
    out, _ = att.custom_attention(types.SimpleNamespace(layer_idx=0), qq, K[:, :, :T].contiguous(),
                                  V[:, :, :T].contiguous(), hf_causal_mask(B, Qn, T), SC, 0.0,
                                  sparse_meta_data={}, layer_idx=0)
    torch.cuda.synchronize()
    want = causal_ref(qq[0], K[0, :, :T], V[0, :, :T], SC)
    rel = rel_rows(out[0].transpose(0, 1).float().cpu().numpy(), want)
    print(f"  full-mask rows: rel err max {rel.max():.2e}", flush=True)
    assert rel.max() < BF16_TOL


def att_state(meta):
    return meta["oa_hip"][0]["m"].st[0]
