"""GPU parity of every decode-stage kernel against the CPU restatement (oracle/) on the same
seeded inputs.  Decision outputs (codes, cluster ids, QGS scores, top-k, ErrorGate scores, tail
counts, quotas, expanded sets) must be bit-exact; floating outputs must be within the tolerance
BASELINE.json states for bf16 (2e-2 relative per row; observed errors are printed).
"""
import math
import types

import numpy as np
import pytest
import torch

from oracle import oracle as O
from openattention_amd import ops
from openattention_amd.budget import budget
from openattention_amd.method import RMAX, C as CTX, OursHIP
from openattention_amd.prefill import LayerState
from tests.helpers import (D, G, HKV, HQ, SC, SC2, bf16_np, bf16_to_f32, build_layer, f32_to_bf16,
                           np_bf16, state_np)

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF16_TOL = 2e-2


def rel_rows(got: np.ndarray, ref: np.ndarray) -> np.ndarray:
    den = np.maximum(np.linalg.norm(ref, axis=-1), 1e-30)
    return np.linalg.norm(got - ref, axis=-1) / den


def _i32(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.int32)).to(DEV)


def _f32(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(DEV)


# ------------------------------------------------------------------ OpenAttention.flash
@pytest.mark.parametrize("proxy_per_kv,kb_dtype,n_split,out_dtype", [
    (False, torch.bfloat16, 1, torch.bfloat16), (False, torch.bfloat16, 4, torch.bfloat16),
    (True, torch.float32, 1, torch.bfloat16), (True, torch.bfloat16, 3, torch.bfloat16),
    (False, torch.float32, 1, torch.float32), (True, torch.float32, 5, torch.float32)])
def test_flash_vs_oracle(proxy_per_kv, kb_dtype, n_split, out_dtype):
    """methods_eager.selftest shapes (methods_eager.py:693-728): B=2, Lmax=4096, C=64, Ns=14,
    Ne=216 with 7 -1 pads, 5 proxies per row at -inf.  bf16 output rows within 2e-2; fp32
    output rows (fp32 proxies) within 1e-3 of the fp64 restatement."""
    print(f"[case] flash proxy_per_kv={proxy_per_kv} kb={kb_dtype} split={n_split} out={out_dtype}", flush=True)
    g = torch.Generator().manual_seed(0)
    B, Lmax, Cn, Ns, Ne = 2, 4096, 64, 14, 216
    R, BH = B * HQ, B * HKV
    k = torch.randn(BH, Lmax, D, generator=g).to(torch.bfloat16)
    v = torch.randn(BH, Lmax, D, generator=g).to(torch.bfloat16)
    q = torch.randn(R, D, generator=g).to(torch.bfloat16)
    perm = torch.stack([torch.randperm(Lmax, generator=g) for _ in range(R)])
    sel, ex = perm[:, :Ns].int(), perm[:, Ns:Ns + Ne].int().clone()
    ex[:, -7:] = -1
    PR = BH if proxy_per_kv else R
    kb = torch.randn(PR, Cn, D, generator=g).to(kb_dtype)
    vb = torch.randn(PR, Cn, D, generator=g).to(kb_dtype)
    ln = torch.rand(R, Cn, generator=g) * 5
    ln[:, :5] = -math.inf
    sel[3, :] = -1           # rows with fewer valid entries
    ex[3, :] = -1
    ln[3, :] = -math.inf     # row 3: nothing valid -> 0
    args = [t.to(DEV) for t in (q, k, v, sel, ex, kb, vb, ln)]
    out = torch.empty(R, D, device=DEV, dtype=out_dtype)
    out = ops.flash_decode(*args, proxy_per_kv=proxy_per_kv, sm_scale=SC, n_split=n_split, out=out)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    ref = O.flash(bf16_np(q), bf16_np(k), bf16_np(v), sel.numpy(), ex.numpy(), kb.double().numpy(),
                  vb.double().numpy(), ln.double().numpy(), HQ // HKV, SC, proxy_per_kv=proxy_per_kv)
    assert np.all(got[3] == 0)
    keep = np.arange(R) != 3
    rel = rel_rows(got[keep], ref[keep])
    print(f"  flash rel err median {np.median(rel):.2e} max {rel.max():.2e}")
    assert rel.max() < (1e-3 if out_dtype == torch.float32 else BF16_TOL)


def test_decode_expand_attention_surface():
    """ops.decode_expand_attention with the reference's call shape (triton_expand_decode.py:139-165):
    proxies per KV head, sm_scale defaulting to D**-0.5, the Triton tuning arguments accepted and
    ignored (two different settings give the same output), -1 / -inf entries no-ops; against the
    fp64 restatement within 2e-2 (bf16 rows)."""
    print("[case] decode_expand_attention", flush=True)
    g = torch.Generator().manual_seed(11)
    B, Lmax, Cn, Ns, Ne = 2, 2048, 32, 15, 96
    R, BH = B * HQ, B * HKV
    k = torch.randn(BH, Lmax, D, generator=g).to(torch.bfloat16)
    v = torch.randn(BH, Lmax, D, generator=g).to(torch.bfloat16)
    q = torch.randn(R, D, generator=g).to(torch.bfloat16)
    perm = torch.stack([torch.randperm(Lmax, generator=g) for _ in range(R)])
    sel, ex = perm[:, :Ns].int(), perm[:, Ns:Ns + Ne].int().clone()
    ex[:, -5:] = -1
    kb = torch.randn(BH, Cn, D, generator=g).to(torch.bfloat16)
    vb = torch.randn(BH, Cn, D, generator=g).to(torch.bfloat16)
    ln = torch.rand(R, Cn, generator=g) * 4
    ln[:, ::7] = -math.inf
    args = [t.to(DEV) for t in (q, k, v, sel, ex, kb, vb, ln)]
    out1 = ops.decode_expand_attention(*args)
    out2 = ops.decode_expand_attention(*args, sm_scale=D ** -0.5, block_n=32, block_b=128, num_warps=8)
    torch.cuda.synchronize()
    assert out1.shape == (R, D) and out1.dtype == torch.bfloat16
    assert torch.equal(out1, out2)
    ref = O.flash(bf16_np(q), bf16_np(k), bf16_np(v), sel.numpy(), ex.numpy(), kb.double().numpy(),
                  vb.double().numpy(), ln.double().numpy(), HQ // HKV, SC, proxy_per_kv=True)
    rel = rel_rows(out1.float().cpu().numpy(), ref)
    print(f"  decode_expand_attention rel err max {rel.max():.2e}", flush=True)
    assert rel.max() < BF16_TOL


def test_ours_flash_nb_zero_is_plain_sparse_softmax():
    print("[case] ours_flash nb=0", flush=True)
    from openattention_amd import ours_flash
    g = torch.Generator().manual_seed(1)
    R, BH, Lmax = 64, 16, 1024
    k = torch.randn(BH, Lmax, D, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(BH, Lmax, D, generator=g).to(torch.bfloat16).to(DEV)
    q = torch.randn(R, D, generator=g).to(torch.bfloat16).to(DEV)
    sel = torch.randint(0, Lmax, (R, 40), generator=g).int().to(DEV)
    ex = torch.full((R, 8), -1, dtype=torch.int32).to(DEV)
    kb = torch.randn(R, 4, D, generator=g).to(torch.bfloat16).to(DEV)
    ln = torch.zeros(R, 4).to(DEV)
    o1 = ours_flash(q, k, v, sel, ex, kb, kb, ln, nb=0).float().cpu().numpy()
    ref = O.flash(bf16_np(q), bf16_np(k), bf16_np(v), sel.cpu().numpy(), ex.cpu().numpy(),
                  np.zeros((R, 1, D)), np.zeros((R, 1, D)), np.full((R, 1), -np.inf), 4, SC)
    assert rel_rows(o1, ref).max() < BF16_TOL


# ------------------------------------------------------------------ state-based stages
@pytest.fixture(scope="module")
def lay32k():
    """Config-2 shape: B=1, N=32768, 256-centre mixture, 1% deployed split (C=64, E=216)."""
    print("[case] build B=1 N=32768 C=64", flush=True)
    return build_layer(cfg=2, B=1, N=32768, Lmax=32768 + 64, C=64, n_centers=256, dev=DEV)


@pytest.fixture(scope="module")
def lay4k():
    """Config-1 shape: B=2, N=4096, 64-centre mixture, 1% split scaled to N (C=8, E=27)."""
    print("[case] build B=2 N=4096 C=8", flush=True)
    return build_layer(cfg=1, B=2, N=4096, Lmax=4096 + 64, C=8, n_centers=64, dev=DEV)


def _stages_gpu(lay, q, n, ns, nl, k, E, rmax=RMAX):
    """Run every stage kernel once; returns the intermediates (numpy)."""
    st = lay.st
    R = lay.B * HQ
    K = lay.K.reshape(-1, lay.Lmax, D)
    V = lay.V.reshape(-1, lay.Lmax, D)
    n_dev = torch.tensor([n], device=DEV, dtype=torch.int32)
    n0_dev = torch.tensor([lay.T], device=DEV, dtype=torch.int32)
    ntiles = -(-lay.Lmax // 64)
    S = torch.empty(R, ntiles * 64, device=DEV)
    TM = torch.empty(R, ntiles, device=DEV)
    limbs = torch.zeros(lay.B * HKV, 16, 32, device=DEV, dtype=torch.int8)
    fexp = torch.zeros(R, device=DEV, dtype=torch.int32)
    zq = torch.zeros(R, 32, device=DEV)
    sel = torch.empty(R, ns + nl + k, device=DEV, dtype=torch.int32)
    score = torch.empty(R, lay.C, device=DEV)
    n_t = torch.empty(R, lay.C, device=DEV)
    quota = torch.empty(R, lay.C, device=DEV)
    exp_idx = torch.empty(R, max(E, 1), device=DEV, dtype=torch.int32)
    out = torch.empty(R, D, device=DEV, dtype=torch.bfloat16)
    kbr = torch.empty(R, lay.C, D, device=DEV, dtype=torch.bfloat16)
    vbr = torch.empty_like(kbr)
    lnr = torch.empty(R, lay.C, device=DEV)
    qr = q.reshape(R, D).contiguous()
    r = {}
    ops.index_update(K, V, st, n_dev, rmax)
    torch.cuda.synchronize()
    r["state"] = st.to_numpy()
    ops.qgs_prep(qr, st.U, st.scale, limbs, fexp, zq)
    ops.qgs_scan(st.codes, limbs, fexp, S, TM, n_dev, ns, nl)
    torch.cuda.synchronize()
    r.update(zq=zq.cpu().numpy(), fexp=fexp.cpu().numpy(), limbs=limbs.cpu().numpy(),
             S=S.cpu().numpy().copy(), TM=TM.cpu().numpy())
    ops.topk_select(S, TM, sel, n_dev, ns, nl, k)
    ops.errorgate(qr, K, st.asg, sel, st.Sk, st.Sk2, st.nb, score, n_t, SC)
    ops.waterfill(score, n_t, quota, E)
    score2, n_t2, quota2 = torch.empty_like(score), torch.empty_like(n_t), torch.empty_like(quota)
    qsk = torch.empty_like(score)
    ops.gate_fill(qr, K, st.asg, sel, st.Sk, st.Sk2, st.nb, score2, n_t2, quota2, SC, E, qsk=qsk)
    ops.topq(S, st.asg8, quota, exp_idx, n_dev)
    ops.residual(K, V, st.asg, sel, exp_idx, quota, n_t, st.Sk, st.Sv, kbr, vbr, lnr)
    ops.residual_flash(qr, K, V, st.asg, sel, exp_idx, quota, n_t, st.Sk, st.Sv, out, SC)
    out_q = torch.empty_like(out)
    ops.residual_flash(qr, K, V, st.asg, sel, exp_idx, quota, n_t, st.Sk, st.Sv, out_q, SC, qsk=qsk)
    torch.cuda.synchronize()
    r.update(qsk=qsk.cpu().numpy(), out_q=bf16_to_f32(bf16_np(out_q)),
             Sk_np=st.Sk.cpu().numpy().astype(np.float64), q_np=bf16_to_f32(bf16_np(qr)).astype(np.float64))
    # the same stages over 16-bit key heads (the pipeline the decode step runs)
    H = torch.empty(R, ntiles * 64, device=DEV, dtype=torch.int16)
    TMh = torch.empty_like(TM)
    TMnh = torch.empty_like(TM)
    selh = torch.empty_like(sel)
    S32 = torch.empty(R, ntiles * 64, device=DEV)
    exph = torch.full_like(exp_idx, 777)
    exph3 = torch.full_like(exp_idx, 777)
    expht = torch.full_like(exp_idx, 777)
    ops.qgs_scan_heads(st.codes, limbs, fexp, H, TMh, n_dev, ns, nl, TMn=TMnh)
    torch.cuda.synchronize()
    r.update(H=H.cpu().numpy().view(np.uint16).copy(), TMh=TMh.cpu().numpy(), TMnh=TMnh.cpu().numpy())
    # top-k, gate and fill in one call (one launch below 256 rows) on a copy of the heads
    Hf = H.clone()
    self_ = torch.full_like(sel, -7)
    scf, ntf, qf, qskf = (torch.empty_like(score2), torch.empty_like(n_t2), torch.empty_like(quota2),
                          torch.empty_like(qsk))
    ops.topk_gate_fill(Hf, TMh, n_dev, ns, nl, k, st.codes, limbs, fexp, qr, K, st.asg, self_, st.Sk,
                       st.Sk2, st.nb, scf, ntf, qf, SC, E, qsk=qskf)
    torch.cuda.synchronize()
    r.update(tgf=dict(sel=self_.cpu().numpy(), H=Hf.cpu().numpy().view(np.uint16).copy(),
                      score=scf.cpu().numpy(), n_t=ntf.cpu().numpy(), quota=qf.cpu().numpy(),
                      qsk=qskf.cpu().numpy()))
    ops.topk_select_heads(H, TMh, selh, n_dev, ns, nl, k, st.codes, limbs, fexp)
    ops.topq_heads(H, st.asg8, quota, exph, n_dev, st.codes, limbs, fexp, S32)
    ops.topq_heads(H, st.asg8, quota, exph3, n_dev, st.codes, limbs, fexp, S32, path=3)
    ops.topq_heads(H, st.asg8, quota, expht, n_dev, st.codes, limbs, fexp, S32, TM=TMh, TMn=TMnh)
    torch.cuda.synchronize()
    r.update(H_after=H.cpu().numpy().view(np.uint16).copy(), selh=selh.cpu().numpy(),
             exph=exph.cpu().numpy()[:, :E], exph3=exph3.cpu().numpy()[:, :E],
             expht=expht.cpu().numpy()[:, :E])
    r.update(S_after=S.cpu().numpy(), sel=sel.cpu().numpy(), score=score.cpu().numpy(),
             n_t=n_t.cpu().numpy(), quota=quota.cpu().numpy(), exp_idx=exp_idx.cpu().numpy()[:, :E],
             fused=(score2.cpu().numpy(), n_t2.cpu().numpy(), quota2.cpu().numpy()),
             kbar_r=bf16_to_f32(bf16_np(kbr)), vbar_r=bf16_to_f32(bf16_np(vbr)), log_n=lnr.cpu().numpy(),
             out=bf16_to_f32(bf16_np(out)))
    return r


def score_heads(S):
    """16-bit heads of the order-preserving keys of fp32 scores (the top 16 bits)."""
    u = np.ascontiguousarray(S, dtype=np.float32).view(np.uint32)
    key = np.where(u >> 31 == 1, ~u, u | np.uint32(0x80000000))
    return (key >> 16).astype(np.uint16)


def _compare_step(lay, rho, rule, step_q=None, n=None, tag=""):
    b = budget(rho, ctx_len=lay.N if lay.N < 32768 else 32768, rule=rule)
    n = lay.N if n is None else n
    ns, nl, k = b.counts(n)
    E = b.E
    assert b.C == lay.C
    q = lay.q if step_q is None else step_q
    pre = state_np(lay)
    print(f"[case] stages {tag} B={lay.B} n={n} C={lay.C} E={E} ns={ns} nl={nl} k={k}", flush=True)
    g = _stages_gpu(lay, q, n, ns, nl, k, E)
    ref = O.decode_step(pre, bf16_np(q.reshape(-1, D)), n, ns, nl, k, E, G, np.float32(SC),
                        np.float32(SC2), rmax=RMAX)
    for f in ("codes", "asg", "nb", "Sk", "Sk2", "Sv", "reclist", "reccnt"):
        assert np.array_equal(g["state"][f], pre[f]), f"index update: {f} differs"
    assert np.array_equal(g["state"]["asg8"][:, :n], pre["asg"][:, :n].astype(np.uint8))
    assert np.array_equal(g["zq"], ref["zq"])
    assert np.array_equal(g["fexp"], ref["fexp"])
    # limbs reconstruct Z exactly
    L = g["limbs"].astype(np.int64).reshape(lay.B * HKV, G, 4, 32)
    Zg = (L[:, :, 0] + 256 * L[:, :, 1] + 65536 * L[:, :, 2] + 16777216 * L[:, :, 3]).reshape(-1, 32)
    assert np.array_equal(Zg, ref["Z"])
    S = g["S"][:, :n]
    assert np.array_equal(S, ref["S"][:, :n]), "QGS scores differ"
    ntile_n = -(-n // 64)
    tm_ref = np.full((S.shape[0], ntile_n), -np.inf, np.float32)
    Sp = np.full((S.shape[0], ntile_n * 64), -np.inf, np.float32)
    Sp[:, :n] = S
    tm_ref = Sp.reshape(S.shape[0], ntile_n, 64).max(-1)
    assert np.array_equal(g["TM"][:, :ntile_n], tm_ref)
    assert np.array_equal(g["sel"], ref["sel"]), "top-k selection differs"
    assert np.all(np.take_along_axis(g["S_after"], g["sel"].astype(np.int64), 1) == -np.inf)
    assert np.array_equal(g["n_t"], ref["n_t"])
    assert np.array_equal(g["score"], ref["score"]), "ErrorGate scores differ"
    assert np.array_equal(g["quota"], ref["quota"]), "quotas differ"
    for got, want in zip(g["fused"], (g["score"], g["n_t"], g["quota"])):
        assert np.array_equal(got, want), "fused gate+fill differs from the separate kernels"
    assert np.array_equal(g["exp_idx"], ref["exp_idx"]), "expanded sets differ"
    # the 16-bit key-head pipeline: heads of the exact scores, the same tile maxima, selection
    # and expanded sets (also with every row through the exact-score rows and key-prefix kernel)
    assert np.array_equal(g["H"][:, :n], score_heads(ref["S"][:, :n])), "score heads differ"
    assert np.array_equal(g["TMh"][:, :ntile_n], tm_ref)
    # tile minima of the finite scores (+inf for a tile without one)
    Sf = np.full((S.shape[0], ntile_n * 64), np.inf, np.float32)
    Sf[:, :n] = np.where(S > -np.inf, S, np.inf)
    assert np.array_equal(g["TMnh"][:, :ntile_n], Sf.reshape(S.shape[0], ntile_n, 64).min(-1)), \
        "tile minima differ"
    assert np.array_equal(g["selh"], ref["sel"]), "top-k over heads differs"
    assert np.all(np.take_along_axis(g["H_after"], g["selh"].astype(np.int64), 1) == 0x007F)
    assert np.array_equal(g["exph"], ref["exp_idx"]), "top-q over heads differs"
    assert np.array_equal(g["exph3"], ref["exp_idx"]), "top-q over heads (key-prefix) differs"
    assert np.array_equal(g["expht"], ref["exp_idx"]), "top-q over heads (tile range) differs"
    # top-k + gate + fill in one call: the same selection, marked heads, gate and fill outputs
    t = g["tgf"]
    assert np.array_equal(t["sel"], ref["sel"]), "top-k + gate + fill: selection differs"
    assert np.array_equal(t["H"], g["H_after"]), "top-k + gate + fill: marked heads differ"
    for name, want in (("score", g["score"]), ("n_t", g["n_t"]), ("quota", g["quota"]),
                       ("qsk", g["qsk"])):
        assert np.array_equal(t[name], want), f"top-k + gate + fill: {name} differs"
    live = np.isfinite(ref["log_n"])
    assert np.array_equal(np.isfinite(g["log_n"]), live)
    assert np.allclose(g["log_n"][live], ref["log_n"][live], rtol=1e-6)
    kb_ref = ref["kbar_r"][live]
    err_k = np.abs(g["kbar_r"][live] - kb_ref) / (np.abs(kb_ref) + 1e-2)
    assert err_k.max() < BF16_TOL, err_k.max()
    rel = rel_rows(g["out"], ref["out"])
    print(f"  out rel err median {np.median(rel):.2e} max {rel.max():.2e}; "
          f"exact reads/row {(g['exp_idx'] >= 0).sum(1).mean():.1f} + {g['sel'].shape[1]}")
    assert rel.max() < BF16_TOL
    # q . Sk handed from the gate to the residual pass: the dot against fp64, and the output
    # with it within the same tolerance
    Rr, Cc = g["qsk"].shape
    want = np.einsum("rd,rcd->rc", g["q_np"], g["Sk_np"].reshape(Rr, Cc, -1))
    err = np.abs(g["qsk"] - want) / np.maximum(np.abs(g["Sk_np"]).reshape(Rr, Cc, -1).sum(-1)
                                               * np.abs(g["q_np"]).max(1, keepdims=True), 1e-30)
    assert err.max() < 1e-6, err.max()
    rel_q = rel_rows(g["out_q"], ref["out"])
    assert rel_q.max() < BF16_TOL, rel_q.max()
    return g, ref


def test_stages_config2_shape(lay32k):
    _compare_step(lay32k, 0.01, "multibin", tag="cfg2")


@pytest.mark.parametrize("rule", ["multibin", "deployed"])
def test_stages_config1_shape_both_rules(lay4k, rule):
    """Both sink/local/top-k rules: the accuracy path's int(1e-4 n) and the deployed
    max(1, .) (methods_eager.py:605-607), which at N=4096 selects one sink and one local token."""
    _compare_step(lay4k, 0.01, rule, tag=f"cfg1-{rule}")


@pytest.mark.parametrize("rho", [0.03, 0.05, 0.10])
def test_stages_config3_reads(rho):
    """Every stage kernel at the reference's 3%, 5% and 10% reads at N=32768 (C=192, 192, 256;
    E=679, 1335, 2877): ErrorGate and the water-fill beyond 128 clusters (three and four
    clusters per lane), top-q's 6-bit histogram levels with large quotas."""
    b = budget(rho, ctx_len=32768)
    print(f"[case] build B=1 N=32768 C={b.C} (rho={rho})", flush=True)
    lay = build_layer(cfg=2, B=1, N=32768, Lmax=32768 + 64, C=b.C, n_centers=256, dev=DEV)
    _compare_step(lay, rho, "multibin", tag=f"cfg3-rho{rho}")


def test_decode_steps_track_oracle(lay4k):
    """Several decode steps through OursHIP.decode: the index state, the selection and the
    output follow the CPU restatement step after step (the generated-token lists matter)."""
    print("[case] OursHIP multi-step", flush=True)
    a = types.SimpleNamespace(rho=0.01)
    lay = lay4k
    m = OursHIP(a, lay.B, lay.Lmax, DEV, n_layers=1, static=lay.static, ctx_len=lay.N, rule="deployed")
    m.st[0] = lay.st.clone()
    CTX.K, CTX.V = [lay.K], [lay.V]
    CTX.n0_dev = torch.tensor([lay.T], device=DEV, dtype=torch.int32)
    st_np = state_np(lay)
    g = torch.Generator().manual_seed(5)
    n = lay.N
    for step in range(6):
        # write a fresh token at n-1 (keys near the existing mixture) and decode
        kn = (lay.K[:, :, :64].float().mean(2) + 0.3 * torch.randn(lay.B, HKV, D, generator=g).to(DEV))
        vn = torch.randn(lay.B, HKV, D, generator=g).to(DEV)
        lay.K[:, :, n - 1] = kn.to(torch.bfloat16)
        lay.V[:, :, n - 1] = vn.to(torch.bfloat16)
        st_np["K"] = bf16_np(lay.K.reshape(-1, lay.Lmax, D))
        st_np["V"] = bf16_np(lay.V.reshape(-1, lay.Lmax, D))
        CTX.n_dev = torch.tensor([n], device=DEV, dtype=torch.int32)
        q = (lay.q.float() + 0.05 * torch.randn(lay.q.shape, generator=g).to(DEV)).to(torch.bfloat16)
        out = m.decode(0, q, n)
        torch.cuda.synchronize()
        ns, nl, k = m.bud.counts(n)
        ref = O.decode_step(st_np, bf16_np(q.reshape(-1, D)), n, ns, nl, k, m.E, G, np.float32(SC),
                            np.float32(SC2), rmax=RMAX)
        assert np.array_equal(m.last_sel.cpu().numpy(), ref["sel"]), f"step {step}: sel"
        assert np.array_equal(m.quota.cpu().numpy(), ref["quota"]), f"step {step}: quota"
        assert np.array_equal(m.exp_idx.cpu().numpy()[:, :m.E], ref["exp_idx"]), f"step {step}: exp"
        rel = rel_rows(bf16_to_f32(bf16_np(out.reshape(-1, D))), ref["out"])
        assert rel.max() < BF16_TOL, (step, rel.max())
        for f in ("asg", "nb", "Sk", "reccnt", "reclist", "codes"):
            assert np.array_equal(getattr(m.st[0], f).cpu().numpy(), st_np[f]), f"step {step}: {f}"
        assert np.array_equal(m.st[0].asg8.cpu().numpy()[:, :n], st_np["asg"][:, :n].astype(np.uint8))
        n += 1


def test_topq_generated_list_overflow_fallback(lay4k):
    """Generated tokens that overflow their cluster's list (count > rmax; ours_graph.py:284-287)
    are still expanded like any member: top-q streams every position [0, n) with its cluster
    id, so the expanded set matches the oracle, which derives members from asg alone."""
    print("[case] topq overflow", flush=True)
    lay = lay4k
    st = lay.st.clone()
    small = LayerState(lay.B, HKV, G, lay.Lmax, lay.C, 1, DEV)
    for f in LayerState.FIELDS:
        if f not in ("reclist", "reccnt"):
            getattr(small, f).copy_(getattr(st, f))
    lay2 = types.SimpleNamespace(**{**lay.__dict__, "st": small})
    n = lay.N
    pre = state_np(lay2)
    # the query of every head points at key 100; three generated copies of that key land in
    # its cluster, whose list (capacity 1) overflows, and that cluster takes most of the quota
    q = lay.K[:, :, 100].repeat_interleave(G, 1).unsqueeze(2).contiguous()
    for step in range(3):
        b = budget(0.01, ctx_len=lay.N)
        ns, nl, k = b.counts(n)
        lay.K[:, :, n - 1] = lay.K[:, :, 100]
        pre["K"] = bf16_np(lay.K.reshape(-1, lay.Lmax, D))
        gres = _stages_gpu(lay2, q, n, ns, nl, k, b.E, rmax=1)
        ref = O.decode_step(pre, bf16_np(q.reshape(-1, D)), n, ns, nl, k, b.E, G, np.float32(SC),
                            np.float32(SC2), rmax=1)
        assert np.array_equal(gres["exp_idx"], ref["exp_idx"])
        n += 1
    cnt = small.reccnt.cpu().numpy()
    quota = gres["quota"]
    assert int(cnt.max()) > 1
    assert np.any((cnt > 1) & (quota > 0)), "no overflowed cluster was expanded"


@pytest.mark.parametrize("path", [None, 1])
@pytest.mark.parametrize("n,C,E,seed", [(20000, 16, 300, 1), (8192, 4, 64, 2), (777, 8, 4096, 3),
                                           (20000, 100, 600, 6), (12000, 200, 1000, 7)])
def test_topq_adversarial_quotas(n, C, E, seed, path):
    """Top-q on synthetic rows built to hit every branch: scores on a coarse grid (many ties,
    broken by position), one cluster holding ~60% of the row (more than 1024 members per
    8192-position chunk), quotas above the member count, quota sums above E (a segment cut at
    E), a partial last chunk, and an output buffer holding stale values.  C = 100 and 200 run
    the 7- and 6-bit histogram levels."""
    print(f"[case] topq adversarial n={n} C={C} E={E} path={path}", flush=True)
    rng = np.random.default_rng(seed)
    R, Lmax = 6, -(-(n + 300) // 64) * 64     # row strides: multiples of 4 (oa_topq reads 4 at a time)
    S = np.round(rng.standard_normal((R, Lmax)) * 4) / 4
    S = S.astype(np.float32) + np.float32(0.0)     # no -0.0, as for exact integer scores
    p = np.full(C, 0.4 / (C - 1))
    p[0] = 0.6
    asg = rng.choice(C, size=(R, Lmax), p=p).astype(np.int32)
    asg[:, n:] = 0
    ns = 16
    sel = np.stack([rng.choice(n, ns, replace=False) for _ in range(R)]).astype(np.int32)
    for r in range(R):
        S[r, sel[r]] = -np.inf
    quota = rng.integers(0, 2 * max(E // C, 1) + 3, size=(R, C)).astype(np.float32)
    quota[0, 0] = min(E, 900)          # deep cluster-0 quota: streaming extraction
    quota[1] = 0.0                     # a row with no quota at all
    quota[2, C - 1] = 10 * n           # quota far above membership, past E
    ref = O.topq(S, asg, sel, quota, n, E)
    exp_idx = torch.full((R, E), 12345, device=DEV, dtype=torch.int32)
    n_dev = torch.tensor([n], device=DEV, dtype=torch.int32)
    asg8 = torch.from_numpy(asg.astype(np.uint8)).to(DEV)
    ops.topq(_f32(S), asg8, _f32(quota), exp_idx, n_dev, path=path)
    torch.cuda.synchronize()
    got = exp_idx.cpu().numpy()
    assert np.array_equal(got, ref), f"rows differ: {np.nonzero((got != ref).any(1))[0]}"


@pytest.mark.parametrize("path", [None, 1])
@pytest.mark.parametrize("n,C,E,seed,grid", [(30000, 2, 300, 4, "coarse"), (60000, 4, 512, 5, "coarse"),
                                                (30000, 2, 300, 8, "fine"), (12000, 2, 300, 9, "fine"),
                                                (60000, 256, 3000, 10, "fine")])
def test_topq_deep_histogram_levels(n, C, E, seed, grid, path):
    """Top-q when boundary bins stay too large for the LDS staging space after two histogram
    levels.  "coarse": every score sits in [1, 2) on a grid of eight values, so each level-2 bin
    holds thousands of equal keys: four levels, then the block-wide search over positions.
    "fine": scores 1 + u 2^-20 (u < 2^16), so a third level separates them.  n = 30000 / 60000
    put the level-1 set beyond the gathering list (register passes; 60000 is two register
    segments), n = 12000 keeps it in the list (list passes); C = 256 runs the 6-bit levels."""
    print(f"[case] topq deep levels n={n} C={C} E={E} grid={grid} path={path}", flush=True)
    rng = np.random.default_rng(seed)
    R, Lmax = 3, -(-(n + 300) // 64) * 64
    if grid == "coarse":
        S = (1.0 + rng.integers(0, 8, size=(R, Lmax)) / 8.0).astype(np.float32)
    else:
        S = (1.0 + rng.integers(0, 1 << 16, size=(R, Lmax)) / float(1 << 20)).astype(np.float32)
    asg = rng.integers(0, C, size=(R, Lmax)).astype(np.int32)
    asg[:, n:] = 0
    sel = np.stack([rng.choice(n, 16, replace=False) for _ in range(R)]).astype(np.int32)
    for r in range(R):
        S[r, sel[r]] = -np.inf
    quota = np.zeros((R, C), np.float32)
    quota[0] = E // C                  # every cluster split inside its level-1 bin
    quota[1, 0] = 7                    # one small quota
    quota[2] = rng.integers(1, max(E // C, 2), size=C)
    ref = O.topq(S, asg, sel, quota, n, E)
    exp_idx = torch.full((R, E), 12345, device=DEV, dtype=torch.int32)
    n_dev = torch.tensor([n], device=DEV, dtype=torch.int32)
    asg8 = torch.from_numpy(asg.astype(np.uint8)).to(DEV)
    ops.topq(_f32(S), asg8, _f32(quota), exp_idx, n_dev, path=path)
    torch.cuda.synchronize()
    got = exp_idx.cpu().numpy()
    assert np.array_equal(got, ref), f"rows differ: {np.nonzero((got != ref).any(1))[0]}"


@pytest.mark.parametrize("n,C,E,seed", [(32768, 64, 216, 11), (30000, 128, 700, 12), (50000, 256, 2000, 13)])
def test_topq_linear_bins_and_marked_rows(n, C, E, seed):
    """The linear-bin kernel alone (path 2) on Gaussian scores resolves every row and equals the
    restatement; rows given one huge score (every other member then lands in the lowest linear
    bin, so the boundary bins overflow the staging space) are marked -2 in slot 0 and left to
    the key-prefix kernel, and the two kernels together (path 0) equal the restatement on
    every row."""
    print(f"[case] topq linear n={n} C={C} E={E}", flush=True)
    rng = np.random.default_rng(seed)
    R, Lmax = 8, -(-(n + 300) // 64) * 64
    S = (rng.standard_normal((R, Lmax)) * 8).astype(np.float32)
    asg = rng.integers(0, C, size=(R, Lmax)).astype(np.int32)
    asg[:, n:] = 0
    sel = np.stack([rng.choice(n, 16, replace=False) for _ in range(R)]).astype(np.int32)
    for r in range(R):
        S[r, sel[r]] = -np.inf
    quota = rng.integers(0, 2 * max(E // C, 1) + 2, size=(R, C)).astype(np.float32)
    outlier = [1, 4, 6]
    for r in outlier:
        p = n // 2
        while p in sel[r]:
            p += 1
        S[r, p] = np.float32(3.0e37)
    n_dev = torch.tensor([n], device=DEV, dtype=torch.int32)
    asg8 = torch.from_numpy(asg.astype(np.uint8)).to(DEV)
    ref = O.topq(S, asg, sel, quota, n, E)
    lin = torch.full((R, E), 12345, device=DEV, dtype=torch.int32)
    ops.topq(_f32(S), asg8, _f32(quota), lin, n_dev, path=2)
    both = torch.full((R, E), 12345, device=DEV, dtype=torch.int32)
    ops.topq(_f32(S), asg8, _f32(quota), both, n_dev, path=0)
    torch.cuda.synchronize()
    lin, both = lin.cpu().numpy(), both.cpu().numpy()
    marked = [r for r in range(R) if lin[r, 0] == -2]
    assert marked == outlier, marked
    for r in range(R):
        if r not in outlier:
            assert np.array_equal(lin[r], ref[r]), f"row {r}"
    assert np.array_equal(both, ref), f"rows differ: {np.nonzero((both != ref).any(1))[0]}"


def test_decode_sequence_groups_match_single_chain(lay4k):
    """Running the stage chain per sequence group on separate streams gives the same bits as
    one chain over the whole batch (captured in a graph and replayed, and eagerly)."""
    print("[case] sequence groups", flush=True)
    a = types.SimpleNamespace(rho=0.01)
    lay = lay4k
    outs = []
    for groups in (1, 2):
        m = OursHIP(a, lay.B, lay.Lmax, DEV, n_layers=1, static=lay.static, ctx_len=lay.N, groups=groups)
        for f in LayerState.FIELDS:
            getattr(m.st[0], f).copy_(getattr(lay.st, f))
        CTX.K, CTX.V = [lay.K], [lay.V]
        CTX.n_dev = torch.tensor([lay.N], device=DEV, dtype=torch.int32)
        CTX.n0_dev = torch.tensor([lay.T], device=DEV, dtype=torch.int32)
        o = m.decode(0, lay.q.clone(), lay.N).clone()
        torch.cuda.synchronize()
        outs.append((o, m.exp_idx.clone(), m.quota.clone(), m.st[0].asg.clone()))
    for x, y in zip(outs[0], outs[1]):
        assert torch.equal(x, y)


def test_index_prep_matches_separate_calls(lay4k):
    """oa_index_prep equals oa_index_update followed by oa_qgs_prep, bit for bit."""
    print("[case] index+prep fused", flush=True)
    lay = lay4k
    K = lay.K.reshape(-1, lay.Lmax, D)
    V = lay.V.reshape(-1, lay.Lmax, D)
    n_dev = torch.tensor([lay.N], device=DEV, dtype=torch.int32)
    qr = lay.q.reshape(-1, D).contiguous()
    res = []
    for fused in (False, True):
        st = lay.st.clone()
        limbs = torch.zeros(lay.B * HKV, 16, 32, device=DEV, dtype=torch.int8)
        fexp = torch.zeros(lay.B * HQ, device=DEV, dtype=torch.int32)
        if fused:
            ops.index_prep(K, V, st, n_dev, RMAX, qr, limbs, fexp)
        else:
            ops.index_update(K, V, st, n_dev, RMAX)
            ops.qgs_prep(qr, st.U, st.scale, limbs, fexp)
        torch.cuda.synchronize()
        res.append((st.to_numpy(), limbs.cpu().numpy(), fexp.cpu().numpy()))
    for f in LayerState.FIELDS:
        assert np.array_equal(res[0][0][f], res[1][0][f]), f
    assert np.array_equal(res[0][1], res[1][1])
    assert np.array_equal(res[0][2], res[1][2])


@pytest.mark.parametrize("n,k", [(4096, 9), (40000, 17), (70000, 40), (200000, 64)])
def test_topk_rows_with_ties_large_k(n, k):
    """Top-k over fp32 score rows built for ties: scores on a coarse grid (many equal tile maxima
    and equal scores, ties to the lower position), a few rows of one repeated value, sink and
    local positions and the unwritten tail at -inf as the scan leaves them.  sel (in order) and
    the rows after marking equal the restatement; k > 16 and long rows take the radix-select
    kernel, up to 4096 tiles and k = 64."""
    print(f"[case] topk ties n={n} k={k}", flush=True)
    rng = np.random.default_rng(n + k)
    R, ns, nl = 8, 3, 5
    Lmax = n + 100
    ncols = -(-Lmax // 64) * 64
    S = np.round(rng.normal(0.0, 2.0, (R, ncols)) * 4.0).astype(np.float32) / np.float32(4.0)
    S[1] = 0.5                                            # one value everywhere
    S[2, ::7] = 9.0                                       # many equal maxima
    S[3, : n // 2] = -3.0                                 # half the row tied low
    S[:, :ns] = -np.inf
    S[:, n - nl:] = -np.inf                               # local positions and the unwritten tail
    TM = S.reshape(R, -1, 64).max(axis=2)
    want = O.topk_select(S, n, ns, nl, k)
    St = torch.from_numpy(S).to(DEV)
    TMt = torch.from_numpy(np.ascontiguousarray(TM)).to(DEV)
    sel = torch.empty(R, ns + nl + k, device=DEV, dtype=torch.int32)
    n_dev = torch.tensor([n], device=DEV, dtype=torch.int32)
    ops.topk_select(St, TMt, sel, n_dev, ns, nl, k)
    torch.cuda.synchronize()
    got = sel.cpu().numpy()
    assert np.array_equal(got, want), f"rows {np.nonzero((got != want).any(1))[0]} differ"
    after = St.cpu().numpy()
    marked = S.copy()
    for r in range(R):
        marked[r, want[r, ns + nl:]] = -np.inf
    assert np.array_equal(after, marked)


@pytest.mark.parametrize("Lmax,n,ns,nl,k", [
    (140000, 12, 3, 3, 20),      # radix kernel (k > 16, 2188 tiles): 6 live positions for 20
    (140000, 500, 3, 3, 0),      # radix kernel at k = 0: sink and local only
    (140000, 40, 3, 3, 40),      # radix kernel: 34 live for 40
    (4096, 10, 3, 3, 9),         # register kernel: 4 live for 9
    (4096, 300, 3, 3, 0),        # register kernel at k = 0
])
def test_topk_heads_underfull_rows(Lmax, n, ns, nl, k):
    """The scan over heads, then top-k over heads, on rows with fewer live positions than k_top
    (and k_top = 0): every live position is selected first, then the lowest dead ones (sink,
    local, unwritten) as -inf candidates; sel equals the restatement's, every selected position
    lies below ntiles * 64 and its head is marked, and nothing else in the head rows changes."""
    print(f"[case] topk heads underfull Lmax={Lmax} n={n} k={k}", flush=True)
    rng = np.random.default_rng(Lmax + n + k)
    BH = 2
    R = BH * G
    codes = np.zeros((BH, Lmax, 32), np.int8)
    codes[:, :n] = rng.integers(-127, 128, (BH, n, 32), dtype=np.int8)
    U = rng.normal(size=(BH, D, 32)).astype(np.float32)
    scale = rng.uniform(0.5, 2.0, (BH, 32)).astype(np.float32)
    q16 = f32_to_bf16(rng.normal(size=(R, D)).astype(np.float32))
    _, fexp_ref, Z = O.qgs_prep(q16, U, scale, G)
    S = O.qgs_scores(codes, Z, fexp_ref, G, n, ns, nl)
    want = O.topk_select(S, n, ns, nl, k)
    ntiles = -(-Lmax // 64)
    codes_t = torch.from_numpy(codes).to(DEV)
    limbs = torch.zeros(BH, 16, 32, device=DEV, dtype=torch.int8)
    fexp = torch.zeros(R, device=DEV, dtype=torch.int32)
    ops.qgs_prep(np_bf16(q16, DEV), _f32(U), _f32(scale), limbs, fexp)
    H = torch.empty(R, ntiles * 64, device=DEV, dtype=torch.int16)
    TM = torch.empty(R, ntiles, device=DEV, dtype=torch.float32)
    n_dev = torch.tensor([n], device=DEV, dtype=torch.int32)
    ops.qgs_scan_heads(codes_t, limbs, fexp, H, TM, n_dev, ns, nl)
    torch.cuda.synchronize()
    before = H.cpu().numpy().copy()
    sel = torch.full((R, ns + nl + k), -7, device=DEV, dtype=torch.int32)
    ops.topk_select_heads(H, TM, sel, n_dev, ns, nl, k, codes_t, limbs, fexp)
    torch.cuda.synchronize()
    got = sel.cpu().numpy()
    assert np.array_equal(got, want), f"rows {np.nonzero((got != want).any(1))[0]} differ"
    assert got.min() >= 0 and got.max() < ntiles * 64
    after = H.cpu().numpy()
    marked = before.copy()
    for r in range(R):
        marked[r, want[r, ns + nl:]] = np.int16(0x007F)
    assert np.array_equal(after, marked)


@pytest.mark.parametrize("N,C,k_top", [(4096, 64, 16), (8192, 100, 12), (16384, 192, 9),
                                         (32768, 256, 16)])
def test_small_batch_fused_launches(N, C, k_top):
    """Below 256 rows (one sequence, 32 query-head rows): oa_topk_gate_fill (top-k, gate and
    fill in one launch; here 1 to 4 cluster slots per lane and the k <= 16 register top-k) equals
    oa_topk_select_heads + oa_gate_fill bit for bit and the restatement's sel, scores, tail counts
    and quotas; the one-launch top-q (7/8-, 6/7- and 5/6-bit histogram pairs, 8 / 16 / 36
    positions per thread) gives the restatement's expanded sets on its linear path (path 0), with
    every row in its key-prefix branch (path 3), and the standalone linear kernel (path 2) agrees
    on every row it does not mark; path 0 and 3 again with the row range from the scan's tile
    maxima and minima."""
    print(f"[case] small-batch fused N={N} C={C} k={k_top}", flush=True)
    lay = build_layer(cfg=2, B=1, N=N, Lmax=N + 64, C=C, n_centers=256, dev=DEV)
    st = lay.st
    R = HQ
    n = lay.T
    ns, nl = 3, 3
    E = max(4 * k_top, N // 50)
    ref = O.decode_step(state_np(lay), bf16_np(lay.q.reshape(-1, D)), n, ns, nl, k_top, E, G,
                        np.float32(SC), np.float32(SC2), rmax=RMAX, update_index=False)
    K = lay.K.reshape(-1, lay.Lmax, D)
    qr = lay.q.reshape(R, D).contiguous()
    n_dev = torch.tensor([n], device=DEV, dtype=torch.int32)
    ntiles = -(-lay.Lmax // 64)
    limbs = torch.zeros(HKV, 16, 32, device=DEV, dtype=torch.int8)
    fexp = torch.zeros(R, device=DEV, dtype=torch.int32)
    zq = torch.zeros(R, 32, device=DEV)
    ops.qgs_prep(qr, st.U, st.scale, limbs, fexp, zq)
    H = torch.empty(R, ntiles * 64, device=DEV, dtype=torch.int16)
    TM = torch.empty(R, ntiles, device=DEV)
    TMn = torch.empty(R, ntiles, device=DEV)
    ops.qgs_scan_heads(st.codes, limbs, fexp, H, TM, n_dev, ns, nl, TMn=TMn)
    got = {}
    for fused in (False, True):
        Hx = H.clone()
        sel = torch.full((R, ns + nl + k_top), -7, device=DEV, dtype=torch.int32)
        score, n_t, quota, qsk = (torch.empty(R, C, device=DEV) for _ in range(4))
        if fused:
            ops.topk_gate_fill(Hx, TM, n_dev, ns, nl, k_top, st.codes, limbs, fexp, qr, K, st.asg,
                               sel, st.Sk, st.Sk2, st.nb, score, n_t, quota, SC, E, qsk=qsk)
        else:
            ops.topk_select_heads(Hx, TM, sel, n_dev, ns, nl, k_top, st.codes, limbs, fexp)
            ops.gate_fill(qr, K, st.asg, sel, st.Sk, st.Sk2, st.nb, score, n_t, quota, SC, E, qsk=qsk)
        torch.cuda.synchronize()
        got[fused] = dict(Ht=Hx, quota_t=quota, H=Hx.cpu().numpy(), sel=sel.cpu().numpy(),
                          score=score.cpu().numpy(), n_t=n_t.cpu().numpy(),
                          quota=quota.cpu().numpy(), qsk=qsk.cpu().numpy())
    for name in ("H", "sel", "score", "n_t", "quota", "qsk"):
        assert np.array_equal(got[True][name], got[False][name]), f"fused {name} differs"
    assert np.array_equal(got[True]["sel"], ref["sel"]), "selection differs from the restatement"
    for name in ("score", "n_t", "quota"):
        assert np.array_equal(got[True][name], ref[name]), f"{name} differs from the restatement"
    Hq, quota = got[True]["Ht"], got[True]["quota_t"]
    S32 = torch.empty(R, ntiles * 64, device=DEV)
    e = {}
    for path in (0, 2, 3, "t0", "t3"):
        ex = torch.full((R, E), 777, device=DEV, dtype=torch.int32)
        tiles = dict(TM=TM, TMn=TMn) if isinstance(path, str) else {}
        ops.topq_heads(Hq, st.asg8, quota, ex, n_dev, st.codes, limbs, fexp, S32,
                       path=int(str(path)[-1]), **tiles)
        torch.cuda.synchronize()
        e[path] = ex.cpu().numpy()
    assert np.array_equal(e[0], ref["exp_idx"]), "one-launch top-q (path 0) differs"
    assert np.array_equal(e[3], ref["exp_idx"]), "one-launch top-q, key-prefix branch (path 3) differs"
    assert np.array_equal(e["t0"], ref["exp_idx"]), "top-q with the scan's tile range (path 0) differs"
    assert np.array_equal(e["t3"], ref["exp_idx"]), "top-q with the tile range, key-prefix branch differs"
    done = e[2][:, 0] != -2
    assert np.array_equal(e[2][done], ref["exp_idx"][done]), "linear-bin kernel alone differs"


@pytest.mark.parametrize("C,E", [(8, 27), (64, 216), (100, 679), (192, 1335), (256, 2877), (256, 40)])
def test_waterfill_rows_with_ties_dead_and_full_clusters(C, E):
    """Water-filling on rows built for the leftover tokens: scores on a coarse grid (ties go to
    the lower cluster id), dead clusters (n_t <= 1), clusters that the fill leaves without room,
    rows whose live total is below E (every cluster gets its whole tail), all-dead rows.  The
    integer quotas equal the restatement's on every row, for 1 to 4 cluster slots per lane."""
    print(f"[case] waterfill C={C} E={E}", flush=True)
    rng = np.random.default_rng(1000 * C + E)
    R = 96
    score = rng.normal(0.0, 2.0, (R, C)).astype(np.float32)
    score[::2] = np.round(score[::2] * 2.0) / 2.0
    score[1::4] = 0.25                                    # every score tied
    n_t = rng.integers(0, 3 * max(E // C, 2) + 4, (R, C)).astype(np.float32)
    n_t[:, ::7] = 0.0
    n_t[:, 3::11] = 1.0
    n_t[5] = np.minimum(n_t[5], 2.0)                      # live total below E
    n_t[6] = 0.0                                          # no live cluster
    n_t[7] = 500.0                                        # every cluster far above its share
    want = O.waterfill(score, n_t, E)
    quota = torch.empty(R, C, device=DEV)
    ops.waterfill(torch.from_numpy(score).to(DEV), torch.from_numpy(n_t).to(DEV), quota, E)
    torch.cuda.synchronize()
    got = quota.cpu().numpy()
    bad = np.nonzero((got != want).any(1))[0]
    assert bad.size == 0, f"rows {bad[:8]} differ"
    assert (got.sum(1) <= E).all()


@pytest.mark.parametrize("C", [64, 256])
def test_waterfill_wide_score_spreads(C):
    """Water-filling where many clusters reach their cap at different levels (scores spread over
    40 units, tails from 2 to 1024 tokens) and budgets from one token to nearly the whole tail:
    the water level's estimate needs several capping rounds and, for some rows, proves no bracket,
    so every step is probed.  Quotas equal the restatement's on every row."""
    print(f"[case] waterfill wide C={C}", flush=True)
    rng = np.random.default_rng(77 + C)
    R = 256
    score = rng.uniform(-20.0, 20.0, (R, C)).astype(np.float32)
    n_t = rng.integers(2, 1025, (R, C)).astype(np.float32)
    tot = n_t.astype(np.float64).sum(1)
    for E_frac in (0.0, 0.01, 0.3, 0.97):
        E = max(1, int(E_frac * float(tot.min())))
        want = O.waterfill(score, n_t, E)
        quota = torch.empty(R, C, device=DEV)
        ops.waterfill(torch.from_numpy(score).to(DEV), torch.from_numpy(n_t).to(DEV), quota, E)
        torch.cuda.synchronize()
        got = quota.cpu().numpy()
        bad = np.nonzero((got != want).any(1))[0]
        assert bad.size == 0, f"E={E}: rows {bad[:8]} differ"
        assert (got.sum(1) == E).all()


@pytest.mark.parametrize("C", [128, 200])
def test_index_update_many_clusters(C):
    """The index update with more clusters than lanes (C = 128, 200: each lane scores several
    centroids before the argmax network) equals the restatement bit for bit: codes, cluster ids
    (also the byte stream), counts, pooled sums and generated lists."""
    print(f"[case] index update C={C}", flush=True)
    lay = build_layer(cfg=1, B=1, N=2048, Lmax=2048 + 64, C=C, n_centers=64, dev=DEV)
    K = lay.K.reshape(-1, lay.Lmax, D)
    V = lay.V.reshape(-1, lay.Lmax, D)
    n = lay.N
    pre = state_np(lay)
    st = lay.st.clone()
    limbs = torch.zeros(lay.B * HKV, 16, 32, device=DEV, dtype=torch.int8)
    fexp = torch.zeros(lay.B * HQ, device=DEV, dtype=torch.int32)
    ops.index_prep(K, V, st, torch.tensor([n], device=DEV, dtype=torch.int32), RMAX,
                   lay.q.reshape(-1, D).contiguous(), limbs, fexp)
    torch.cuda.synchronize()
    got = st.to_numpy()
    O.index_update(pre, n - 1, G, RMAX)
    for f in ("codes", "asg", "nb", "Sk", "Sk2", "Sv", "reclist", "reccnt"):
        assert np.array_equal(got[f], pre[f]), f"index update: {f} differs"
    assert np.array_equal(got["asg8"][:, :n], pre["asg"][:, :n].astype(np.uint8))
    assert (pre["asg"][:, n - 1] >= 64).any()         # a winner past the first lane round


def test_dense_decode_vs_oracle(lay4k):
    print("[case] dense", flush=True)
    lay = lay4k
    K = lay.K.reshape(-1, lay.Lmax, D)
    V = lay.V.reshape(-1, lay.Lmax, D)
    n = lay.N - 10
    n_dev = torch.tensor([n], device=DEV, dtype=torch.int32)
    qr = lay.q.reshape(-1, D).contiguous()
    out = ops.dense_decode(qr, K, V, n_dev)
    torch.cuda.synchronize()
    ref = O.dense(bf16_np(qr), bf16_np(K), bf16_np(V), n, G, SC)
    rel = rel_rows(bf16_to_f32(bf16_np(out)), ref)
    print(f"  dense rel err max {rel.max():.2e}")
    assert rel.max() < BF16_TOL


def test_decode_step_graph_replay(lay4k):
    """One decode step captured in a hipGraph replays to the eager result, several times, with
    eager work and synchronisations in between."""
    print("[case] graph replay", flush=True)
    a = types.SimpleNamespace(rho=0.01)
    lay = lay4k
    m = OursHIP(a, lay.B, lay.Lmax, DEV, n_layers=1, static=lay.static, ctx_len=lay.N)
    CTX.K, CTX.V = [lay.K], [lay.V]
    n = lay.N
    CTX.n_dev = torch.tensor([n], device=DEV, dtype=torch.int32)
    CTX.n0_dev = torch.tensor([lay.T], device=DEV, dtype=torch.int32)
    base = lay.st.clone()
    q = lay.q.clone()

    def reset():
        for f in LayerState.FIELDS:
            getattr(m.st[0], f).copy_(getattr(base, f))

    reset()
    eager = m.decode(0, q, n).clone()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        reset()
        m.decode(0, q, n)        # warm-up on the side stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    reset()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        out = m.decode(0, q, n)
    for rep in range(3):
        reset()
        torch.cuda.synchronize()
        _ = torch.randn(1000, device=DEV).sum()   # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep} differs from eager"


# ------------------------------------------------------------------ prefill index build (a11-a13)
def _bf16_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(DEV)


@pytest.mark.parametrize("T", [4095, 777])
def test_build_codes_bit_exact(T):
    print(f"[case] build codes T={T}", flush=True)
    rng = np.random.default_rng(T)
    HKV_, Lmax = 8, 4160
    K = f32_to_bf16(rng.standard_normal((HKV_, Lmax, D)).astype(np.float32))
    U = np.linalg.qr(rng.standard_normal((HKV_, D, D)))[0][..., :32].astype(np.float32)
    codes = torch.zeros(HKV_, Lmax, 32, device=DEV, dtype=torch.int8)
    scale = torch.zeros(HKV_, 32, device=DEV)
    ws = torch.empty(HKV_ * 32, device=DEV, dtype=torch.int32)
    rc, rs = O.qgs_codes(K, T, U)
    # both forms: zc formed twice, and kept in a workspace between the passes
    for zc in (None, torch.full((HKV_ * T * 32,), float("nan"), device=DEV)):
        codes.zero_()
        scale.zero_()
        ops.qgs_codes(_bf16_dev(K), T, _f32(U), codes, scale, ws, zc)
        torch.cuda.synchronize()
        assert np.array_equal(scale.cpu().numpy(), rs)
        assert np.array_equal(codes.cpu().numpy(), rc)


@pytest.mark.parametrize("T,G_", [(4095, 4), (1000, 4), (1000, 2)])
def test_build_projection_and_kmeans(T, G_):
    """QGC projection on the bf16 matrix cores: bf16(k W) agrees with the exact-sum restatement
    up to rare bf16 ties; colmean and zP are bit-exact given the device's bf16(k W), and the
    projection without the fp32 zP writes the same bf16(k W) and colmean.  k-means (zP formed from
    the bf16 projection and colmean as the kernels read it): the assignment agrees with the
    restatement's on the same zP and centroids up to rare ties; the update is bit-exact given the
    device's assignment."""
    print(f"[case] build projection + k-means T={T} G={G_}", flush=True)
    rng = np.random.default_rng(7 + T)
    HKV_, Lmax, C = 2, 4160, 64
    R = HKV_ * G_
    K = f32_to_bf16(rng.standard_normal((HKV_, Lmax, D)).astype(np.float32))
    W = f32_to_bf16((rng.standard_normal((R, D, 16)) * 0.3).astype(np.float32))
    zP = torch.empty(R, T, 16, device=DEV)
    zraw = torch.empty(R, T, 16, device=DEV, dtype=torch.int16)
    cm = torch.empty(R, 16, device=DEV)
    ops.qgc_project(_bf16_dev(K), T, _bf16_dev(W), G_, zraw, cm, zP=zP)
    zraw2 = torch.full((R, T, 16), 7, device=DEV, dtype=torch.int16)
    cm2 = torch.full((R, 16), float("nan"), device=DEV)
    ops.qgc_project(_bf16_dev(K), T, _bf16_dev(W), G_, zraw2, cm2)
    torch.cuda.synchronize()
    assert torch.equal(zraw, zraw2) and torch.equal(cm, cm2)
    zr_gpu = zraw.cpu().numpy().view(np.uint16)
    zr_ref = O.qgc_zraw(K, T, W, G_)
    agree = (zr_gpu == zr_ref).mean()
    print(f"  bf16(kW) agreement {agree:.6f}")
    assert agree > 0.999
    zP_ref, cm_ref = O.qgc_center(zr_gpu)
    assert np.array_equal(cm.cpu().numpy(), cm_ref)
    assert np.array_equal(zP.cpu().numpy(), zP_ref)
    init = rng.choice(T, C, replace=False).astype(np.int32)
    cent = zP[:, torch.from_numpy(init).long().to(DEV)].contiguous()
    asg = torch.full((R, Lmax), -1, device=DEV, dtype=torch.int32)
    asg8 = torch.zeros(R, -(-Lmax // 64) * 64, device=DEV, dtype=torch.uint8)
    zP_np = zP.cpu().numpy()
    init_d = _i32(init)
    for it in range(4):
        cent_np = cent.cpu().numpy()
        ops.kmeans_assign(zraw, cm, T, cent, asg, asg8)
        torch.cuda.synchronize()
        a_gpu = asg.cpu().numpy()[:, :T]
        a_ref = O.kmeans_assign(zP_np, cent_np)
        agree = (a_gpu == a_ref).mean()
        print(f"  iteration {it}: assignment agreement {agree:.6f}")
        assert agree > 0.999
        assert np.array_equal(asg8.cpu().numpy()[:, :T], a_gpu.astype(np.uint8))
        assert np.all(asg.cpu().numpy()[:, T:] == -1)
        cnt = torch.empty(R, C, device=DEV)
        mem_ws = torch.full((R, Lmax), -9, device=DEV, dtype=torch.int32)
        cs_ws, cl_ws = (torch.full((R, C), -9, device=DEV, dtype=torch.int32) for _ in range(2))
        ops.kmeans_update(zraw, cm, T, asg8, init_d, cent, mem_ws, cs_ws, cl_ws, cnt)
        torch.cuda.synchronize()
        c_ref, n_ref = O.kmeans_update(zP_np, a_gpu, C, init)
        assert np.array_equal(cent.cpu().numpy(), c_ref)
        assert np.array_equal(cnt.cpu().numpy(), n_ref)
        # the member lists the update went through: a stable sort of the assignment by cluster
        counts = np.stack([np.bincount(a_gpu[r], minlength=C) for r in range(R)]).astype(np.int32)
        assert np.array_equal(cl_ws.cpu().numpy(), counts)
        assert np.array_equal(cs_ws.cpu().numpy(), np.cumsum(counts, axis=1) - counts)
        mem_ref = np.argsort(a_gpu, axis=1, kind="stable").astype(np.int32)
        assert np.array_equal(mem_ws.cpu().numpy()[:, :T], mem_ref)


def test_kmeans_update_uneven_clusters():
    """The update's member-ordered fp64 sums over clusters of 0, 1, 15, 16, 17, 129 and 2100 +
    members (several staged batches, more than one LDS load of member positions, partial 16-value
    chunks) and a planted assignment: bit-exact with the restatement."""
    print("[case] k-means update, uneven clusters", flush=True)
    rng = np.random.default_rng(23)
    R, T, Lmax, C = 4, 4095, 4160, 8
    zraw = torch.from_numpy(f32_to_bf16((rng.standard_normal((R, T, 16)) * 2.0).astype(np.float32))
                            .view(np.int16)).to(DEV)
    cm = torch.from_numpy(rng.standard_normal((R, 16)).astype(np.float32)).to(DEV)
    zP_np = (bf16_to_f32(zraw.cpu().numpy().view(np.uint16)) - cm.cpu().numpy()[:, None, :]).astype(np.float32)
    sizes = [0, 1, 15, 16, 17, 129]
    a = np.empty((R, T), np.int32)
    for r in range(R):
        lab = np.concatenate([np.full(n, c, np.int32) for c, n in enumerate(sizes)]
                             + [np.full(T - sum(sizes) - 300, 6, np.int32), np.full(300, 7, np.int32)])
        a[r] = rng.permutation(lab)
    asg8 = torch.zeros(R, -(-Lmax // 64) * 64, device=DEV, dtype=torch.uint8)
    asg8[:, :T] = torch.from_numpy(a.astype(np.uint8)).to(DEV)
    init = rng.choice(T, C, replace=False).astype(np.int32)
    cent = torch.full((R, C, 16), float("nan"), device=DEV)
    cnt = torch.empty(R, C, device=DEV)
    mem_ws = torch.empty(R, Lmax, device=DEV, dtype=torch.int32)
    cs_ws, cl_ws = (torch.empty(R, C, device=DEV, dtype=torch.int32) for _ in range(2))
    ops.kmeans_update(zraw, cm, T, asg8, _i32(init), cent, mem_ws, cs_ws, cl_ws, cnt)
    torch.cuda.synchronize()
    c_ref, n_ref = O.kmeans_update(zP_np, a, C, init)
    assert np.array_equal(cnt.cpu().numpy(), n_ref)
    assert np.array_equal(cent.cpu().numpy(), c_ref)


def test_kmeans_assign_with_a_zero_centroid():
    """A centroid at the origin (bf16(|c|^2 / 2) = +0, where bf16(dot - half) can be -0): the
    assignment takes its -0 -> +0 path for the whole row set and still agrees with the
    restatement (-0 and +0 rank as one score, ties to the lower cluster)."""
    print("[case] k-means assignment with a zero centroid", flush=True)
    rng = np.random.default_rng(23)
    HKV_, G_, Lmax, C, T = 2, 4, 4160, 64, 4095
    R = HKV_ * G_
    K = f32_to_bf16(rng.standard_normal((HKV_, Lmax, D)).astype(np.float32))
    W = f32_to_bf16((rng.standard_normal((R, D, 16)) * 0.3).astype(np.float32))
    zP = torch.empty(R, T, 16, device=DEV)
    zraw = torch.empty(R, T, 16, device=DEV, dtype=torch.int16)
    cm = torch.empty(R, 16, device=DEV)
    ops.qgc_project(_bf16_dev(K), T, _bf16_dev(W), G_, zraw, cm, zP=zP)
    init = rng.choice(T, C, replace=False)
    cent = zP[:, torch.from_numpy(init).long().to(DEV)].contiguous()
    cent[:, 5] = 0.0
    asg = torch.full((R, Lmax), -1, device=DEV, dtype=torch.int32)
    asg8 = torch.zeros(R, -(-Lmax // 64) * 64, device=DEV, dtype=torch.uint8)
    ops.kmeans_assign(zraw, cm, T, cent, asg, asg8)
    torch.cuda.synchronize()
    a_gpu = asg.cpu().numpy()[:, :T]
    a_ref = O.kmeans_assign(zP.cpu().numpy(), cent.cpu().numpy())
    agree = (a_gpu == a_ref).mean()
    print(f"  assignment agreement {agree:.6f}; cluster 5 holds {(a_gpu == 5).sum()} tokens")
    assert agree > 0.999
    assert np.array_equal(asg8.cpu().numpy()[:, :T], a_gpu.astype(np.uint8))


@pytest.mark.parametrize("T,C", [(4095, 64), (600, 8)])
def test_build_cluster_stats_bit_exact(T, C):
    print(f"[case] build cluster stats T={T} C={C}", flush=True)
    rng = np.random.default_rng(T + C)
    HKV_, G_, Lmax = 2, 4, 4160
    R = HKV_ * G_
    K = f32_to_bf16(rng.standard_normal((HKV_, Lmax, D)).astype(np.float32))
    V = f32_to_bf16(rng.standard_normal((HKV_, Lmax, D)).astype(np.float32))
    p = rng.dirichlet(np.ones(C) * 0.5)
    asg = rng.choice(C, size=(R, T), p=p).astype(np.int32)
    asg[0, :] = np.where(asg[0] == 1, 0, asg[0])                # an empty cluster in row 0
    asg8 = torch.zeros(R, -(-Lmax // 64) * 64, device=DEV, dtype=torch.uint8)
    asg8[:, :T] = torch.from_numpy(asg.astype(np.uint8)).to(DEV)
    nb = torch.empty(R, C, device=DEV)
    Sk, Sk2, Sv = (torch.empty(R, C, D, device=DEV) for _ in range(3))
    mem = torch.full((R, Lmax), -1, device=DEV, dtype=torch.int32)
    cstart = torch.empty(R, C, device=DEV, dtype=torch.int32)
    clen = torch.empty(R, C, device=DEV, dtype=torch.int32)
    ops.cluster_build(_bf16_dev(K), _bf16_dev(V), T, G_, asg8, C, nb, Sk, Sk2, Sv, mem, cstart, clen)
    torch.cuda.synchronize()
    ref = O.cluster_build(K, V, T, asg, C, G_)
    got = (nb, Sk, Sk2, Sv, mem[:, :T], cstart, clen)
    for name, g, r in zip(("nb", "Sk", "Sk2", "Sv", "mem", "cstart", "clen"), got, ref):
        assert np.array_equal(g.cpu().numpy(), r), name
    assert np.all(mem.cpu().numpy()[:, T:] == -1)
    # the statistics over lists already built (the k-means update's, in the build) are the same
    nb2 = torch.full((R, C), float("nan"), device=DEV)
    Sk_2, Sk2_2, Sv_2 = (torch.full((R, C, D), float("nan"), device=DEV) for _ in range(3))
    ops.cluster_sums(_bf16_dev(K), _bf16_dev(V), T, G_, C, nb2, Sk_2, Sk2_2, Sv_2, mem, cstart, clen)
    torch.cuda.synchronize()
    for name, g, r in zip(("nb", "Sk", "Sk2", "Sv"), (nb2, Sk_2, Sk2_2, Sv_2), (nb, Sk, Sk2, Sv)):
        assert torch.equal(g, r), name


def test_build_rows_equals_build_row():
    """prefill.build_rows (every row's bases from one batched eigh) leaves the same state as
    build_row called row by row."""
    print("[case] build_rows vs build_row", flush=True)
    from openattention_amd import synth
    from openattention_amd.prefill import build_row, build_rows
    B, N, Lmax, C = 2, 2048, 2048 + 64, 8
    K, V, _q, qq, _ = synth.make_layer(1, B, N, Lmax, 64, DEV)
    static = synth.static_metric(1, dev="cpu")
    args = (static["M"][0], static["inv_freq"], float(static["attention_scaling"]), 0, G)
    a = LayerState(B, HKV, G, Lmax, C, RMAX, DEV)
    b = LayerState(B, HKV, G, Lmax, C, RMAX, DEV)
    for r in range(B):
        build_row(a, r, K[r], V[r], qq[r], N - 1, *args)
    build_rows(b, K, V, qq, N - 1, *args)
    torch.cuda.synchronize()
    sa, sb = a.to_numpy(), b.to_numpy()
    for f in LayerState.FIELDS:
        assert np.array_equal(sa[f], sb[f]), f


def test_build_layers_equals_build_rows():
    """prefill.build_layers (every layer's bases from one batched eigh) leaves each layer in the
    state build_rows leaves it in."""
    print("[case] build_layers vs build_rows", flush=True)
    from openattention_amd import synth
    from openattention_amd.prefill import build_layers, build_rows
    B, N, Lmax, C, L = 1, 2048, 2048 + 64, 8, 3
    static = synth.static_metric(L, dev="cpu")
    sc = float(static["attention_scaling"])
    lay = [synth.make_layer(1, B, N, Lmax, 64, DEV, layer=l) for l in range(L)]
    a = [LayerState(B, HKV, G, Lmax, C, RMAX, DEV) for _ in range(L)]
    b = [LayerState(B, HKV, G, Lmax, C, RMAX, DEV) for _ in range(L)]
    for l in range(L):
        build_rows(a[l], lay[l][0], lay[l][1], lay[l][3], N - 1, static["M"][l], static["inv_freq"], sc, l, G)
    build_layers(b, [x[0] for x in lay], [x[1] for x in lay], [x[3] for x in lay], N - 1, static["M"],
                 static["inv_freq"], sc, list(range(L)), G)
    torch.cuda.synchronize()
    for l in range(L):
        sa, sb = a[l].to_numpy(), b[l].to_numpy()
        for f in LayerState.FIELDS:
            assert np.array_equal(sa[f], sb[f]), (l, f)


def test_build_row_bases_match_fp64_restatement():
    """The bases the device build stores (metric in torch on the device, rocSOLVER eigh in fp32)
    span the subspaces of the oracle's fp64 restatement (explicit rotation matrices, numpy
    eigh): projectors U U^T agree, and W W^T is the fp64 metric's best rank-16 part within the
    bf16 bar."""
    print("[case] build_row bases vs fp64 restatement", flush=True)
    lay = build_layer(cfg=1, B=1, N=2048, Lmax=2048 + 64, C=8, n_centers=64, dev=DEV)
    M = O.query_metric(lay.static["M"][0].double().numpy(), lay.qq[0].float().cpu().numpy(), lay.T,
                       lay.static["inv_freq"].double().numpy(), float(lay.static["attention_scaling"]))
    Uo, Wo = O.bases(M, HKV, G)
    U = lay.st.U[:HKV].double().cpu().numpy()
    W = lay.st.W[:HQ].float().double().cpu().numpy()
    PU = U @ np.swapaxes(U, 1, 2)
    PUo = Uo @ np.swapaxes(Uo, 1, 2)
    du = np.abs(PU - PUo).max()
    WW = W @ np.swapaxes(W, 1, 2)
    WWo = Wo @ np.swapaxes(Wo, 1, 2)
    dw = (np.linalg.norm(WW - WWo, axis=(1, 2)) / np.linalg.norm(WWo, axis=(1, 2))).max()
    print(f"  projector max diff {du:.2e}; W W^T rel diff {dw:.2e}")
    assert du < 1e-2
    assert dw < BF16_TOL


def test_build_row_on_device_matches_restated_stages():
    """prefill.build_row (HIP stages) on a fresh layer leaves a state whose codes are the
    restated codes from its own U and whose statistics and member lists are the restated ones
    over its own assignment."""
    print("[case] build_row on device", flush=True)
    lay = build_layer(cfg=1, B=1, N=2048, Lmax=2048 + 64, C=8, n_centers=64, dev=DEV)
    st, T = lay.st, lay.T
    s = st.to_numpy()
    Kb = bf16_np(lay.K[0])
    Vb = bf16_np(lay.V[0])
    rc, rs = O.qgs_codes(Kb, T, s["U"][:HKV])
    assert np.array_equal(s["scale"][:HKV], rs)
    assert np.array_equal(s["codes"][:HKV], rc)
    asg = s["asg"][:HQ, :T]
    nb, Sk, Sk2, Sv, mem, cstart, clen = O.cluster_build(Kb, Vb, T, asg, lay.C, G)
    assert np.array_equal(s["nb"][:HQ], nb)
    assert np.array_equal(s["Sk"][:HQ], Sk) and np.array_equal(s["Sk2"][:HQ], Sk2)
    assert np.array_equal(s["Sv"][:HQ], Sv)
    assert np.array_equal(s["mem"][:HQ, :T], mem)
    assert np.array_equal(s["cstart"][:HQ], cstart) and np.array_equal(s["clen"][:HQ], clen)
    assert np.array_equal(s["asg8"][:HQ, :T], asg.astype(np.uint8))


def test_decode_long_context_needles_match_oracle():
    """Config-4 shape at B=1, N=65536, 1% (C=128, the 7-bit top-q histogram and two register
    segments per row), 512-centre mixture with 8 planted needles per KV head: one decode step
    equals the CPU restatement (selection bit-exact, output within the bf16 bar) and both read
    the same needles."""
    print("[case] decode N=65536 needles", flush=True)
    N = 65536
    b = budget(0.01, ctx_len=N)
    lay = build_layer(cfg=4, B=1, N=N, Lmax=N + 64, C=b.C, n_centers=512, dev=DEV, needles=8)
    m = OursHIP(types.SimpleNamespace(rho=0.01), 1, lay.Lmax, DEV, n_layers=1, static=lay.static, ctx_len=N)
    m.st[0] = lay.st.clone()
    st_np = state_np(lay)
    CTX.K, CTX.V = [lay.K], [lay.V]
    CTX.n_dev = torch.tensor([N], device=DEV, dtype=torch.int32)
    CTX.n0_dev = torch.tensor([lay.T], device=DEV, dtype=torch.int32)
    out = m.decode(0, lay.q, N)
    torch.cuda.synchronize()
    ns, nl, k = m.bud.counts(N)
    ref = O.decode_step(st_np, bf16_np(lay.q.reshape(-1, D)), N, ns, nl, k, m.E, G, np.float32(SC),
                        np.float32(SC2), rmax=RMAX)
    sel, ex = m.last_sel.cpu().numpy(), m.exp_idx.cpu().numpy()[:, :m.E]
    assert np.array_equal(sel, ref["sel"]) and np.array_equal(ex, ref["exp_idx"])
    assert np.array_equal(m.quota.cpu().numpy(), ref["quota"])
    rel = rel_rows(bf16_to_f32(bf16_np(out.reshape(-1, D))), ref["out"])
    assert rel.max() < BF16_TOL
    hit = tot = 0
    for r in range(HQ):
        h, gq = divmod(r, G)
        read = set(sel[r].tolist()) | set(ex[r][ex[r] >= 0].tolist())
        for j in range(8):
            if j % G == gq:
                tot += 1
                hit += int(lay.npos[0, h, j]) in read
    print(f"  needle recall {hit}/{tot}")
    assert tot == 64


def test_model_step_graph_replay_matches_eager():
    """A 2-layer Llama-shaped model on the sparse stage: three captured-step replays give the
    same tokens and leave the same KV cache and index state as three eager steps (KV append at
    the device-side n - 1, n advancing on the device)."""
    print("[case] model step graph replay", flush=True)
    from openattention_amd.model import LlamaShaped
    B_, N, L = 2, 4096, 2
    Lmax = N + 16
    b = budget(0.01, ctx_len=N)
    lays = [build_layer(cfg=1, B=B_, N=N, Lmax=Lmax, C=b.C, n_centers=64, dev=DEV, layer=l) for l in range(L)]
    static = lays[0].static

    def fresh():
        m = OursHIP(types.SimpleNamespace(rho=0.01), B_, Lmax, DEV, n_layers=L, static=static, ctx_len=N)
        m.st = [lays[l].st.clone() for l in range(L)]
        CTX.K = [lays[l].K.clone() for l in range(L)]
        CTX.V = [lays[l].V.clone() for l in range(L)]
        CTX.n0_dev = torch.tensor([N - 1], device=DEV, dtype=torch.int32)
        CTX.n_dev = torch.tensor([N], device=DEV, dtype=torch.int32)
        return m

    model = LlamaShaped(B_, Lmax, DEV, layers=L, method=None)
    model.method = fresh()
    model.tok.fill_(7)
    eager = []
    for i in range(3):
        eager.append(model.step(N + i).clone())
        CTX.n_dev.add_(1)
    torch.cuda.synchronize()
    e_state = [(CTX.K[l].clone(), model.method.st[l].Sk.clone(), model.method.st[l].asg.clone()) for l in range(L)]
    model.method = fresh()
    model.tok.fill_(7)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        model.step(N)
        CTX.n_dev.add_(1)
    torch.cuda.synchronize()
    # capture ran nothing: the state is still the fresh one
    got = []
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        got.append(model.tok.clone())
    for a_, b_ in zip(eager, got):
        assert torch.equal(a_, b_)
    for l in range(L):
        assert torch.equal(CTX.K[l], e_state[l][0])
        assert torch.equal(model.method.st[l].Sk, e_state[l][1])
        assert torch.equal(model.method.st[l].asg, e_state[l][2])
    assert int(CTX.n_dev) == N + 3


@pytest.mark.parametrize("B,N,rho", [(1, 32768, 0.01), (32, 32768, 0.01), (2, 32768, 0.03),
                                     (2, 32768, 0.10), (1, 131072, 0.01), (1, 131072, 0.03)])
def test_split_gate_equals_whole_gate(B, N, rho):
    """The three launch layouts of top-k, ErrorGate and water-fill from one index update:
    oa_qgs_scan_heads + oa_topk_select_heads + oa_gate_fill ("whole"); oa_qgs_scan_gate +
    oa_topk_fix_fill (the pooled ErrorGate in the scan launch, the selected tokens' correction
    with the top-k and the fill: "split"); oa_qgs_scan_heads + oa_topk_gate_fill (each row's top-k
    beside its pooled ErrorGate in one workgroup: "fused").  Key heads, tile maxima, sel, marked
    heads, ErrorGate scores, tail counts, quotas and q . Sk agree bit for bit.  Covers 1 to 4
    cluster slots per lane (C = 64, 192, 256), the register top-k over up to 2048 tiles, the
    radix top-k with the separate launches, and both workgroup widths of the fused launch."""
    bud = budget(rho, ctx_len=N, c_max=256)
    n = N
    ns, nl, k = bud.counts(n)
    E, C = bud.E, bud.C
    print(f"[case] split gate B={B} N={N} rho={rho} C={C} E={E} k={k}", flush=True)
    lay = build_layer(cfg=3 if N == 32768 else 4, B=B, N=N, Lmax=N + 64, C=C,
                      n_centers=256 if N == 32768 else 512, dev=DEV)
    R, BH = B * HQ, B * HKV
    st = lay.st
    K = lay.K.reshape(BH, lay.Lmax, D)
    V = lay.V.reshape(BH, lay.Lmax, D)
    qr = lay.q.reshape(R, D).contiguous()
    limbs = torch.zeros(BH, 16, 32, device=DEV, dtype=torch.int8)
    fexp = torch.zeros(R, device=DEV, dtype=torch.int32)
    n_dev = torch.tensor([n], device=DEV, dtype=torch.int32)
    ops.index_prep(K, V, st, n_dev, RMAX, qr, limbs, fexp)
    ntiles = -(-lay.Lmax // 64)
    res = {}
    for mode in ("whole", "split", "fused"):
        H = torch.empty(R, ntiles * 64, device=DEV, dtype=torch.int16)
        TM = torch.empty(R, ntiles, device=DEV)
        TMn = torch.full((R, ntiles), float("nan"), device=DEV)     # tile minima: whole and split
        sel = torch.full((R, ns + nl + k), -7, device=DEV, dtype=torch.int32)
        score, n_t, quota, qsk = (torch.full((R, C), float("nan"), device=DEV) for _ in range(4))
        if mode == "whole":
            ops.qgs_scan_heads(st.codes, limbs, fexp, H, TM, n_dev, ns, nl, TMn=TMn)
            H0 = H.clone()
            ops.topk_select_heads(H, TM, sel, n_dev, ns, nl, k, st.codes, limbs, fexp)
            ops.gate_fill(qr, K, st.asg, sel, st.Sk, st.Sk2, st.nb, score, n_t, quota, SC, E, qsk=qsk)
        elif mode == "split":
            ops.qgs_scan_gate(st.codes, limbs, fexp, H, TM, n_dev, ns, nl, qr, st.Sk, st.Sk2, st.nb, score, n_t,
                              SC, qsk=qsk, TMn=TMn)
            H0 = H.clone()
            ops.topk_fix_fill(H, TM, n_dev, ns, nl, k, st.codes, limbs, fexp, qr, K, st.asg, sel, st.Sk, st.Sk2,
                              st.nb, score, n_t, quota, SC, E)
        else:
            ops.qgs_scan_heads(st.codes, limbs, fexp, H, TM, n_dev, ns, nl)
            H0 = H.clone()
            ops.topk_gate_fill(H, TM, n_dev, ns, nl, k, st.codes, limbs, fexp, qr, K, st.asg, sel, st.Sk, st.Sk2,
                               st.nb, score, n_t, quota, SC, E, qsk=qsk)
        torch.cuda.synchronize()
        res[mode] = {name: t.cpu().numpy() for name, t in (("H0", H0), ("H", H), ("TM", TM), ("sel", sel),
                                                            ("score", score), ("n_t", n_t), ("quota", quota),
                                                            ("qsk", qsk), ("TMn", TMn))}
    for other in ("split", "fused"):
        for name in ("H0", "H", "TM", "sel", "score", "n_t", "quota", "qsk"):
            a, b = res["whole"][name], res[other][name]
            assert np.array_equal(a, b, equal_nan=False), f"{other}: {name} differs"
    assert np.array_equal(res["whole"]["TMn"], res["split"]["TMn"]), "split: tile minima differ"
    hits = (res["split"]["sel"] >= 0).sum()
    print(f"  bit-exact over {R} rows ({hits} selected tokens)", flush=True)
