"""The BASELINE configurations end to end on the GPU against the CPU restatement (oracle/):

  config 3  B=32 sequences at N=32768 with the reference's four reads (1%, 3%, 5%, 10%:
            (C, E) = (64, 216), (192, 679), (192, 1335), (256, 2877)), one decode step of
            OursHIP over the whole batch; sequences 0, 15 and 31 restated on the CPU.  Selection,
            quotas and expanded sets bit-exact; the output within 2e-2 (bf16 rows) and, from the
            same kernels with fp32 output rows, within 1e-3 relative error per row.
  config 4  B=1 at N=131072, 1% and 3% (C capped at 256), 512-centre mixture with planted
            needles: the same bar.
"""
import types

import numpy as np
import pytest
import torch

from oracle import oracle as O
from openattention_amd import ops, synth
from openattention_amd.budget import budget
from openattention_amd.method import RMAX, C as CTX, OursHIP
from openattention_amd.prefill import LayerState, build_rows
from tests.helpers import D, G, HKV, HQ, SC, SC2, bf16_np, build_layer, seq_state_np, state_np

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF16_TOL = 2e-2      # north_star: bf16 outputs
F32_TOL = 1e-3       # north_star: fp32 outputs


def rel_rows(got, ref):
    return np.linalg.norm(got - ref, axis=-1) / np.maximum(np.linalg.norm(ref, axis=-1), 1e-30)


def _decode_both_dtypes(st, K, V, q, rho, N, Lmax, B, static, prefix_topq=False):
    """One decode step from (clones of) st with bf16 and with fp32 output rows.  prefix_topq: after
    the bf16 step, top-q again over the step's heads and quotas with every row left to the
    key-prefix kernel (path 3), whose expanded sets land in res["exp_idx_prefix"]."""
    CTX.K, CTX.V = [K], [V]
    CTX.n_dev = torch.tensor([N], device=DEV, dtype=torch.int32)
    CTX.n0_dev = torch.tensor([N - 1], device=DEV, dtype=torch.int32)
    res = {}
    for dt in (torch.bfloat16, torch.float32):
        m = OursHIP(types.SimpleNamespace(rho=rho), B, Lmax, DEV, n_layers=1, static=static, ctx_len=N,
                    out_dtype=dt)
        m.st[0] = st.clone()
        out = m.decode(0, q, N)
        torch.cuda.synchronize()
        res[dt] = dict(out=out.float().reshape(-1, D).cpu().numpy(), sel=m.last_sel.cpu().numpy(),
                       quota=m.quota.cpu().numpy(), exp_idx=m.exp_idx.cpu().numpy()[:, :m.E],
                       E=m.E, counts=m.bud.counts(N))
        if prefix_topq and dt == torch.bfloat16:
            ex = torch.full_like(m.exp_idx, 777)
            ops.topq_heads(m.H, m.st[0].asg8, m.quota, ex, CTX.n_dev, m.st[0].codes, m.limbs, m.fexp, m.S,
                           path=3)
            torch.cuda.synchronize()
            res["exp_idx_prefix"] = ex.cpu().numpy()[:, :m.E]
        del m
        torch.cuda.empty_cache()
    return res


def _check_rows(res, ref, rows, tag):
    for dt, tol in ((torch.bfloat16, BF16_TOL), (torch.float32, F32_TOL)):
        r = res[dt]
        assert np.array_equal(r["sel"][rows], ref["sel"]), f"{tag}: top-k selection differs"
        assert np.array_equal(r["quota"][rows], ref["quota"]), f"{tag}: quotas differ"
        assert np.array_equal(r["exp_idx"][rows], ref["exp_idx"]), f"{tag}: expanded sets differ"
        rel = rel_rows(r["out"][rows], ref["out"])
        print(f"  {tag} {str(dt)[6:]}: out rel err median {np.median(rel):.2e} max {rel.max():.2e}", flush=True)
        assert rel.max() < tol, (tag, str(dt), rel.max())


@pytest.mark.parametrize("rho", [0.01, 0.03, 0.05, 0.10])
def test_config3_batch32_matches_oracle(rho):
    B, N = 32, 32768
    Lmax = N + 64
    bud = budget(rho, ctx_len=N)
    print(f"[case] config3 B={B} N={N} rho={rho} C={bud.C} E={bud.E}", flush=True)
    K, V, q, qq, _ = synth.make_layer(3, B, N, Lmax, 256, DEV)
    static = synth.static_metric(1, dev="cpu")
    st = LayerState(B, HKV, G, Lmax, bud.C, RMAX, DEV)
    build_rows(st, K, V, qq, N - 1, static["M"][0], static["inv_freq"], 1.0, 0, G)
    del qq
    torch.cuda.synchronize()
    seqs = (0, 15, 31)
    pre = {b: seq_state_np(st, K, V, b) for b in seqs}
    res = _decode_both_dtypes(st, K, V, q, rho, N, Lmax, B, static, prefix_topq=rho in (0.01, 0.10))
    ns, nl, k = res[torch.bfloat16]["counts"]
    if "exp_idx_prefix" in res:
        # all 1024 rows through the key-prefix kernel (64 workgroups walking sixteen rows each)
        # equal the step's linear-bin top-q on every row
        bad = np.nonzero((res["exp_idx_prefix"] != res[torch.bfloat16]["exp_idx"]).any(1))[0]
        assert bad.size == 0, f"key-prefix top-q over every row: rows {bad[:8]} differ"
    for b in seqs:
        ref = O.decode_step(pre[b], bf16_np(q[b].reshape(-1, D)), N, ns, nl, k, bud.E, G, np.float32(SC),
                            np.float32(SC2), rmax=RMAX)
        _check_rows(res, ref, slice(b * HQ, (b + 1) * HQ), f"seq {b}")


@pytest.mark.parametrize("rho", [0.01, 0.03])
def test_config4_n131072_matches_oracle(rho):
    N = 131072
    bud = budget(rho, ctx_len=N, c_max=256)
    print(f"[case] config4 B=1 N={N} rho={rho} C={bud.C} E={bud.E}", flush=True)
    lay = build_layer(cfg=4, B=1, N=N, Lmax=N + 64, C=bud.C, n_centers=512, dev=DEV, needles=8)
    pre = state_np(lay)
    res = _decode_both_dtypes(lay.st, lay.K, lay.V, lay.q, rho, N, lay.Lmax, 1, lay.static)
    ns, nl, k = res[torch.bfloat16]["counts"]
    ref = O.decode_step(pre, bf16_np(lay.q.reshape(-1, D)), N, ns, nl, k, bud.E, G, np.float32(SC),
                        np.float32(SC2), rmax=RMAX)
    _check_rows(res, ref, slice(0, HQ), f"N={N}")
    if rho == 0.03:
        # every row through the key-prefix top-q kernel, several times: its refinement levels
        # reserve staging space from many clusters at once (a reservation race once lost a member
        # here now and then)
        m = OursHIP(types.SimpleNamespace(rho=rho), 1, lay.Lmax, DEV, n_layers=1, static=lay.static, ctx_len=N)
        m.st[0] = lay.st.clone()
        m.decode(0, lay.q, N)
        st = m.st[0]
        for rep in range(6):
            ex = torch.full_like(m.exp_idx, -2 if rep % 2 else 777)
            ops.topq_heads(m.H, st.asg8, m.quota, ex, CTX.n_dev, st.codes, m.limbs, m.fexp, m.S, path=3)
            torch.cuda.synchronize()
            got = ex.cpu().numpy()[:, :bud.E]
            bad = np.nonzero((got != ref["exp_idx"]).any(1))[0]
            assert bad.size == 0, f"key-prefix top-q, repeat {rep}: rows {bad} differ"


@pytest.mark.parametrize("N,rho", [(65536, 0.03), (131072, 0.01)])
def test_config4_batch8_matches_oracle(N, rho):
    """Config 4 at its own batch, B = 8 (256 query-head rows: the two-launch ErrorGate path and the
    full-batch top-q), 512-centre mixture with 8 needles per KV head: one decode step of every
    sequence; sequences 0 and 7 restated on the CPU, selection bit-exact, outputs within 2e-2
    (bf16) and 1e-3 (fp32 rows)."""
    B = 8
    bud = budget(rho, ctx_len=N, c_max=256)
    print(f"[case] config4 B={B} N={N} rho={rho} C={bud.C} E={bud.E}", flush=True)
    lay = build_layer(cfg=4, B=B, N=N, Lmax=N + 64, C=bud.C, n_centers=512, dev=DEV, needles=8)
    pres = {b: seq_state_np(lay.st, lay.K, lay.V, b) for b in (0, 7)}
    res = _decode_both_dtypes(lay.st, lay.K, lay.V, lay.q, rho, N, lay.Lmax, B, lay.static)
    ns, nl, k = res[torch.bfloat16]["counts"]
    for b, pre in pres.items():
        ref = O.decode_step(pre, bf16_np(lay.q[b].reshape(-1, D)), N, ns, nl, k, bud.E, G, np.float32(SC),
                            np.float32(SC2), rmax=RMAX)
        _check_rows(res, ref, slice(b * HQ, (b + 1) * HQ), f"N={N} b={b}")
