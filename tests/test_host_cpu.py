"""Host-side logic on the CPU: budget accounting, the prefill build (metric, codes, clusters,
sums, CSR) and the composed restatement of the decode step."""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from openattention_amd import prefill, synth
from openattention_amd.budget import DEPLOYED, budget
from tests.helpers import D, G, HKV, HQ, SC, SC2, bf16_np, bf16_to_f32, build_layer, state_np


# ------------------------------------------------------------------ budget
def test_budget_counts_match_reference_accounting():
    # run_openattention.sh:27-31 split, methods_eager.py:605-607 counts at n = 32768
    assert budget(0.01).counts(32768) == (3, 3, 9)
    assert budget(0.03).counts(32768) == (3, 3, 9)
    assert budget(0.05).counts(32768) == (3, 3, 8)
    assert budget(0.10).counts(32768) == (3, 3, 9)
    assert {r: (budget(r).C, budget(r).E) for r in DEPLOYED} == DEPLOYED
    # config 1 (N=4096, C and E scaled with the accounting context): the multibin masker sizes
    # int(1e-4 * n) are 0 there, the deployed floor is 1
    b = budget(0.01, ctx_len=4096)
    assert (b.C, b.E) == (8, 27)
    assert b.counts(4096) == (0, 0, 1)
    assert budget(0.01, ctx_len=4096, rule="deployed").counts(4096) == (1, 1, 1)
    # realised read at 32K and 1% (reference accounting): (6 + 9 + 216 + 96) / 32768
    assert abs(budget(0.01).realised_read(32768) - 327 / 32768) < 1e-12
    with pytest.raises(ValueError):
        budget(0.02)


# ------------------------------------------------------------------ build (a11-a13)
@pytest.fixture(scope="module")
def lay():
    return build_layer(cfg=1, B=1, N=4096, Lmax=4096 + 16, C=8, n_centers=64, dev="cpu")


def test_build_invariants(lay):
    st, T = lay.st, lay.T
    codes = st.codes[:, :T].to(torch.int32)
    assert int(codes.abs().max()) == 127                       # scale = max|zc| / 127
    # codes reproduce k U / scale up to rounding
    k = lay.K[0, :, :T].float()
    zc = torch.matmul(k, st.U[:HKV])
    assert torch.all((zc / st.scale[:HKV, None, :] - codes).abs() <= 0.5 + 1e-3)
    # U orthonormal columns, W = eigvecs * sqrt(eigvals) (rank 16)
    assert torch.allclose(st.U[0].T @ st.U[0], torch.eye(32), atol=1e-4)
    # every token assigned, counts and sums consistent, CSR grouped and position-ordered
    asg = st.asg[:, :T].long()
    assert int(asg.min()) >= 0 and int(asg.max()) < lay.C
    assert torch.all(st.nb.sum(1) == T)
    for r in (0, 5, 31):
        kv = r // G
        kr = lay.K[0, kv, :T].float()
        ref = torch.zeros(lay.C, D).index_add_(0, asg[r], kr)
        assert torch.allclose(st.Sk[r], ref, atol=1e-3, rtol=1e-4)
        mem = st.mem[r, :T].long()
        assert torch.equal(torch.sort(mem).values, torch.arange(T))
        for c in range(lay.C):
            s, l = int(st.cstart[r, c]), int(st.clen[r, c])
            seg = mem[s:s + l]
            assert torch.all(asg[r, seg] == c)
            assert torch.all(seg[1:] > seg[:-1])


def test_kmeans_assignment_is_nearest_under_bf16_rule(lay):
    """After the last Lloyd step every point sits at its nearest centroid of the previous
    centroids; re-running one assignment with the final centroids moves few points (Lloyd
    has converged in 4 iterations on the mixture)."""
    st, T = lay.st, lay.T
    k = lay.K[0, :, :T]
    krep = k.repeat_interleave(G, 0)
    zP = torch.matmul(krep, st.W[:HQ]).float() - st.colmean[:HQ, None, :]
    half = (0.5 * (st.cent[:HQ] ** 2).sum(-1)).to(torch.bfloat16).unsqueeze(1)
    a = (torch.matmul(zP.to(torch.bfloat16), st.cent[:HQ].to(torch.bfloat16).transpose(1, 2)) - half).argmax(-1)
    moved = (a != st.asg[:HQ, :T].long()).float().mean().item()
    assert moved < 0.05, moved


# ------------------------------------------------------------------ composed decode step
def test_oracle_decode_step_invariants_and_accuracy(lay):
    n = lay.N
    b = budget(0.01, ctx_len=lay.N)
    assert b.C == lay.C
    ns, nl, k = b.counts(n)
    st = state_np(lay)
    q = bf16_np(lay.q.reshape(-1, D))
    r = O.decode_step(st, q, n, ns, nl, k, b.E, G, np.float32(SC), np.float32(SC2))
    R = HQ
    assert r["sel"].shape == (R, ns + nl + k)
    assert np.array_equal(r["quota"].sum(1), np.minimum(b.E, np.where(r["n_t"] > 1, r["n_t"], 0).sum(1)))
    for row in range(R):
        ex = r["exp_idx"][row]
        ex = ex[ex >= 0]
        assert len(set(ex.tolist())) == len(ex)
        assert not (set(ex.tolist()) & set(r["sel"][row].tolist()))
        assert np.all(ex < n)
        # each expanded token belongs to the cluster of its segment
        base = 0
        for c in range(lay.C):
            qc = int(r["quota"][row, c])
            assert np.all(st["asg"][row, r["exp_idx"][row, base:base + qc]] == c)
            base += qc

    # the estimator converges to dense attention as the exact-read budget grows, and equals it
    # once every tail token is read (each query here attends ~64 near-tied keys of its mixture
    # component, which the 1% budget cannot cover, so no accuracy bound is asserted at 1%)
    dense = O.dense(q, st["K"], st["V"], n, G, SC)
    for E, bound in ((500, 1e-2), (5000, 1e-6)):
        st2 = state_np(lay)
        r2 = O.decode_step(st2, q, n, ns, nl, k, E, G, np.float32(SC), np.float32(SC2))
        rel = np.linalg.norm(r2["out"] - dense, axis=1) / np.linalg.norm(dense, axis=1)
        assert rel.max() < bound, (E, rel.max())


# ------------------------------------------------------------------ accuracy-path surface
def test_custom_attention_protocol_errors_on_the_host():
    """UTAMultiBinHIP.custom_attention raises the reference's errors before touching a device:
    no sparse_meta_data (multibin.py:2886-2887), no layer_idx (static_top_k.py:226-228), and a
    HIP device is required for the kernels (no CPU fallback)."""
    from openattention_amd.multibin import UTAMultiBinHIP
    att = UTAMultiBinHIP(rho=0.01, static=synth.static_metric(1), ctx_len=4096)
    q = torch.zeros(1, HQ, 1, D, dtype=torch.bfloat16)
    k = torch.zeros(1, HKV, 4096, D, dtype=torch.bfloat16)
    mod = object()
    with pytest.raises(ValueError, match="sparse_meta_data"):
        att.custom_attention(mod, q, k, k, None, SC, 0.0, layer_idx=0)
    with pytest.raises(ValueError, match="layer_idx"):
        att.custom_attention(mod, q, k, k, None, SC, 0.0, sparse_meta_data={})
    with pytest.raises(ValueError, match="bfloat16"):
        att.custom_attention(mod, q.float(), k, k, None, SC, 0.0, sparse_meta_data={}, layer_idx=0)
    with pytest.raises(RuntimeError, match="HIP device"):
        att.custom_attention(mod, q, k, k, None, SC, 0.0, sparse_meta_data={}, layer_idx=0)
    with pytest.raises(ValueError, match="static"):
        UTAMultiBinHIP(rho=0.01)


def test_kmeans_init_is_a_seeded_sample_of_distinct_positions():
    """The initial centroid positions: C distinct prefix positions, the product's and the
    restatement's the same, a different draw per layer, and a prefix of one permutation (so a
    larger C extends a smaller one), which is what taking the first C of randperm(T) means."""
    T, C = 4095, 64
    for layer in (0, 5):
        got = prefill.kmeans_init(T, C, layer).numpy()
        assert np.array_equal(got, O.kmeans_init(T, C, layer))
        assert len(set(got.tolist())) == C and got.min() >= 0 and got.max() < T
        assert np.array_equal(prefill.kmeans_init(T, 2 * C, layer).numpy()[:C], got)
    assert not np.array_equal(prefill.kmeans_init(T, C, 0).numpy(), prefill.kmeans_init(T, C, 1).numpy())
    with pytest.raises(ValueError):
        prefill.kmeans_init(10, 64, 0)


def test_wrapper_layout_checks_reject_wrong_dtype_shape_and_strides():
    """The decode-stage wrappers' host checks (ops._chk): dtype, exact and minimum extents,
    contiguity -- the layouts the kernels index without checking."""
    import torch
    from openattention_amd import ops
    t = torch.zeros(4, 8, 128, dtype=torch.float32)
    ops._chk(t, "t", torch.float32, (4, 8, 128), contiguous=True)
    ops._chk(t, "t", torch.float32, (4, -6, None))
    with pytest.raises(ValueError, match="dtype"):
        ops._chk(t, "t", torch.bfloat16)
    with pytest.raises(ValueError, match="shape"):
        ops._chk(t, "t", torch.float32, (4, -9, 128))
    with pytest.raises(ValueError, match="shape"):
        ops._chk(t, "t", torch.float32, (4, 8))
    with pytest.raises(ValueError, match="contiguous"):
        ops._chk(t[:, ::2], "t", torch.float32, contiguous=True)
    with pytest.raises(ValueError, match="last dimension"):
        ops._chk(t.transpose(1, 2), "t", torch.float32)
    with pytest.raises(ValueError, match="contiguous"):
        ops._stats(4, 4, (t[:, :4], "Sk"))


def test_causal_mask_check_accepts_hf_causal_masks_only():
    """The accuracy-path surface accepts HF's additive causal mask (0 where row i may attend
    j <= K - Q + i, the dtype's minimum or -inf elsewhere; any broadcastable leading dims, longer
    masks sliced to K as multibin.py:2213 does) and None for one row; padding masks are refused."""
    from openattention_amd.multibin import causal_mask_ok

    def causal(Q, K, fill, dtype=torch.bfloat16, lead=(1, 1), extra=0):
        i = torch.arange(Q).view(Q, 1)
        j = torch.arange(K + extra).view(1, K + extra)
        m = torch.zeros(*lead, Q, K + extra, dtype=dtype)
        return m.masked_fill_(j > (K - Q) + i, fill)

    for dtype in (torch.bfloat16, torch.float16, torch.float32):
        assert causal_mask_ok(causal(5, 40, torch.finfo(dtype).min, dtype), 5, 40)
    assert causal_mask_ok(causal(64, 300, float("-inf"), torch.float32, lead=(2, 32)), 64, 300)
    assert causal_mask_ok(causal(3, 50, float("-inf"), torch.float32, extra=7), 3, 50)
    assert causal_mask_ok(None, 1, 50) and not causal_mask_ok(None, 2, 50)
    assert causal_mask_ok(torch.zeros(1, 1, 1, 50), 1, 50)
    bad = causal(5, 40, torch.finfo(torch.float32).min, torch.float32)
    bad[..., 2, 3] = torch.finfo(torch.float32).min              # a padded position
    assert not causal_mask_ok(bad, 5, 40)
    off = causal(5, 40, torch.finfo(torch.float32).min, torch.float32)
    off[..., 4, 39] = -1.0                                        # not a removal, not zero
    assert not causal_mask_ok(off, 5, 40)
    assert not causal_mask_ok(causal(5, 40, -1e4, torch.float32), 5, 40)   # too weak to remove
    assert not causal_mask_ok(causal(4, 40, float("-inf"), torch.float32), 5, 40)
