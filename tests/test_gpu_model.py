"""BASELINE config 5 end to end on the GPU, and config 1's fp32 level.

Config 5: a Llama-3.1-8B-shaped decoder with random-init bf16 weights and a 32K-token random
prompt.  The prompt is prefilled one batch row at a time through the attention hook's prefill
branch (graph_runner.py:615-622, 469-482: K, V into the cache, dense causal attention, the
index built per layer), one decode step runs eagerly, then the next decode step of the whole
model (embedding, every layer, LM head) is captured in a hipGraph and replayed.  At the probed
layers the step's sparse attention is compared with the CPU restatement's decode step
(oracle.decode_step, index update of position n - 1 included) on that layer's captured query
rows and its state before the step: sel, quotas and expanded sets bit-exact; the attention
output within 2e-2 (bf16 rows) and within 1e-3 (fp32 rows).
"""
import types

import numpy as np
import pytest
import torch

from oracle import oracle as O
from openattention_amd import synth
from openattention_amd.method import RMAX, C as CTX, OursHIP
from openattention_amd.model import VOCAB, LlamaShaped
from tests.helpers import D, G, HKV, HQ, SC, SC2, bf16_np, build_layer, seq_state_np

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.bfloat16: 2e-2, torch.float32: 1e-3}


def rel_rows(got, ref):
    return np.linalg.norm(got - ref, axis=-1) / np.maximum(np.linalg.norm(ref, axis=-1), 1e-30)


def _model_step_vs_oracle(B: int, layers: int, probe_layers, seqs, out_dtype, N: int = 32768):
    Lmax = N + 8
    static = synth.static_metric(layers)
    m = OursHIP(types.SimpleNamespace(rho=0.01), B, Lmax, DEV, n_layers=layers, static=static,
                out_dtype=out_dtype)
    CTX.K = [torch.zeros(B, HKV, Lmax, D, device=DEV, dtype=torch.bfloat16) for _ in range(layers)]
    CTX.V = [torch.zeros(B, HKV, Lmax, D, device=DEV, dtype=torch.bfloat16) for _ in range(layers)]
    model = LlamaShaped(B, Lmax, DEV, layers=layers, seed=5, method=m)
    gen = torch.Generator(device="cpu").manual_seed(123 + B)
    tokens = torch.randint(0, VOCAB, (B, N), generator=gen).to(DEV)
    print(f"[case] model prefill B={B} layers={layers} N={N} out={out_dtype}", flush=True)
    model.prefill(tokens, qlen=64)
    torch.cuda.synchronize()
    assert not m._pending, "every layer's index must be built after the prefill"
    probes = model.probe(probe_layers)
    # one eager decode step (n = N + 1) on a side stream, then the step at n = N + 2 captured
    CTX.n_dev = torch.tensor([N + 1], device=DEV, dtype=torch.int32)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        model.step(N + 1)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    n = N + 2
    CTX.n_dev.fill_(n)
    pre = {}
    for l in probe_layers:
        for b in seqs:
            d = seq_state_np(m.st[l], CTX.K[l], CTX.V[l], b)
            del d["K"], d["V"]
            pre[l, b] = d
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        model.step(n)
    torch.cuda.synchronize()
    CTX.n_dev.fill_(n)
    graph.replay()
    torch.cuda.synchronize()
    print(f"[case] captured step replayed; checking layers {list(probe_layers)} sequences {list(seqs)}",
          flush=True)
    ns, nl, k = m.bud.counts(n)
    worst = 0.0
    for l in probe_layers:
        p = {name: t.cpu() for name, t in probes[l].items()}
        for b in seqs:
            r = slice(b * HQ, (b + 1) * HQ)
            st = pre[l, b]
            full = seq_state_np(m.st[l], CTX.K[l], CTX.V[l], b)
            st["K"], st["V"] = full["K"], full["V"]        # K, V after the step: position n - 1 written
            q = bf16_np(p["q"][r])
            ref = O.decode_step(st, q, n, ns, nl, k, m.E, G, np.float32(SC), np.float32(SC2), rmax=RMAX)
            tag = f"layer {l} seq {b}"
            assert np.array_equal(p["sel"][r].numpy(), ref["sel"]), f"{tag}: sel"
            assert np.array_equal(p["quota"][r].numpy(), ref["quota"]), f"{tag}: quota"
            assert np.array_equal(p["exp_idx"][r].numpy()[:, :m.E], ref["exp_idx"]), f"{tag}: exp_idx"
            # the step's index update equals the restatement's
            now = seq_state_np(m.st[l], CTX.K[l], CTX.V[l], b)
            for f in ("codes", "asg", "nb", "Sk", "Sk2", "Sv", "reccnt"):
                assert np.array_equal(now[f], st[f]), f"{tag}: index update {f}"
            rel = rel_rows(p["out"][r].float().numpy(), ref["out"])
            worst = max(worst, float(rel.max()))
            assert rel.max() < TOL[out_dtype], (tag, rel.max())
    print(f"  model step: selection bit-exact at every probed layer, out rel err max {worst:.2e}", flush=True)
    del graph, model, m
    CTX.K, CTX.V = [], []
    torch.cuda.empty_cache()


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_config5_b1_32_layers_prefilled_through_the_hook(out_dtype):
    """B = 1, all 32 layers, a 32K random prompt; layers 0, 15 and 31 checked."""
    _model_step_vs_oracle(1, 32, (0, 15, 31), (0,), out_dtype)


def test_config5_b32_two_layers_prefilled_through_the_hook():
    """B = 32 at N = 32768 through a 2-layer model of the same shapes; sequences 0, 15 and 31 of
    both layers checked."""
    _model_step_vs_oracle(32, 2, (0, 1), (0, 15, 31), torch.bfloat16)


@pytest.mark.parametrize("rule", ["multibin", "deployed"])
def test_config1_shape_fp32_output_rows(rule):
    """Config 1's shape (B = 2, N = 4096, the 1% split scaled to N: C = 8, E = 27) with both
    sink/local/top-k rules: one decode step with bf16 output rows within 2e-2 and, from the
    same kernels with fp32 output rows, within 1e-3 of the restatement; selection bit-exact."""
    print(f"[case] config1 fp32 rows rule={rule}", flush=True)
    lay = build_layer(cfg=1, B=2, N=4096, Lmax=4096 + 64, C=8, n_centers=64, dev=DEV)
    CTX.K, CTX.V = [lay.K], [lay.V]
    CTX.n_dev = torch.tensor([lay.N], device=DEV, dtype=torch.int32)
    res = {}
    for dt in (torch.bfloat16, torch.float32):
        m = OursHIP(types.SimpleNamespace(rho=0.01), lay.B, lay.Lmax, DEV, n_layers=1, static=lay.static,
                    ctx_len=lay.N, rule=rule, out_dtype=dt)
        m.st[0] = lay.st.clone()
        out = m.decode(0, lay.q, lay.N)
        torch.cuda.synchronize()
        res[dt] = (out.float().reshape(-1, D).cpu().numpy(), m.last_sel.cpu().numpy(), m.quota.cpu().numpy(),
                   m.exp_idx.cpu().numpy()[:, :m.E], m.E, m.bud.counts(lay.N))
    for b in range(lay.B):
        pre = seq_state_np(lay.st, lay.K, lay.V, b)
        r = slice(b * HQ, (b + 1) * HQ)
        out, sel, quota, ex, E, (ns, nl, k) = res[torch.float32]
        ref = O.decode_step(pre, bf16_np(lay.q[b].reshape(-1, D)), lay.N, ns, nl, k, E, G, np.float32(SC),
                            np.float32(SC2), rmax=RMAX)
        for dt in (torch.bfloat16, torch.float32):
            out, sel, quota, ex, _, _ = res[dt]
            assert np.array_equal(sel[r], ref["sel"]) and np.array_equal(quota[r], ref["quota"])
            assert np.array_equal(ex[r], ref["exp_idx"])
            rel = rel_rows(out[r], ref["out"])
            print(f"  config1 {rule} b={b} {str(dt)[6:]}: out rel err max {rel.max():.2e}", flush=True)
            assert rel.max() < TOL[dt]
