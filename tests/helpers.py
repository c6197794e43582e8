"""Shared test helpers: seeded small layer states and torch <-> numpy conversion."""
from __future__ import annotations

import types

import numpy as np
import torch

from openattention_amd import synth
from openattention_amd.budget import budget
from openattention_amd.prefill import LayerState, build_row
from oracle import oracle as O

HQ, HKV, D, G = 32, 8, 128, 4
SC = D ** -0.5
SC2 = float(np.float32(SC * SC))


def bf16_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def np_bf16(a: np.ndarray, dev="cpu") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)


def bf16_to_f32(a: np.ndarray) -> np.ndarray:
    return (a.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return (u >> 16).astype(np.uint16)


def build_layer(cfg: int, B: int, N: int, Lmax: int, C: int, n_centers: int, dev, layer: int = 0,
                rmax: int = 256, static: dict | None = None, needles: int = 0):
    """Synthetic keys/values/queries and a built LayerState for one layer; the prefix is
    N-1 tokens (the decode step writes position N-1)."""
    K, V, q, qq, npos = synth.make_layer(cfg, B, N, Lmax, n_centers, dev, layer=layer, needles=needles)
    if static is None:
        static = synth.static_metric(layer + 1, dev="cpu")
    st = LayerState(B, HKV, G, Lmax, C, rmax, dev)
    T = N - 1
    # the product build runs on the HIP kernels; on the CPU the restatement builds the state
    build = build_row if torch.device(dev).type == "cuda" else O.build_row
    for b in range(B):
        build(st, b, K[b], V[b], qq[b], T, static["M"][layer], static["inv_freq"],
              float(static["attention_scaling"]), layer, G)
    return types.SimpleNamespace(K=K, V=V, q=q, qq=qq, st=st, T=T, N=N, Lmax=Lmax, B=B, C=C,
                                 static=static, npos=npos)


def state_np(lay) -> dict:
    d = lay.st.to_numpy()
    d["K"] = bf16_np(lay.K.reshape(-1, lay.Lmax, D))
    d["V"] = bf16_np(lay.V.reshape(-1, lay.Lmax, D))
    return d


def budget_for(rho: float, N: int):
    return budget(rho, ctx_len=N if N != 32768 else 32768)


def seq_state_np(st, K: torch.Tensor, V: torch.Tensor, b: int) -> dict:
    """Sequence b's slice of a batched LayerState (its HKV KV rows and HQ query-head rows) and
    of K, V (B, HKV, Lmax, D), as the numpy dict the CPU restatement's decode_step takes."""
    kv, qr = slice(b * HKV, (b + 1) * HKV), slice(b * HQ, (b + 1) * HQ)
    d = {}
    for f in st.FIELDS:
        t = getattr(st, f)[kv if f in ("codes", "U", "scale") else qr].detach()
        d[f] = bf16_np(t) if t.dtype == torch.bfloat16 else t.cpu().contiguous().numpy().copy()
    # the restatement indexes K, V, asg and codes with one row length: K, V at the state's Lmax
    L = st.Lmax
    for name, X in (("K", K), ("V", V)):
        x = bf16_np(X[b][:, :L])
        if x.shape[1] < L:
            x = np.concatenate([x, np.zeros((x.shape[0], L - x.shape[1], x.shape[2]), np.uint16)], 1)
        d[name] = x
    return d
