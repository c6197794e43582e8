"""Seeded synthetic inputs of the benchmark configurations (Llama-3.1-8B attention shapes).

Per (sequence b, KV head h) of configuration `cfg`, one generator seeded 1000*cfg + 97*b + h
(+ 7919*layer for multi-layer runs) draws
  keys    : a Gaussian mixture -- `n_centers` centres ~ N(0, I_128), uniform component
            assignment, within-component std 0.3
  values  : N(0, I)
  queries : per query head of the group, a uniformly chosen key of its KV head + N(0, 0.2^2 I)
  question: `n_question` more queries drawn the same way (the rows the QGS/QGC metric and the
            reference's question-chunk build consume)
Config 4 plants `needles` keys per KV head with cosine 0.9 to one of the group's queries.

The static query metric M_st (the reference ships it as assets/...query_metric.triu.pt) is
synthesised per (layer, query head) as E[q q^T] over 4096 calibration queries drawn from an
independent mixture of the same family; inv_freq follows the Llama-3.1 RoPE formula
(base 500000, llama3 scaling factor 8, low/high frequency factors 1/4, original context 8192);
attention_scaling = 1.
"""
from __future__ import annotations

import math

import torch

HQ, HKV, D = 32, 8, 128
G = HQ // HKV


def llama31_inv_freq(dim: int = D, base: float = 500000.0, factor: float = 8.0,
                     low_freq_factor: float = 1.0, high_freq_factor: float = 4.0,
                     old_context_len: int = 8192) -> torch.Tensor:
    inv = 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.float64) / dim))
    low_wavelen = old_context_len / low_freq_factor
    high_wavelen = old_context_len / high_freq_factor
    out = []
    for f in inv.tolist():
        wavelen = 2 * math.pi / f
        if wavelen < high_wavelen:
            out.append(f)
        elif wavelen > low_wavelen:
            out.append(f / factor)
        else:
            smooth = (old_context_len / wavelen - low_freq_factor) / (high_freq_factor - low_freq_factor)
            out.append((1 - smooth) * f / factor + smooth * f)
    return torch.tensor(out, dtype=torch.float32)


def seed_of(cfg: int, b: int, h: int, layer: int = 0) -> int:
    return 1000 * cfg + 97 * b + h + 7919 * layer


def _gen(dev, seed: int) -> torch.Generator:
    g = torch.Generator(device=dev)
    g.manual_seed(int(seed))
    return g


def make_layer(cfg: int, B: int, N: int, Lmax: int, n_centers: int, dev, layer: int = 0,
               n_question: int = 64, dtype=torch.bfloat16, needles: int = 0,
               needle_cos: float = 0.9):
    """Keys/values (B, HKV, Lmax, D) (positions >= N are zero), decode queries (B, HQ, 1, D)
    and question rows (B, HQ, n_question, D).  Needle positions (B, HKV, needles) when planted."""
    K = torch.zeros(B, HKV, Lmax, D, device=dev, dtype=dtype)
    V = torch.zeros(B, HKV, Lmax, D, device=dev, dtype=dtype)
    q = torch.empty(B, HQ, 1, D, device=dev, dtype=dtype)
    qq = torch.empty(B, HQ, n_question, D, device=dev, dtype=dtype)
    npos = torch.full((B, HKV, max(needles, 1)), -1, dtype=torch.long)
    for b in range(B):
        for h in range(HKV):
            g = _gen(dev, seed_of(cfg, b, h, layer))
            centers = torch.randn(n_centers, D, device=dev, generator=g)
            comp = torch.randint(0, n_centers, (N,), device=dev, generator=g)
            k = centers[comp] + 0.3 * torch.randn(N, D, device=dev, generator=g)
            v = torch.randn(N, D, device=dev, generator=g)
            pick = torch.randint(0, N, (G, 1 + n_question), device=dev, generator=g)
            noise = 0.2 * torch.randn(G, 1 + n_question, D, device=dev, generator=g)
            qs = k[pick] + noise
            if needles > 0:
                # plant needle keys with cosine `needle_cos` to the group's decode queries
                pos = torch.randperm(N - 64, device=dev, generator=g)[:needles] + 32
                for j in range(needles):
                    qd = qs[j % G, 0]
                    u = qd / qd.norm()
                    r = torch.randn(D, device=dev, generator=g)
                    r = r - (r @ u) * u
                    r = r / r.norm()
                    nk = (needle_cos * u + math.sqrt(1 - needle_cos ** 2) * r) * k.norm(dim=-1).mean()
                    k[pos[j]] = nk
                npos[b, h, :needles] = pos.cpu()
            K[b, h, :N] = k.to(dtype)
            V[b, h, :N] = v.to(dtype)
            q[b, h * G:(h + 1) * G, 0] = qs[:, 0].to(dtype)
            qq[b, h * G:(h + 1) * G] = qs[:, 1:].to(dtype)
    return K, V, q, qq, npos


def static_metric(n_layers: int, seed: int = 4242, n_calib: int = 4096, n_centers: int = 256,
                  dev="cpu") -> dict:
    """Synthetic M_st (L, HQ, D, D) fp32, pre-RoPE, plus inv_freq and attention_scaling."""
    M = torch.empty(n_layers, HQ, D, D, dtype=torch.float32)
    for l in range(n_layers):
        for h in range(HQ):
            g = _gen("cpu", seed + 131 * l + h)
            centers = torch.randn(n_centers, D, generator=g)
            comp = torch.randint(0, n_centers, (n_calib,), generator=g)
            x = centers[comp] + 0.3 * torch.randn(n_calib, D, generator=g)
            x = x + 0.2 * torch.randn(n_calib, D, generator=g)
            M[l, h] = (x.T @ x) / n_calib
    return dict(M=M.to(dev), inv_freq=llama31_inv_freq().to(dev), attention_scaling=1.0)
