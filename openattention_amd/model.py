"""A Llama-3.1-8B-shaped decoder with random-init bf16 weights, for timing a whole decode step
with the sparse attention stage against dense decode attention.

Shapes follow Llama-3.1-8B (32 layers, hidden 4096, 32 query / 8 KV heads of 128, SwiGLU FFN
14336, vocabulary 128256, RMSNorm eps 1e-5, RoPE theta 500000 with the Llama-3 frequency
scaling).  The attention of each layer is the reference's decode hook contract
(methods_eager.py:198-224, graph_runner.py:469-482): the new K/V row is written at position
n - 1 of the cache C.K[l], C.V[l] before the attention runs, and n lives on the device
(C.n_dev), so a whole step -- embedding, 32 layers, final norm, LM head and the greedy next
token -- is captured once in a hipGraph and replayed with n advancing on the device.

With `method` an OursHIP the attention is its decode (the gfx950 sparse stage); with
method = None it is the dense split-K decode kernel over [0, n) on the same cache.
"""
from __future__ import annotations

import torch

from openattention_amd import ops
from openattention_amd.method import C as CTX
from openattention_amd.synth import llama31_inv_freq

HID, NLAYER, HQ, HKV, D, FFN, VOCAB = 4096, 32, 32, 8, 128, 14336, 128256
EPS = 1e-5


def rmsnorm(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + EPS)).to(x.dtype) * w


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x (B, H, D) at one position per row; cos, sin (B, 1, D)."""
    h = D // 2
    xf = x.float()
    rot = torch.cat([-xf[..., h:], xf[..., :h]], -1)
    return (xf * cos + rot * sin).to(x.dtype)


class LlamaShaped:
    def __init__(self, B: int, Lmax: int, dev, layers: int = NLAYER, seed: int = 0, method=None):
        """method: an OursHIP over these layers (sparse attention) or None (dense attention).
        The KV cache is C.K / C.V (set by the caller), (B, 8, Lmax, 128) bf16 per layer."""
        self.B, self.Lmax, self.dev, self.L = B, Lmax, dev, layers
        self.method = method
        g = torch.Generator(device=dev).manual_seed(seed)

        def w(*shape):
            return torch.randn(*shape, generator=g, device=dev, dtype=torch.bfloat16) * 0.02

        bf = dict(device=dev, dtype=torch.bfloat16)
        self.embed = w(VOCAB, HID)
        self.wqkv = [w(HID, (HQ + 2 * HKV) * D) for _ in range(layers)]
        self.wo = [w(HQ * D, HID) for _ in range(layers)]
        self.w13 = [w(HID, 2 * FFN) for _ in range(layers)]
        self.w2 = [w(FFN, HID) for _ in range(layers)]
        self.ln1 = [torch.ones(HID, **bf) for _ in range(layers)]
        self.ln2 = [torch.ones(HID, **bf) for _ in range(layers)]
        self.lnf = torch.ones(HID, **bf)
        self.lm_head = w(HID, VOCAB)
        inv = llama31_inv_freq().to(dev)
        t = torch.arange(Lmax, device=dev, dtype=torch.float32)
        fr = torch.outer(t, inv)
        emb = torch.cat([fr, fr], -1)
        self.cos, self.sin = emb.cos(), emb.sin()                       # (Lmax, D) fp32
        self.tok = torch.zeros(B, device=dev, dtype=torch.long)         # token at position n - 1
        self.ws = None

    def params(self) -> int:
        per = HID * (HQ + 2 * HKV) * D + HQ * D * HID + HID * 2 * FFN + FFN * HID + 2 * HID
        return self.L * per + 2 * VOCAB * HID + HID

    @torch.no_grad()
    def step(self, n: int) -> torch.Tensor:
        """One decode step: the token in self.tok sits at position n - 1 (n = C.n_dev on the
        device; the host n only fixes the sparse stage's sink/local/top-k counts).  Writes the
        greedy next token into self.tok and returns it."""
        B = self.B
        pos = (CTX.n_dev - 1).long()                                    # (1,) on the device
        cos = self.cos.index_select(0, pos).unsqueeze(0)                # (1, 1, D)
        sin = self.sin.index_select(0, pos).unsqueeze(0)
        x = self.embed.index_select(0, self.tok)                        # (B, HID)
        for l in range(self.L):
            h = rmsnorm(x, self.ln1[l])
            qkv = h @ self.wqkv[l]
            q = rope(qkv[:, :HQ * D].view(B, HQ, D), cos, sin)
            k = rope(qkv[:, HQ * D:(HQ + HKV) * D].view(B, HKV, D), cos, sin)
            v = qkv[:, (HQ + HKV) * D:].view(B, HKV, D)
            CTX.K[l].index_copy_(2, pos, k.unsqueeze(2))
            CTX.V[l].index_copy_(2, pos, v.unsqueeze(2))
            if self.method is not None:
                o = self.method.decode(l, q.reshape(B, HQ, 1, D), n).reshape(B, HQ * D)
            else:
                R = B * HQ
                need = R * ops.DENSE_SPLITS * (D + 2)
                if self.ws is None or self.ws.numel() < need:
                    self.ws = torch.empty(need, device=self.dev, dtype=torch.float32)
                o = ops.dense_decode(q.reshape(R, D).contiguous(), CTX.K[l].view(-1, self.Lmax, D),
                                     CTX.V[l].view(-1, self.Lmax, D), CTX.n_dev, ws=self.ws).reshape(B, HQ * D)
            x = x + o @ self.wo[l]
            h = rmsnorm(x, self.ln2[l])
            gu = h @ self.w13[l]
            x = x + (torch.nn.functional.silu(gu[:, :FFN]) * gu[:, FFN:]) @ self.w2[l]
        logits = rmsnorm(x, self.lnf) @ self.lm_head
        self.tok.copy_(logits.argmax(-1))
        return self.tok
