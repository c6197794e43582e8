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

`prefill` runs a prompt through the model one batch row at a time, as the reference's runner
does (graph_runner.py:615-622): every layer's attention goes through the hook's prefill branch
(method.attn_hook: K, V into the cache, dense causal attention, the method's index build with the
prompt's last `qlen` query rows as the question chunk).  `probe(layers)` makes each decode step
copy the attention's inputs and decisions of those layers into per-layer buffers (inside a
captured graph too): the query rows, sel, quota, exp_idx and the attention output.
"""
from __future__ import annotations

import torch

import types

from openattention_amd import ops
from openattention_amd.method import C as CTX, Method, attn_hook
from openattention_amd.synth import llama31_inv_freq

HID, NLAYER, HQ, HKV, D, FFN, VOCAB = 4096, 32, 32, 8, 128, 14336, 128256
EPS = 1e-5


def rmsnorm(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + EPS)).to(x.dtype) * w


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x (N, H, D) at one position per row n; cos, sin (N, 1, D) (or (1, 1, D) for one shared
    position)."""
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
        self.mods = [types.SimpleNamespace(layer_idx=l) for l in range(layers)]
        self.probes = {}

    def params(self) -> int:
        per = HID * (HQ + 2 * HKV) * D + HQ * D * HID + HID * 2 * FFN + FFN * HID + 2 * HID
        return self.L * per + 2 * VOCAB * HID + HID

    def probe(self, layers) -> dict:
        """Per-layer probe buffers that every later decode step fills (inside a captured graph
        too): q (B*HQ, D) bf16, and with a sparse method sel, quota, exp_idx and the attention
        output out (B*HQ, D) in the method's output dtype.  Returns {layer: {name: tensor}}."""
        R = self.B * HQ
        self.probes = {}
        for l in layers:
            p = {"q": torch.empty(R, D, device=self.dev, dtype=torch.bfloat16)}
            if self.method is not None:
                m = self.method
                p["quota"] = torch.empty_like(m.quota)
                p["exp_idx"] = torch.empty_like(m.exp_idx)
                p["out"] = torch.empty_like(m.out)
                p["sel"] = None          # sized at the first step (the sel width follows n)
            self.probes[l] = p
        return self.probes

    @torch.no_grad()
    def prefill(self, tokens: torch.Tensor, qlen: int = 64) -> torch.Tensor:
        """Prompt prefill of every batch row (tokens (B, T) int64), one row at a time through all
        layers (graph_runner.py:615-622).  Each layer's attention is attn_hook's prefill branch:
        the row's K, V are written to C.K[l][b, :, :T], its causal attention is dense and the
        method builds the row's index (C.qlen[b] = qlen question rows).  Leaves C.phase at
        "decode" and the greedy next token of every row in self.tok; returns it."""
        B, T = tokens.shape
        if B != self.B or T > self.Lmax:
            raise ValueError(f"tokens must be ({self.B}, <= {self.Lmax})")
        CTX.phase = "prefill"
        CTX.qlen = [qlen] * B
        CTX.method = self.method if self.method is not None else Method(None, B, self.Lmax, self.dev)
        cos, sin = self.cos[:T].unsqueeze(1), self.sin[:T].unsqueeze(1)           # (T, 1, D)
        for b in range(B):
            CTX.brow = b
            x = self.embed.index_select(0, tokens[b])                              # (T, HID)
            for l in range(self.L):
                h = rmsnorm(x, self.ln1[l])
                qkv = h @ self.wqkv[l]
                q = rope(qkv[:, :HQ * D].view(T, HQ, D), cos, sin).transpose(0, 1).unsqueeze(0)
                k = rope(qkv[:, HQ * D:(HQ + HKV) * D].view(T, HKV, D), cos, sin).transpose(0, 1).unsqueeze(0)
                v = qkv[:, (HQ + HKV) * D:].view(T, HKV, D).transpose(0, 1).unsqueeze(0)
                del qkv
                o, _ = attn_hook(self.mods[l], q, k, v, None)                       # (1, T, HQ, D)
                x = x + o.reshape(T, HQ * D) @ self.wo[l]
                del q, k, v, o
                h = rmsnorm(x, self.ln2[l])
                gu = h @ self.w13[l]
                x = x + (torch.nn.functional.silu(gu[:, :FFN]) * gu[:, FFN:]) @ self.w2[l]
                del gu
            logits = rmsnorm(x[-1:], self.lnf) @ self.lm_head
            self.tok[b] = logits.argmax(-1)[0]
        CTX.phase = "decode"
        return self.tok

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
            p = self.probes.get(l)
            if p is not None:
                p["q"].copy_(q.reshape(B * HQ, D))
            if self.method is not None:
                o = self.method.decode(l, q.reshape(B, HQ, 1, D), n)
                if p is not None:
                    m = self.method
                    if p["sel"] is None or p["sel"].shape != m.last_sel.shape:
                        p["sel"] = torch.empty_like(m.last_sel)
                    p["sel"].copy_(m.last_sel)
                    p["quota"].copy_(m.quota)
                    p["exp_idx"].copy_(m.exp_idx)
                    p["out"].copy_(o.reshape(B * HQ, D))
                o = o.reshape(B, HQ * D).to(x.dtype)
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
