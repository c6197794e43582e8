"""The accuracy path's operator surface on the gfx950 kernels.

UTAMultiBinHIP.custom_attention mirrors UTAMultiBinAttention.custom_attention
(sparse_attention_hub/sparse_attention/uta_attention/multibin.py:2875-2970), the attention
function the reference registers with the HF model (adapters/huggingface.py:354-433):

  custom_attention(module, queries (B, H, Q, D), keys, values (B, Hkv, K, D), attention_mask,
                   scaling, dropout, sparse_meta_data=dict, layer_idx=int)
      -> (out (B, Q, H, D), None)

with the protocol of its selector and profile caches (static_top_k.py:242-255,
multibin.py:2098-2120):
  * `sparse_meta_data` missing -> ValueError; `layer_idx` missing -> ValueError;
  * a call with Q >= 8 rows is the request's question chunk: the layer's index is (re)built over
    all K keys, the question rows give the query moment, and the metric is rotated to position
    K (build_rows: QGS codes, QGC clusters, cluster sums);
  * a call with Q == 1 is a decode step at n = K: the index is extended with the keys appended
    since the last call, and the sparse step (QGS scan, top-k, ErrorGate, water-fill, top-q,
    residual proxies, fused softmax) gives the output;
  * a decode-sized call with no index for the layer -> ValueError, as the reference's profile
    cache raises.

Where this surface differs from the accuracy path, and why:
  * the question chunk's own rows get dense causal attention (the deployed path's prefill
    branch, graph_runner.py:472-475): this build implements the sparse estimator for the
    decode step only;
  * keys and values must be bfloat16 (the kernels read bf16 rows); Q between 2 and 7 and
    additive masks with nonzero entries are refused (the kernels decode one row per head and
    take no padding mask).
The index state lives in sparse_meta_data["oa_hip"][layer_idx] (one request's cache, as the
reference keeps its own caches in sparse_meta_data).
"""
from __future__ import annotations

import types

import torch

from openattention_amd import ops
from openattention_amd.budget import CTX_LEN
from openattention_amd.method import D, G, HKV, HQ, RMAX, OursHIP, prefill_attention
from openattention_amd.prefill import build_rows

QUESTION_ROWS = 8       # calls with at least this many query rows build the index


class UTAMultiBinHIP:
    """OpenAttention's estimator at read fraction rho, deployed split (C, E), on the gfx950
    kernels; `static` is the static query metric dict (M (L, HQ, D, D), inv_freq, attention_
    scaling).  `headroom` tokens can be decoded after each build before the layer's state is
    full (the reference rebuilds its profile past 4096 new keys, multibin.py:2103)."""

    def __init__(self, rho: float = 0.01, static: dict | None = None, ctx_len: int = CTX_LEN,
                 rule: str = "multibin", headroom: int = 4096, out_dtype=torch.bfloat16):
        if static is None:
            raise ValueError("UTAMultiBinHIP needs the static query metric (M, inv_freq, attention_scaling)")
        self.rho, self.static, self.ctx_len, self.rule = rho, static, ctx_len, rule
        self.headroom, self.out_dtype = headroom, out_dtype

    # ------------------------------------------------------------------ surface
    def custom_attention(self, module, queries: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                         attention_mask, scaling: float, dropout: float, **kwargs):
        if "sparse_meta_data" not in kwargs:
            raise ValueError("sparse_meta_data must be provided in kwargs")
        meta = kwargs.pop("sparse_meta_data")
        if meta is None:
            raise ValueError("sparse_meta_data cannot be None")
        layer_idx = kwargs.get("layer_idx")
        if layer_idx is None:
            raise ValueError("layer_idx must be provided in kwargs")
        B, H, Q, Dq = queries.shape
        if H != HQ or Dq != D or keys.shape[:2] != (B, HKV) or keys.shape[3] != D or values.shape != keys.shape:
            raise ValueError(f"expected queries (B, {HQ}, Q, {D}) and keys/values (B, {HKV}, K, {D})")
        if keys.dtype != torch.bfloat16 or values.dtype != torch.bfloat16 or queries.dtype != torch.bfloat16:
            raise ValueError("the HIP path reads bfloat16 queries, keys and values")
        if keys.device.type != "cuda":
            raise RuntimeError("the HIP path needs the tensors on a HIP device")
        if attention_mask is not None and bool((attention_mask[..., :keys.shape[2]] != 0).any()):
            raise NotImplementedError("additive masks with nonzero entries (padding) are not supported")
        cache = meta.setdefault("oa_hip", {})
        if Q >= QUESTION_ROWS:
            out = self._question_chunk(cache, int(layer_idx), queries, keys, values, scaling)
        elif Q == 1:
            out = self._decode(cache, int(layer_idx), queries, keys, values, scaling)
        else:
            raise ValueError(f"{Q} query rows: this path takes a question chunk (>= {QUESTION_ROWS} "
                             "rows) or one decode row per call")
        return out.transpose(1, 2).contiguous(), None

    # ------------------------------------------------------------------ phases
    @torch.no_grad()
    def _question_chunk(self, cache: dict, layer: int, queries, keys, values, scaling):
        B, _, Q, _ = queries.shape
        T = keys.shape[2]
        dev = keys.device
        ent = cache.get(layer)
        Lmax = T + self.headroom
        if ent is None or ent["m"].B != B or ent["m"].Lmax < Lmax:
            m = OursHIP(types.SimpleNamespace(rho=self.rho), B, Lmax, dev, n_layers=1, static=self.static,
                        ctx_len=self.ctx_len, rule=self.rule, out_dtype=self.out_dtype)
            ent = {"m": m, "n_dev": torch.zeros(1, device=dev, dtype=torch.int32)}
            cache[layer] = ent
        m = ent["m"]
        build_rows(m.st[0], keys.contiguous(), values.contiguous(), queries, T,
                   self.static["M"][layer], self.static["inv_freq"],
                   float(self.static.get("attention_scaling", 1.0)), layer, G)
        ent["n"] = T
        out = torch.empty_like(queries)
        for b in range(B):
            out[b:b + 1] = prefill_attention(queries[b:b + 1], keys[b:b + 1], values[b:b + 1], scaling)
        return out

    @torch.no_grad()
    def _decode(self, cache: dict, layer: int, queries, keys, values, scaling):
        ent = cache.get(layer)
        n = keys.shape[2]
        if ent is None:
            raise ValueError(f"a decode-sized call with no index for layer {layer}: the request's "
                             f"question chunk (>= {QUESTION_ROWS} rows) must come first")
        m = ent["m"]
        if queries.shape[0] != m.B:
            raise ValueError(f"batch {queries.shape[0]} differs from the build's {m.B}")
        if n <= ent["n"] or n > m.Lmax:
            raise ValueError(f"{n} keys after an index of {ent['n']} (capacity {m.Lmax}): rebuild with a "
                             "question chunk")
        K = keys.reshape(m.B * HKV, n, D)
        V = values.reshape(m.B * HKV, n, D)
        if not (K.is_contiguous() and V.is_contiguous()):
            K, V = K.contiguous(), V.contiguous()
        st = m.st[0]
        n_dev = ent["n_dev"]
        for pos in range(ent["n"], n - 1):      # keys appended without a decode call
            n_dev.fill_(pos + 1)
            ops.index_update(K, V, st, n_dev, RMAX)
        n_dev.fill_(n)
        m.sm_scale = float(scaling)
        out = m.step(st, K, V, queries, n_dev, n)
        ent["n"] = n
        return out.view(m.B, HQ, 1, D)
