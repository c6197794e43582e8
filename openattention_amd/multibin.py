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
  * a call with fewer rows extends the index with the keys appended since the last call
    (ops.index_update, the deployed step's index update);
  * every row then gets the estimator's output (multibin.py:2195-2747 with the masks of
    basic_fixed.py:180-214, 384-418 and static_top_k.py:221-262): row i sits at position
    K - Q + i and, under the causal mask, attends the n_i = K - Q + i + 1 keys before it --
    sink, the local window ending at the row, top-k of the QGS scores over the rest, ErrorGate
    and water-filling over its tail's clusters, within-cluster top-q, residual proxies and the
    fused softmax.  The sink / local / top-k sizes come from K, as the maskers size them from
    seq_len_keys (maskers/base.py:152-158).  A one-row call is the deployed decode step
    (OursHIP.step); a multi-row call runs its rows through OursHIP.rows_step;
  * when a masker would return the full mask (K <= local + Q or K <= top-k,
    basic_fixed.py:208-214, static_top_k.py:233-234) every row gets dense causal attention,
    as the reference returns get_true_attention_output (multibin.py:2916-2920): this library's
    dense decode kernel, one launch per row at n_i;
  * a decode-sized call with no index for the layer -> ValueError, as the reference's profile
    cache raises.

What the surface accepts, and why:
  * keys, values and queries in bfloat16 (the kernels read bf16 rows);
  * attention_mask None for a one-row call, or HF's additive causal mask (0 where a row may
    attend, <= -3e4 -- the dtype's minimum or -inf -- where it may not; any broadcastable
    (B|1, H|1, Q, >=K) layout).  A
    multi-row call needs the causal mask: without it the reference's rows would attend later
    keys as well.  Other masks (padding) raise NotImplementedError.
The index state lives in sparse_meta_data["oa_hip"][layer_idx] (one request's cache, as the
reference keeps its own caches in sparse_meta_data).
"""
from __future__ import annotations

import types

import torch

from openattention_amd import ops
from openattention_amd.budget import CTX_LEN
from openattention_amd.method import D, G, HKV, HQ, RMAX, OursHIP
from openattention_amd.prefill import build_rows

QUESTION_ROWS = 8       # calls with at least this many query rows build the index
MASKED = -3e4           # an additive mask entry at or below this removes the position: the
                        # estimator keeps raw = q.k * scale + mask > -1e4 (multibin.py:2213-2218)


def causal_mask_ok(attention_mask, Q: int, K: int) -> bool:
    """True when attention_mask[..., :K] is the additive causal mask of Q rows ending at K - 1
    (row i may attend j <= K - Q + i: entry 0; the rest <= MASKED, as HF's minimum of bf16, fp16
    or fp32 and -inf are), or None for one row."""
    if attention_mask is None:
        return Q == 1
    m = attention_mask[..., :K]
    if m.dim() < 2 or m.shape[-2] != Q or m.shape[-1] != K:
        return False
    i = torch.arange(Q, device=m.device).view(Q, 1)
    j = torch.arange(K, device=m.device).view(1, K)
    allowed = j <= (K - Q) + i
    mf = m.float()
    return bool(torch.where(allowed, mf == 0, mf <= MASKED).all())


class UTAMultiBinHIP:
    """OpenAttention's estimator at read fraction rho, deployed split (C, E), on the gfx950
    kernels; `static` is the static query metric dict (M (L, HQ, D, D), inv_freq, attention_
    scaling).  `headroom` tokens can be decoded after each build before the layer's state is
    full (the reference rebuilds its profile past 4096 new keys, multibin.py:2103).  record_rows,
    when set, keeps each row's (sel, quota, exp_idx) of the last call per layer in
    sparse_meta_data["oa_hip"][layer]["rows"] (inspection and tests)."""

    def __init__(self, rho: float = 0.01, static: dict | None = None, ctx_len: int = CTX_LEN,
                 rule: str = "multibin", headroom: int = 4096, out_dtype=torch.bfloat16,
                 record_rows: bool = False):
        if static is None:
            raise ValueError("UTAMultiBinHIP needs the static query metric (M, inv_freq, attention_scaling)")
        self.rho, self.static, self.ctx_len, self.rule = rho, static, ctx_len, rule
        self.headroom, self.out_dtype, self.record_rows = headroom, out_dtype, record_rows

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
        Kn = keys.shape[2]
        if Q < 1 or Q > Kn:
            raise ValueError(f"{Q} query rows over {Kn} keys")
        if not causal_mask_ok(attention_mask, Q, Kn):
            if attention_mask is None:
                raise NotImplementedError(f"a {Q}-row call needs the additive causal mask: without it the "
                                          "reference's rows would attend later keys too")
            raise NotImplementedError("only the additive causal mask (0 / <= -3e4) is supported, not padding")
        cache = meta.setdefault("oa_hip", {})
        layer = int(layer_idx)
        if Q >= QUESTION_ROWS:
            ent = self._build(cache, layer, queries, keys, values)
        else:
            ent = cache.get(layer)
            if ent is None:
                raise ValueError(f"a decode-sized call with no index for layer {layer}: the request's "
                                 f"question chunk (>= {QUESTION_ROWS} rows) must come first")
            if queries.shape[0] != ent["m"].B:
                raise ValueError(f"batch {queries.shape[0]} differs from the build's {ent['m'].B}")
            if Kn < ent["n"] or Kn > ent["m"].Lmax:
                raise ValueError(f"{Kn} keys after an index of {ent['n']} (capacity {ent['m'].Lmax}): "
                                 "rebuild with a question chunk")
        out = self._rows(ent, queries, keys, values, scaling)
        return out.transpose(1, 2).contiguous(), None

    # ------------------------------------------------------------------ phases
    @torch.no_grad()
    def _build(self, cache: dict, layer: int, queries, keys, values) -> dict:
        B = queries.shape[0]
        T = keys.shape[2]
        dev = keys.device
        ent = cache.get(layer)
        Lmax = T + self.headroom
        if ent is None or ent["m"].B != B or ent["m"].Lmax < Lmax:
            m = OursHIP(types.SimpleNamespace(rho=self.rho), B, Lmax, dev, n_layers=1, static=self.static,
                        ctx_len=self.ctx_len, rule=self.rule, out_dtype=self.out_dtype)
            ent = {"m": m, "n_dev": torch.zeros(1, device=dev, dtype=torch.int32)}
            cache[layer] = ent
        build_rows(ent["m"].st[0], keys.contiguous(), values.contiguous(), queries, T,
                   self.static["M"][layer], self.static["inv_freq"],
                   float(self.static.get("attention_scaling", 1.0)), layer, G)
        ent["n"] = T
        return ent

    @torch.no_grad()
    def _rows(self, ent: dict, queries, keys, values, scaling) -> torch.Tensor:
        """Every query row's output (B, HQ, Q, D) over the layer's index (see the module text)."""
        m = ent["m"]
        B, _, Q, _ = queries.shape
        n = keys.shape[2]
        K = keys.reshape(B * HKV, n, D)
        V = values.reshape(B * HKV, n, D)
        if not (K.is_contiguous() and V.is_contiguous()):
            K, V = K.contiguous(), V.contiguous()
        st = m.st[0]
        n_dev = ent["n_dev"]
        m.sm_scale = float(scaling)
        ns, nl, k_top = m.bud.counts(n)
        full = n <= nl + Q or n <= k_top
        step_row = Q == 1 and not full and n > ent["n"]
        # keys appended since the last call join the index (the deployed decode step adds the
        # last one itself)
        for pos in range(ent["n"], n - 1 if step_row else n):
            n_dev.fill_(pos + 1)
            ops.index_update(K, V, st, n_dev, RMAX)
        ent["n"] = n
        record = [] if self.record_rows else None
        if full:
            out = torch.empty(B, HQ, Q, D, device=queries.device, dtype=m.out.dtype)
            q = queries.to(torch.bfloat16)
            for i in range(Q):
                n_dev.fill_(n - Q + i + 1)
                o = ops.dense_decode(q[:, :, i].reshape(B * HQ, D).contiguous(), K, V, n_dev,
                                     sm_scale=float(scaling))
                out[:, :, i] = o.view(B, HQ, D)
            n_dev.fill_(n)
        elif step_row:
            n_dev.fill_(n)
            out = m.step(st, K, V, queries, n_dev, n).view(B, HQ, 1, D).clone()
            if record is not None:
                record.append((0, m.last_sel.clone(), m.quota.clone(), m.exp_idx.clone()))
        else:
            out = torch.empty(B, HQ, Q, D, device=queries.device, dtype=m.out.dtype)
            m.rows_step(st, K, V, queries, n_dev, n, out, record=record)
        if record is not None:
            ent["rows"] = sorted(record, key=lambda t: t[0])
        return out
