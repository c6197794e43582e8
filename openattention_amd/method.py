"""Method surface of the deployed decode step, backed by the gfx950 kernels.

Mirrors inference/methods_eager.py:176-265 (Ctx, attn_hook, Method) and the deployed method
OursG3/OursG2 (inference/ours_fastbuild.py:143-304, inference/ours_graph.py:265-347):
  OursHIP(a, B, Lmax, dev).build(l, b, q, T)   prefill index build of layer l, batch row b
  OursHIP(...).decode(l, q, n) -> (B, HQ, 1, D)  one decode step of layer l; the new K,V is
                                                already at position n-1; n is also in C.n_dev
Every buffer of the step is preallocated (per layer for the index, shared for the step's
work buffers), nothing is read back on the host, and n / n0 are read on the device, so one
decode step can be captured in a hipGraph (torch.cuda.CUDAGraph) and replayed.  The host
only computes (ns, nl, k_top) from n, which the reference also keys its graphs by
(eval_accuracy.py:64-66).
"""
from __future__ import annotations

import types

import torch
import torch.nn.functional as TF

from openattention_amd import ops
from openattention_amd.budget import CTX_LEN, budget
from openattention_amd.prefill import LayerState, build_row, build_rows

HQ, HKV, D, NL = 32, 8, 128, 32
G = HQ // HKV
SC = D ** -0.5
RMAX = 256
SCAN_TILE = 64
TOPQ_SEGMENT = 36 * 1024   # positions the top-q kernel holds in registers at once (36 per thread)


class Ctx:
    """Run state shared by the attention hook and the method (methods_eager.py:176-189)."""
    phase = "prefill"
    brow = 0
    n = 0
    K = None            # per layer (B, HKV, Lmax, D)
    V = None
    qlen = []           # question-chunk length per batch row
    method = None
    n_dev = None        # int32 (1,) device scalar: current length
    n0_dev = None       # int32 (1,) device scalar: prefix length at the build
    kv_idx = None       # int64 (1,) device index of the write position (n-1)


C = Ctx()


def prefill_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scale: float,
                      block: int = 512) -> torch.Tensor:
    """Dense causal attention of the prefill rows of one sequence, as the deployed hook's prefill
    branch computes it (graph_runner.py:472-475): query (1, HQ, Q, D) at positions K - Q .. K - 1
    of key, value (1, HKV, K, D); returns (1, HQ, Q, D) in query's dtype.  GQA groups are
    expanded.  When Q == K the fused flash / memory-efficient kernels run on the cache's dtype;
    otherwise (or where those kernels are unavailable) blocks of query rows run in fp32, so the
    score matrix never exceeds (HQ, block, K)."""
    Gq = query.shape[1] // key.shape[1]
    Q, K = query.shape[2], key.shape[2]
    if Q == K:
        from torch.nn.attention import SDPBackend, sdpa_kernel
        try:
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                return TF.scaled_dot_product_attention(query, key.repeat_interleave(Gq, 1),
                                                       value.repeat_interleave(Gq, 1), is_causal=True,
                                                       scale=scale)
        except RuntimeError:
            pass
    out = torch.empty_like(query)
    kf = key[0].float()                                                  # (HKV, K, D)
    vf = value[0].float()
    pos = torch.arange(K, device=key.device)
    for r0 in range(0, Q, block):
        r1 = min(Q, r0 + block)
        qf = query[0, :, r0:r1].float().reshape(key.shape[1], Gq * (r1 - r0), -1)   # (HKV, G*b, D)
        sc = torch.matmul(qf, kf.transpose(1, 2).contiguous()) * scale              # (HKV, G*b, K)
        last = (K - Q + torch.arange(r0, r1, device=key.device)).repeat(Gq)          # (G*b,)
        sc.masked_fill_(pos[None, :] > last[:, None], float("-inf"))
        o = torch.matmul(torch.softmax(sc, -1), vf)                                 # (HKV, G*b, D)
        out[0, :, r0:r1] = o.reshape(query.shape[1], r1 - r0, -1).to(query.dtype)
    return out


def attn_hook(module, query, key, value, attention_mask, dropout=0.0, scaling=None, is_causal=None, **kw):
    """Attention-function hook with device-side positions (graph_runner.py:469-482).  Prefill:
    the batch row C.brow's K, V go into the cache, its causal attention is computed densely and
    the method builds the row's index.  Decode: the new K, V go to C.kv_idx (= n - 1, on the
    device) and the method's sparse step runs.  Returns (out (B, T, HQ, D), None)."""
    l = module.layer_idx
    T = query.shape[2]
    if C.phase == "prefill":
        b = C.brow
        C.K[l][b:b + 1, :, :T] = key
        C.V[l][b:b + 1, :, :T] = value
        out = prefill_attention(query, key, value, SC if scaling is None else scaling)
        C.method.build(l, b, query, T)
        return out.transpose(1, 2).contiguous(), None
    C.K[l].index_copy_(2, C.kv_idx, key)
    C.V[l].index_copy_(2, C.kv_idx, value)
    out = C.method.decode(l, query, C.n)
    return out.transpose(1, 2).contiguous(), None


class Method:
    name = "base"

    def __init__(self, a, B, Lmax, dev):
        self.a, self.B, self.Lmax, self.dev = a, B, Lmax, dev
        self.R = B * HQ

    def build(self, l, b, q, T):
        pass


class OursHIP(Method):
    """The deployed OpenAttention decode step (QGS scan + top-k, ErrorGate, water-filling,
    within-cluster top-q, residual proxies, fused softmax) on the gfx950 kernels."""
    name = "ours_hip"

    def __init__(self, a, B, Lmax, dev, n_layers: int = NL, static: dict | None = None,
                 ctx_len: int = CTX_LEN, rule: str = "multibin", fused: bool = True,
                 groups: int = 1, c_max: int = 256, out_dtype: torch.dtype = torch.bfloat16,
                 gate_mode: str = "fused"):
        super().__init__(a, B, Lmax, dev)
        # how the top-k, ErrorGate and water-fill are launched (the results are the same):
        #   "fused": one launch after the scan (each row's top-k beside its pooled ErrorGate, then
        #            the selected tokens' correction and the fill);
        #   "split": the pooled ErrorGate in the scan's launch, then top-k + correction + fill;
        #   "separate": top-k, then ErrorGate and fill
        if gate_mode not in ("fused", "split", "separate"):
            raise ValueError(f"gate_mode must be 'fused', 'split' or 'separate', got {gate_mode!r}")
        self.gate_mode = gate_mode
        if out_dtype not in (torch.bfloat16, torch.float32):
            raise ValueError("out_dtype must be torch.bfloat16 or torch.float32")
        if groups < 1 or B % groups:
            raise ValueError(f"groups={groups} must divide B={B}")
        # the batch is split into `groups` sets of whole sequences whose stage chains run on
        # their own streams (rows are independent): one group's latency-bound stages overlap
        # another group's bandwidth-bound scan
        self.groups = groups
        self.streams = [torch.cuda.Stream(device=dev) for _ in range(groups)] if groups > 1 else []
        self.bud = budget(a.rho, ctx_len=ctx_len, rule=rule, c_max=c_max)
        self.Cn, self.E = self.bud.C, self.bud.E
        self.n_layers = n_layers
        self.fused = fused
        self.sm_scale = SC
        self.static = static
        self.st = [LayerState(B, HKV, G, Lmax, self.Cn, RMAX, dev) for _ in range(n_layers)]
        R, BH = self.R, B * HKV
        self.ntiles = -(-Lmax // SCAN_TILE)
        self.SW = self.ntiles * SCAN_TILE
        f32 = dict(device=dev, dtype=torch.float32)
        i32 = dict(device=dev, dtype=torch.int32)
        self.limbs = torch.zeros(BH, 16, 32, device=dev, dtype=torch.int8)
        self.fexp = torch.zeros(R, **i32)
        # 16-bit key heads of the scores (what the scan writes and top-k / top-q read); S holds
        # exact fp32 scores only for rows top-q leaves to its key-prefix kernel
        self.H = torch.empty(R, self.SW, device=dev, dtype=torch.int16)
        self.S = torch.empty(R, self.SW, **f32)
        self.TM = torch.empty(R, self.ntiles, **f32)
        # tile minima of the scores, the row range top-q bins with, for rows of several top-q
        # register segments (longer than 36864): there they spare a pass over the row
        self.TMn = torch.empty(R, self.ntiles, **f32) if Lmax > TOPQ_SEGMENT else None
        self.TMt = self.TM if self.TMn is not None else None
        self.score = torch.empty(R, self.Cn, **f32)
        self.n_t = torch.empty(R, self.Cn, **f32)
        self.quota = torch.empty(R, self.Cn, **f32)
        self.qsk = torch.empty(R, self.Cn, **f32)      # q . Sk_c, from the gate to the residual
        self.exp_idx = torch.empty(R, max(self.E, 1), **i32)
        # the step's output rows: bf16 as the reference's, or the fp32 accumulators unrounded
        self.out = torch.empty(R, D, device=dev, dtype=out_dtype)
        self._sel = {}
        self._pending = {}          # layer -> {batch row: (question rows, T, K, V)} awaiting build
        self.build_events = None    # a list: (start, end) events around every layer's build
        if not fused:
            self.kbar_r = torch.empty(R, self.Cn, D, device=dev, dtype=torch.bfloat16)
            self.vbar_r = torch.empty(R, self.Cn, D, device=dev, dtype=torch.bfloat16)
            self.log_n = torch.empty(R, self.Cn, **f32)

    # ---------------------------------------------------------------- prefill
    def build(self, l, b, q, T):
        """Index build of layer l, batch row b after K,V of the prefix are in C.K[l][b, :, :T].
        q: (1, HQ, Tq, D) prefill queries; the last C.qlen[b] rows are the question chunk.

        The rows of a layer are collected and built together (prefill.build_rows: one batched
        eigh and one launch per stage for all of them) once the layer's last batch row arrives;
        the state is the one build_row gives row by row.  A decode step first builds any row
        still waiting (flush_builds), so the order of calls stays free."""
        if self.static is None:
            raise RuntimeError("OursHIP needs the static query metric (dict with M, inv_freq, "
                               "attention_scaling)")
        Qn = C.qlen[b]
        qrows = q[0, :, q.shape[2] - Qn:, :].clone()
        pend = self._pending.setdefault(l, {})
        pend[b] = (qrows, T, C.K[l], C.V[l])
        if len(pend) == self.B:
            self._build_layer(l)

    def _build_layer(self, l):
        pend = self._pending.pop(l, {})
        if not pend:
            return
        if self.build_events is not None:
            e0 = torch.cuda.Event(enable_timing=True)
            e0.record()
        self._build_rows_of(l, pend)
        if self.build_events is not None:
            e1 = torch.cuda.Event(enable_timing=True)
            e1.record()
            self.build_events.append((e0, e1))

    def _build_rows_of(self, l, pend):
        scal = float(self.static.get("attention_scaling", 1.0))
        M, inv = self.static["M"][l], self.static["inv_freq"]
        rows = sorted(pend)
        Ts = {pend[b][1] for b in rows}
        Qs = {pend[b][0].shape[1] for b in rows}
        K, V = pend[rows[0]][2], pend[rows[0]][3]
        if (rows == list(range(self.B)) and len(Ts) == 1 and len(Qs) == 1 and K.is_contiguous()
                and V.is_contiguous() and all(pend[b][2] is K and pend[b][3] is V for b in rows)):
            build_rows(self.st[l], K, V, torch.stack([pend[b][0] for b in rows]), Ts.pop(), M, inv, scal, l, G)
        else:
            for b in rows:
                qrows, T, Kc, Vc = pend[b]
                build_row(self.st[l], b, Kc[b], Vc[b], qrows, T, M, inv, scal, l, G)

    def flush_builds(self):
        """Build every row whose build() call is still waiting for the rest of its layer."""
        for l in list(self._pending):
            self._build_layer(l)

    # ---------------------------------------------------------------- decode
    def sel_buffer(self, NS: int) -> torch.Tensor:
        if NS not in self._sel:
            self._sel[NS] = torch.empty(self.R, NS, device=self.dev, dtype=torch.int32)
        return self._sel[NS]

    def decode(self, l, q, n, marks: list | None = None):
        """One decode step of layer l over the cache C.K[l], C.V[l] (the new K, V already at
        n - 1; n also in C.n_dev).  `marks`, when given, receives (stage, event) pairs recorded
        on the current stream after each stage (per-stage timing)."""
        if self._pending:
            self.flush_builds()
        return self.step(self.st[l], C.K[l].view(-1, self.Lmax, D), C.V[l].view(-1, self.Lmax, D), q,
                         C.n_dev, n, marks)

    def decode_stages(self, l, q, n) -> list:
        """The stages of decode(l, q, n) as (name, call) pairs in launch order: each call
        launches that stage alone on the current stream (its inputs are the previous stages'
        outputs in the method's work buffers)."""
        return self.stages(self.st[l], C.K[l].view(-1, self.Lmax, D), C.V[l].view(-1, self.Lmax, D), q,
                           C.n_dev, n)[0]

    def stages(self, st, K, V, q, n_dev, n, counts: tuple | None = None, update_index: bool = True):
        """The decode stages over an explicit index state and K, V (B * HKV, >= n, D) bf16 rows
        (any row stride), as (name, call) pairs in launch order, and the step's sel buffer.
        n on the host fixes the sink / local / top-k counts unless `counts` = (ns, nl, k_top)
        gives them; n_dev holds n on the device.  update_index: the first stage adds the token
        at n - 1 to the index (the decode step); otherwise it only projects the queries (a row
        of a multi-row call over an index that already holds its keys)."""
        qr = q.reshape(self.R, D)
        if not qr.is_contiguous():
            qr = qr.contiguous()
        if not 1 <= n <= self.Lmax:
            raise ValueError(f"n={n} outside [1, Lmax={self.Lmax}]: the step writes position n-1")
        if K.shape[0] != self.B * HKV or K.shape[1] < n or V.shape != K.shape:
            raise ValueError(f"K, V must be ({self.B * HKV}, >= n={n}, {D}) with equal shapes")
        ns, nl, k_top = self.bud.counts(n) if counts is None else counts
        if n - ns - nl < k_top:
            raise ValueError(f"n={n} too small for sink {ns} + local {nl} + top-k {k_top}")
        NS = ns + nl + k_top
        sel = self.sel_buffer(NS)
        sc = self.sm_scale
        out = []
        if update_index:
            out.append(("index_prep", lambda: ops.index_prep(K, V, st, n_dev, RMAX, qr, self.limbs, self.fexp)))
        else:
            out.append(("qgs_prep", lambda: ops.qgs_prep(qr, st.U, st.scale, self.limbs, self.fexp)))
        if self.gate_mode == "split":
            # the pooled ErrorGate with the scan, the selected tokens' correction with the top-k
            # and the fill
            out.append(("qgs_scan_gate", lambda: ops.qgs_scan_gate(
                st.codes, self.limbs, self.fexp, self.H, self.TM, n_dev, ns, nl, qr, st.Sk, st.Sk2, st.nb,
                self.score, self.n_t, sc, qsk=self.qsk, TMn=self.TMn)))
            out.append(("topk_fix_fill", lambda: ops.topk_fix_fill(
                self.H, self.TM, n_dev, ns, nl, k_top, st.codes, self.limbs, self.fexp, qr, K, st.asg, sel,
                st.Sk, st.Sk2, st.nb, self.score, self.n_t, self.quota, sc, self.E)))
        else:
            out.append(("qgs_scan", lambda: ops.qgs_scan_heads(st.codes, self.limbs, self.fexp, self.H, self.TM,
                                                               n_dev, ns, nl, TMn=self.TMn)))
            if self.gate_mode == "fused":
                # each row's top-k beside its pooled ErrorGate, then the correction and the fill
                out.append(("topk_gate_fill", lambda: ops.topk_gate_fill(
                    self.H, self.TM, n_dev, ns, nl, k_top, st.codes, self.limbs, self.fexp, qr, K, st.asg,
                    sel, st.Sk, st.Sk2, st.nb, self.score, self.n_t, self.quota, sc, self.E, qsk=self.qsk)))
            else:
                out.append(("topk_select", lambda: ops.topk_select_heads(
                    self.H, self.TM, sel, n_dev, ns, nl, k_top, st.codes, self.limbs, self.fexp)))
                out.append(("gate_fill", lambda: ops.gate_fill(
                    qr, K, st.asg, sel, st.Sk, st.Sk2, st.nb, self.score, self.n_t, self.quota, sc, self.E,
                    qsk=self.qsk)))
        out.append(("topq", lambda: ops.topq_heads(self.H, st.asg8, self.quota, self.exp_idx, n_dev, st.codes,
                                                   self.limbs, self.fexp, self.S, TM=self.TMt, TMn=self.TMn)))
        if self.fused:
            out.append(("residual_flash", lambda: ops.residual_flash(
                qr, K, V, st.asg, sel, self.exp_idx, self.quota, self.n_t, st.Sk, st.Sv, self.out, sc,
                qsk=self.qsk)))
        else:
            out.append(("residual", lambda: ops.residual(K, V, st.asg, sel, self.exp_idx, self.quota, self.n_t,
                                                         st.Sk, st.Sv, self.kbar_r, self.vbar_r, self.log_n)))
            out.append(("flash", lambda: ops.flash_decode(qr, K, V, sel, self.exp_idx, self.kbar_r, self.vbar_r,
                                                          self.log_n, proxy_per_kv=False, sm_scale=sc,
                                                          out=self.out)))
        return out, sel

    def step(self, st, K, V, q, n_dev, n, marks: list | None = None, counts: tuple | None = None,
             update_index: bool = True):
        """The decode stages (`stages`) launched in order; returns the output rows
        (B, HQ, 1, D).  `marks`, when given, receives (stage, event) pairs recorded on the current
        stream after each stage."""
        def mark(name):
            if marks is not None:
                ev = torch.cuda.Event(enable_timing=True)
                ev.record()
                marks.append((name, ev))

        if self.groups > 1 and marks is None and counts is None and update_index:
            qr = q.reshape(self.R, D)
            if not qr.is_contiguous():
                qr = qr.contiguous()
            if not 1 <= n <= self.Lmax:
                raise ValueError(f"n={n} outside [1, Lmax={self.Lmax}]: the step writes position n-1")
            if K.shape[0] != self.B * HKV or K.shape[1] < n or V.shape != K.shape:
                raise ValueError(f"K, V must be ({self.B * HKV}, >= n={n}, {D}) with equal shapes")
            ns, nl, k_top = self.bud.counts(n)
            if n - ns - nl < k_top:
                raise ValueError(f"n={n} too small for sink {ns} + local {nl} + top-k {k_top}")
            sel = self.sel_buffer(ns + nl + k_top)
            main = torch.cuda.current_stream()
            per = self.B // self.groups
            for g, s in enumerate(self.streams):
                s.wait_stream(main)
                with torch.cuda.stream(s):
                    self._chain(st, K, V, qr, sel, slice(g * per * HQ, (g + 1) * per * HQ),
                                slice(g * per * HKV, (g + 1) * per * HKV), ns, nl, k_top, n_dev)
            for s in self.streams:
                main.wait_stream(s)
            self.last_sel = sel
            return self.out.view(self.B, HQ, 1, D)
        calls, sel = self.stages(st, K, V, q, n_dev, n, counts=counts, update_index=update_index)
        mark("start")
        for name, fn in calls:
            fn()
            mark(name)
        self.last_sel = sel
        return self.out.view(self.B, HQ, 1, D)

    def rows_step(self, st, K, V, q, n_dev, n_keys: int, out: torch.Tensor,
                  record: list | None = None) -> torch.Tensor:
        """A multi-row call of the estimator over an index that already holds all n_keys keys
        (UTAMultiBinAttention.custom_attention with Q rows, multibin.py:2875-2970): row i of
        q (B, HQ, Q, D) sits at position n_keys - Q + i and, under the causal mask, attends the
        n_i = n_keys - Q + i + 1 keys before it (multibin.py:2210-2218 keeps raw > NEG only);
        the sink / local / top-k sizes come from the call's key count, as the maskers size them
        from seq_len_keys (maskers/base.py:152-158), and the local window ends at the row.
        The rows run from the last to the first; after row i the key at n_i - 1 leaves the
        cluster statistics (ops.index_downdate), so row i - 1 sees those of [0, n_{i-1}); the
        statistics are restored afterwards and n_dev is left at n_keys.  Writes and returns out
        (B, HQ, Q, D).  record, when a list, receives (i, sel, quota, exp_idx) copies per row."""
        B, H, Q, _ = q.shape
        if H != HQ or B != self.B or out.shape != q.shape:
            raise ValueError(f"q and out must be ({self.B}, {HQ}, Q, {D})")
        counts = self.bud.counts(n_keys)
        ns, nl, k_top = counts
        if n_keys - Q + 1 - ns - nl < k_top:
            raise ValueError(f"{n_keys} keys leave the first of {Q} causal rows too few positions for "
                             f"sink {ns} + local {nl} + top-k {k_top}")
        snap = (st.nb.clone(), st.Sk.clone(), st.Sk2.clone(), st.Sv.clone())
        try:
            for i in range(Q - 1, -1, -1):
                n_i = n_keys - Q + i + 1
                n_dev.fill_(n_i)
                o = self.step(st, K, V, q[:, :, i], n_dev, n_i, counts=counts, update_index=False)
                out[:, :, i] = o.view(B, H, D)
                if record is not None:
                    record.append((i, self.last_sel.clone(), self.quota.clone(), self.exp_idx.clone()))
                if i > 0:
                    ops.index_downdate(K, V, st, n_dev)
        finally:
            for t, s in zip((st.nb, st.Sk, st.Sk2, st.Sv), snap):
                t.copy_(s)
            n_dev.fill_(n_keys)
        return out

    def _chain(self, st, K, V, qr, sel, rs: slice, ks: slice, ns: int, nl: int, k_top: int, n_dev):
        """The decode stages on query-head rows `rs` and their KV rows `ks` (whole sequences)."""
        sub = types.SimpleNamespace(
            codes=st.codes[ks], U=st.U[ks], scale=st.scale[ks], W=st.W[rs], colmean=st.colmean[rs],
            cent=st.cent[rs], asg=st.asg[rs], asg8=st.asg8[rs], nb=st.nb[rs], Sk=st.Sk[rs],
            Sk2=st.Sk2[rs], Sv=st.Sv[rs], reclist=st.reclist[rs], reccnt=st.reccnt[rs])
        Kg, Vg, qg, selg = K[ks], V[ks], qr[rs], sel[rs]
        ops.index_prep(Kg, Vg, sub, n_dev, RMAX, qg, self.limbs[ks], self.fexp[rs])
        ops.qgs_scan_heads(sub.codes, self.limbs[ks], self.fexp[rs], self.H[rs], self.TM[rs],
                           n_dev, ns, nl, TMn=None if self.TMn is None else self.TMn[rs])
        ops.topk_select_heads(self.H[rs], self.TM[rs], selg, n_dev, ns, nl, k_top, sub.codes,
                              self.limbs[ks], self.fexp[rs])
        ops.gate_fill(qg, Kg, sub.asg, selg, sub.Sk, sub.Sk2, sub.nb, self.score[rs], self.n_t[rs],
                      self.quota[rs], self.sm_scale, self.E, qsk=self.qsk[rs])
        ops.topq_heads(self.H[rs], sub.asg8, self.quota[rs], self.exp_idx[rs], n_dev, sub.codes,
                       self.limbs[ks], self.fexp[rs], self.S[rs],
                       TM=None if self.TMn is None else self.TM[rs],
                       TMn=None if self.TMn is None else self.TMn[rs])
        if self.fused:
            ops.residual_flash(qg, Kg, Vg, sub.asg, selg, self.exp_idx[rs], self.quota[rs],
                               self.n_t[rs], sub.Sk, sub.Sv, self.out[rs], self.sm_scale, qsk=self.qsk[rs])
        else:
            ops.residual(Kg, Vg, sub.asg, selg, self.exp_idx[rs], self.quota[rs], self.n_t[rs],
                         sub.Sk, sub.Sv, self.kbar_r[rs], self.vbar_r[rs], self.log_n[rs])
            ops.flash_decode(qg, Kg, Vg, selg, self.exp_idx[rs], self.kbar_r[rs], self.vbar_r[rs],
                             self.log_n[rs], proxy_per_kv=False, sm_scale=self.sm_scale, out=self.out[rs])
