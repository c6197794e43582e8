/*
 * openattention_amd -- C ABI of the gfx950 kernels of OpenAttention's sparse decode path.
 *
 * Conventions for every entry point:
 *   - plain device pointers, element strides (not bytes) and sizes; no torch types.
 *   - `stream` is a hipStream_t passed as void*; every launch goes on it, nothing synchronises,
 *     nothing allocates and nothing is read back on the host, so a caller may capture a whole
 *     decode step in a hipGraph.
 *   - the current length n (and n0, the prefix length at build time) are read from device
 *     memory (`n_dev`, `n0_dev`: one int32 each), as the reference's graph-safe kernels do.
 *   - return 0 on success, -22 (OA_EINVAL) when a shape/stride/size check fails, -28
 *     (OA_ENOSPC) when a request exceeds a fixed device scratch area, otherwise the hipError_t
 *     of the launch.  oa_error_string() gives the text.
 *   - head_dim is 128, the QGS rank 32, the QGC rank 16 and the GQA group 4 (Llama-3.1-8B);
 *     other values are rejected.
 *   - rows R = B * HQ query-head rows; kv_rows = B * HKV; row r reads KV row r / (R / kv_rows).
 *
 * Reference interfaces (paths relative to the hyunwoo137/OpenAttention checkout) each function
 * replaces are cited per declaration.  The reference binds these stages from Python; the
 * ctypes binding of this library is openattention_amd/lib.py.
 */
#ifndef OPENATTENTION_AMD_H
#define OPENATTENTION_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OA_ABI_VERSION 9
#define OA_EINVAL (-22)
#define OA_ENOSPC (-28)

/* ABI version of the loaded library (OA_ABI_VERSION of the header it was built from). */
int oa_abi_version(void);

/* Text for a status returned by any entry point. */
const char* oa_error_string(int status);

/*
 * OpenAttention.flash: one online softmax per query-head row over the selected tokens (sel),
 * the expanded tokens (exp_idx) and the cluster proxies (kbar, vbar, log_n).
 * Replaces ours_flash (inference/methods_eager.py:161-172; kernel :91-158) when
 * proxy_per_kv == 0 and decode_expand_attention (triton_expand_decode.py:139-165; kernel
 * :31-136) when proxy_per_kv == 1 (kbar/vbar rows indexed by KV head).
 *   q (rows, 128) bf16; k, v (kv_rows, Lmax, 128) bf16; sel (rows, n_sel), exp_idx
 *   (rows, n_exp) int32 with -1 padding; kbar, vbar (rows or kv_rows, n_bins, 128) bf16 or
 *   fp32 (kbar_is_f32); log_n (rows, n_bins) fp32 natural log, -inf = no proxy;
 *   out (rows, 128) bf16, or fp32 when out_is_f32 (the fp32 accumulators unrounded).  A row
 *   with nothing valid returns 0.
 *   n_split > 1 splits each row's list over n_split workgroups (the reference's split-K
 *   variant for few rows, inference/ours_graph.py:214-262 + graph_runner.py:299-312); the
 *   caller passes workspaces ws_m, ws_l (rows*n_split fp32) and ws_acc (rows*n_split*128).
 */
int oa_flash_decode(const void* q, long q_stride, const void* k, const void* v, long kv_stride_b,
                    long kv_stride_s, const int32_t* sel, long sel_stride, int n_sel,
                    const int32_t* exp_idx, long exp_stride, int n_exp, const void* kbar,
                    const void* vbar, long kbar_stride_b, long kbar_stride_n, int kbar_is_f32,
                    int proxy_per_kv, const float* log_n, long log_n_stride, int n_bins, void* out,
                    long out_stride, int out_is_f32, int rows, int kv_rows, int head_dim,
                    float sm_scale, int n_split, float* ws_m, float* ws_l, float* ws_acc,
                    void* stream);

/*
 * oa_flash_decode without workspaces, for callers that cannot allocate device memory (code
 * under hipGraph capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  The split partials of n_split > 1 live in a fixed per-GPU
 * device array of 4 MiB, so rows * n_split * 130 must not exceed 1048576 (else OA_ENOSPC,
 * nothing launched).  The library allocates nothing: the array is part of the code object,
 * held on each GPU until the process ends.  Calls that overlap on one GPU (concurrent streams)
 * share that array and race; calls in stream order do not.  Results equal oa_flash_decode's
 * with the same arguments.
 */
int oa_flash_decode_noalloc(const void* q, long q_stride, const void* k, const void* v,
                            long kv_stride_b, long kv_stride_s, const int32_t* sel,
                            long sel_stride, int n_sel, const int32_t* exp_idx, long exp_stride,
                            int n_exp, const void* kbar, const void* vbar, long kbar_stride_b,
                            long kbar_stride_n, int kbar_is_f32, int proxy_per_kv,
                            const float* log_n, long log_n_stride, int n_bins, void* out,
                            long out_stride, int out_is_f32, int rows, int kv_rows, int head_dim,
                            float sm_scale, int n_split, void* stream);

/*
 * Index update of the token at position n-1: its int8 QGS code (KV-head rows), its nearest
 * QGC centroid, the cluster's pooled sums (n, sum k, sum k^2, sum v) and the cluster's list
 * of generated tokens (capacity rmax; the count keeps growing past it, marking overflow).
 * Replaces _k_index_update_d2 (inference/ours_graph.py:43-90).
 *   codes (kv_rows, codes_lmax, 32) int8; U (kv_rows, 128, 32), scale (kv_rows, 32) fp32;
 *   W (rows, 128, 16) bf16; colmean (rows, 16), cent (rows, C, 16) fp32; asg (rows,
 *   asg_stride) int32 and its byte copy asg8 (rows, asg8_stride) uint8 (C <= 256); nb (rows, C),
 *   Sk, Sk2, Sv (rows, C, 128) fp32; reclist (rows, C, rmax), reccnt (rows, C) int32.
 */
int oa_index_update(const void* K, const void* V, long kv_stride_b, long kv_stride_s, int rows,
                    int kv_rows, int head_dim, int8_t* codes, int codes_lmax, int rank_q,
                    const float* U, const float* scale, const void* W, const float* colmean,
                    int rank_c, const float* cent, int C, int32_t* asg, long asg_stride,
                    uint8_t* asg8, long asg8_stride, float* nb, float* Sk, float* Sk2, float* Sv,
                    int32_t* reclist, int32_t* reccnt, int rmax, const int* n_dev, void* stream);

/*
 * The token at position n-1 leaves the cluster statistics of every query row: n_c -= 1,
 * Sk_c -= k, Sk2_c -= k*k, Sv_c -= v in fp32, c = asg[row][n-1] (the index update's statistics
 * step, undone; codes, cluster ids and lists are untouched).  A multi-row call (the question
 * chunk) takes its keys back one at a time from the last, so that its causal row i, which
 * attends the keys before n_i = K - Q + i + 1, sees the statistics of exactly those keys: the
 * reference's estimator keeps only positions with raw > NEG in each row's tail
 * (multibin.py:2210-2218, the causal mask added to the logits).  No kernel of the reference's
 * deployed path does this: its question chunk runs dense (graph_runner.py:472-475).
 *   asg (rows, asg_stride) int32; nb (rows, C), Sk, Sk2, Sv (rows, C, 128) fp32; C <= 256.
 */
int oa_index_downdate(const void* K, const void* V, long kv_stride_b, long kv_stride_s, int rows,
                      int kv_rows, int head_dim, const int32_t* asg, long asg_stride, float* nb,
                      float* Sk, float* Sk2, float* Sv, int C, const int* n_dev, void* stream);

/*
 * QGS query projection zq = (q U) * scale and its exact fixed-point form (exponent fexp per
 * row, four int8 limbs of round(zq * 2^fexp) per KV-head block).  Replaces the torch
 * projection of inference/ours_graph.py:298 (StaticTopKMasker._scores,
 * static_top_k.py:203-213).
 *   limbs (kv_rows, 16, 32) int8; fexp (rows) int32; zq_out (rows, 32) fp32 or NULL.
 */
int oa_qgs_prep(const void* q, long q_stride, const float* U, const float* scale, int rows,
                int kv_rows, int head_dim, int rank, int8_t* limbs, int* fexp, float* zq_out,
                void* stream);

/*
 * oa_index_update and oa_qgs_prep in one launch (the two touch disjoint data; per query-head
 * row one wave does each).  Replaces the pair _k_index_update_d2 + the zq projection at the
 * start of the deployed step (inference/ours_graph.py:290-298).  Arguments: those of
 * oa_index_update followed by q, q_stride, limbs, fexp of oa_qgs_prep; rows = 4 * kv_rows.
 */
int oa_index_prep(const void* K, const void* V, long kv_stride_b, long kv_stride_s, int rows,
                  int kv_rows, int head_dim, int8_t* codes, int codes_lmax, int rank_q,
                  const float* U, const float* scale, const void* W, const float* colmean,
                  int rank_c, const float* cent, int C, int32_t* asg, long asg_stride,
                  uint8_t* asg8, long asg8_stride, float* nb, float* Sk, float* Sk2, float* Sv,
                  int32_t* reclist, int32_t* reccnt, int rmax, const int* n_dev, const void* q,
                  long q_stride, int8_t* limbs, int* fexp, void* stream);

/*
 * QGS scan: exact score of every position for the 4 query heads of each KV head, on the
 * int8 matrix cores; sink (< ns), local (>= n - nl) and unwritten positions are -inf; plus
 * the maximum of every 64-token tile.  Replaces _k_qgs_scan_tm
 * (inference/graph_runner.py:100-120).
 *   S (rows, s_stride >= ceil(Lmax/64)*64) fp32; TM (rows, tm_stride >= ceil(Lmax/64)) fp32.
 */
int oa_qgs_scan(const int8_t* codes, int kv_rows, int Lmax, int rank, const int8_t* limbs,
                const int* fexp, float* S, long s_stride, float* TM, long tm_stride,
                const int* n_dev, int ns, int nl, void* stream);

/*
 * oa_qgs_scan writing the 16-bit head of every score's order-preserving key (the key's top 16
 * bits: non-decreasing in the score; -inf is 0x007f) instead of the fp32 score: half the
 * bytes, and all that the top-q binning uses.  TM is the same exact fp32 tile maximum.  The
 * same stage as oa_qgs_scan (_k_qgs_scan_tm, inference/graph_runner.py:100-120); the reduced
 * score rows have no counterpart in the reference.
 *   H (rows, h_stride >= ceil(Lmax/64)*64, a multiple of 4) 16-bit, 8-byte aligned.
 *   TMn (NULL, or like TM): each tile's least finite score, +inf for a tile without one -- the
 *   row range oa_topq_heads bins with, known before the row is read.  No reference counterpart.
 */
int oa_qgs_scan_heads(const int8_t* codes, int kv_rows, int Lmax, int rank, const int8_t* limbs,
                      const int* fexp, uint16_t* H, long h_stride, float* TM, long tm_stride,
                      float* TMn, const int* n_dev, int ns, int nl, void* stream);

/*
 * Exact top-k per row (ties to the lower position) among the k tiles with the largest
 * maxima; sel = [0..ns) ++ [n-nl..n) ++ top; the selected scores in S are set to -inf.
 * Replaces _k_select (inference/graph_runner.py:123-159).
 *   0 <= k_top <= min(64, ntiles), ns, nl <= 64; the decode step keeps k_top <= n - ns - nl.
 *   A row with fewer live positions ([ns, n - nl)) than k_top is filled, after every live
 *   position, with the lowest sink, local or unwritten positions (scored -inf, as the
 *   reference's -inf candidates): every selected position is below ntiles * 64.
 */
int oa_topk_select(float* S, long s_stride, const float* TM, long tm_stride, int rows,
                   int ntiles, int32_t* sel, long sel_stride, const int* n_dev, int ns, int nl,
                   int k_top, void* stream);

/*
 * oa_topk_select over key-head rows (oa_qgs_scan_heads): the candidate tiles' exact scores are
 * recomputed from the codes with the scan's integer arithmetic, so sel is the same; the
 * selected tokens' heads are set to that of -inf.  Replaces _k_select
 * (inference/graph_runner.py:123-159) in the head pipeline.
 *   codes (kv_rows, Lmax, 32) int8, 16-byte aligned; limbs (kv_rows, 16, 32); fexp (rows,).
 */
int oa_topk_select_heads(uint16_t* H, long h_stride, const float* TM, long tm_stride, int rows,
                         int ntiles, int32_t* sel, long sel_stride, const int* n_dev, int ns,
                         int nl, int k_top, const int8_t* codes, int kv_rows, int Lmax,
                         const int8_t* limbs, const int* fexp, void* stream);

/*
 * ErrorGate: wl1 score and tail count of every cluster (pooled sums minus the selected
 * tokens).  Replaces _k_errorgate (inference/ours_fused.py:122-154).
 *   sm_scale_sq is the fp32 value of the squared scale as the estimator forms it (the square
 *   taken in double, then rounded: multibin.py:643), which can differ from fp32(s)^2 by 1 ulp.
 *   score, n_t (rows, C) fp32.
 */
int oa_errorgate(const void* q, long q_stride, const void* K, long k_stride_b, long k_stride_s,
                 int rows, int kv_rows, int head_dim, const int32_t* asg, long asg_stride,
                 const int32_t* sel, long sel_stride, int n_sel, const float* Sk, const float* Sk2,
                 const float* nb, int C, float sm_scale, float sm_scale_sq, float* score,
                 float* n_t, void* stream);

/*
 * Hierarchical water-filling of the exact-read budget E over the clusters (fp64 bisection of
 * UTAMultiBinAttention._hier_quota_impl, multibin.py:1385-1422).  Replaces _k_waterfill
 * (inference/ours_fused.py:157-216).   quota (rows, C) fp32 (integer valued, sums to
 * min(E, sum of live tail counts)).
 */
int oa_waterfill(const float* score, const float* n_t, int rows, int C, int budget, float* quota,
                 void* stream);

/*
 * ErrorGate and water-filling (one launch below 256 rows, two above; score and n_t are also
 * written out).  Same results as oa_errorgate followed by oa_waterfill.  qsk (rows, C) fp32, when not
 * null, receives q . Sk_c of every cluster (pooled sums, before the selected tokens leave them)
 * for oa_residual_flash; no counterpart in the reference.
 */
int oa_gate_fill(const void* q, long q_stride, const void* K, long k_stride_b, long k_stride_s,
                 int rows, int kv_rows, int head_dim, const int32_t* asg, long asg_stride,
                 const int32_t* sel, long sel_stride, int n_sel, const float* Sk, const float* Sk2,
                 const float* nb, int C, float sm_scale, float sm_scale_sq, int budget,
                 float* score, float* n_t, float* quota, float* qsk, void* stream);

/*
 * oa_topk_select_heads followed by oa_gate_fill (n_sel = ns + nl + k_top, sel written as by
 * oa_topk_select_heads): the same sel, marked heads, score, n_t, quota and qsk.  With a register
 * top-k (k_top <= 16 and at most 2048 score tiles), and below 256 rows or at C <= 64, it is one
 * launch: each row's workgroup runs its top-k on one wave while its other waves compute every
 * cluster's ErrorGate from the pooled sums, then the clusters holding a selected token are
 * computed again without those tokens (the same arithmetic) and the row's water-fill runs;
 * otherwise the two calls.
 * Replaces the consecutive _k_select and _k_errorgate / _k_waterfill steps of the deployed decode
 * graph (inference/graph_runner.py:123-159, inference/ours_fused.py:122-216); the fusion itself
 * has no counterpart in the reference.
 */
int oa_topk_gate_fill(uint16_t* H, long h_stride, const float* TM, long tm_stride, int ntiles,
                      const int* n_dev, int ns, int nl, int k_top, const int8_t* codes, int Lmax,
                      const int8_t* limbs, const int* fexp, const void* q, long q_stride,
                      const void* K, long k_stride_b, long k_stride_s, int rows, int kv_rows,
                      int head_dim, const int32_t* asg, long asg_stride, int32_t* sel,
                      long sel_stride, const float* Sk, const float* Sk2, const float* nb, int C,
                      float sm_scale, float sm_scale_sq, int budget, float* score, float* n_t,
                      float* quota, float* qsk, void* stream);

/*
 * oa_qgs_scan_heads and the pooled part of the ErrorGate in one launch: besides the key heads
 * and tile maxima, every cluster's wl1 score and tail count as if it held no selected token
 * (the pooled sums; score, n_t (rows, C)) and q . Sk_c (qsk, or NULL).  Scan blocks and gate
 * blocks (one row, 16 clusters each) are interleaved in one grid, so the gate's dependent chains
 * run under the code stream.  For the clusters that hold no selected token these are the final
 * ErrorGate outputs (the same arithmetic as oa_errorgate); oa_topk_fix_fill corrects the others
 * once the selection is known.  The fusion has no counterpart in the reference: it splits
 * _k_errorgate (inference/ours_fused.py:122-154) into its selection-independent part, run with
 * the scan (inference/graph_runner.py:100-120), and the selected tokens' part.
 *   Arguments: those of oa_qgs_scan_heads, then q (rows = 4 * kv_rows, 128) bf16, Sk, Sk2
 *   (rows, C, 128), nb (rows, C) fp32, C <= 256, the softmax scale and its square.
 */
int oa_qgs_scan_gate(const int8_t* codes, int kv_rows, int Lmax, int rank, const int8_t* limbs,
                     const int* fexp, uint16_t* H, long h_stride, float* TM, long tm_stride,
                     float* TMn, const int* n_dev, int ns, int nl, const void* q, long q_stride, const float* Sk,
                     const float* Sk2, const float* nb, int C, float sm_scale, float sm_scale_sq,
                     float* score, float* n_t, float* qsk, void* stream);

/*
 * After oa_qgs_scan_gate: the top-k over the key heads (as oa_topk_select_heads), then the
 * ErrorGate of the clusters holding a selected token done again from the pooled sums minus
 * their selected keys (score and n_t updated in place; the others keep the pooled values), then
 * the water-filling.  The same sel, marked heads, score, n_t and quota as oa_topk_select_heads
 * followed by oa_gate_fill.  One launch (a workgroup per row: its top-k, correction and fill)
 * with a register top-k (k_top <= 16 and at most 2048 score tiles), else the radix top-k and a
 * second launch.  Replaces the consecutive _k_select and _k_errorgate / _k_waterfill steps
 * (inference/graph_runner.py:123-159, inference/ours_fused.py:122-216).
 */
int oa_topk_fix_fill(uint16_t* H, long h_stride, const float* TM, long tm_stride, int ntiles,
                     const int* n_dev, int ns, int nl, int k_top, const int8_t* codes, int Lmax,
                     const int8_t* limbs, const int* fexp, const void* q, long q_stride,
                     const void* K, long k_stride_b, long k_stride_s, int rows, int kv_rows,
                     int head_dim, const int32_t* asg, long asg_stride, int32_t* sel,
                     long sel_stride, const float* Sk, const float* Sk2, const float* nb, int C,
                     float sm_scale, float sm_scale_sq, int budget, float* score, float* n_t,
                     float* quota, void* stream);

/*
 * Within-cluster top-q: the q_c best tail members of every cluster by QGS score (ties to the
 * lower position), written to exp_idx in segments grouped by cluster (position order inside a
 * segment, -1 past the chosen members), -1 past the quota total; a segment straddling E keeps
 * its best E - base members.  Replaces _k_topq_d2 (inference/ours_graph.py:138-166): instead
 * of gathering member scores through the CSR lists, one workgroup streams each row once
 * (scores S from oa_topk_select, byte cluster ids asg8) and selects by per-cluster histogram
 * thresholds.
 *   quota (rows, C) fp32; exp_idx (rows, E) int32.  E <= 4096, C <= 256, Lmax < 2^24.
 */
int oa_topq(const float* S, long s_stride, const uint8_t* asg8, long asg8_stride,
            const float* quota, int rows, int C, int Lmax, int32_t* exp_idx, int E,
            const int* n_dev, void* stream);

/*
 * oa_topq with the algorithm chosen: path 0 (what oa_topq runs) bins scores linearly over each
 * row's score range and leaves rows whose boundary bins overflow the staging space to the
 * key-prefix histogram kernel; path 1 runs the key-prefix kernel on every row; path 2 runs the
 * linear-bin kernel alone, and a row it leaves to the other kernel holds -2 in exp_idx[row][0]
 * (its other slots are not written).  Paths 0 and 1 give the same exp_idx.  No counterpart in
 * the reference: paths 1 and 2 exist so that each kernel can be checked on its own.
 */
int oa_topq_path(const float* S, long s_stride, const uint8_t* asg8, long asg8_stride,
                 const float* quota, int rows, int C, int Lmax, int32_t* exp_idx, int E,
                 const int* n_dev, int path, void* stream);

/*
 * Within-cluster top-q over key-head rows (oa_qgs_scan_heads, oa_topk_select_heads): the
 * linear-bin kernel bins the heads, recomputes exact scores from the codes for the staged
 * members, and writes a row it cannot resolve into S32 as exact fp32 scores for the key-prefix
 * kernel.  Same result as oa_topq on the fp32 scores.  Replaces _k_topq_d2 + _topq_core
 * (inference/ours_graph.py:93-166) in the head pipeline.  path 0: as described; 2: the
 * linear-bin kernel alone (rows it leaves hold -2 in exp_idx[row][0]); 3 (tests): every row
 * through S32 and the key-prefix kernel.
 *   H as oa_qgs_scan_heads; S32 (rows, s32_stride >= round_up(Lmax, 4)) fp32, 16-byte aligned;
 *   rows = 4 * kv_rows.  TM, TMn (both NULL, or both the scan's, tm_stride >= ceil(Lmax/64)):
 *   the row's range is taken from the tile extremes instead of a pass over the row, and each
 *   group of positions is binned as it arrives (same result).
 */
int oa_topq_heads(const uint16_t* H, long h_stride, const uint8_t* asg8, long asg8_stride,
                  const float* quota, int rows, int C, int Lmax, int32_t* exp_idx, int E,
                  const int* n_dev, const int8_t* codes, int kv_rows, const int8_t* limbs,
                  const int* fexp, float* S32, long s32_stride, const float* TM, const float* TMn,
                  long tm_stride, int path, void* stream);

/*
 * Residual proxies: kbar', vbar' (bf16, rows x C x 128) and ln n' (fp32, -inf = none) of the
 * tokens still unread.  Replaces _k_resid_scatter + _k_resid_norm
 * (inference/ours_fused.py:366-407).
 */
int oa_residual(const void* K, const void* V, long kv_stride_b, long kv_stride_s, int rows,
                int kv_rows, int head_dim, const int32_t* asg, long asg_stride,
                const int32_t* sel, long sel_stride, int n_sel, const int32_t* exp_idx, int E,
                const float* quota, const float* n_t, const float* Sk, const float* Sv, int C,
                void* kbar_r, void* vbar_r, float* log_n, void* stream);

/*
 * Residual proxies fused with OpenAttention.flash: every K/V row read once, proxies kept in
 * registers (fp32).  Replaces the residual + ours_flash pair of the deployed step
 * (inference/ours_graph.py:324-344).   out (rows, 128) bf16, or fp32 when out_is_f32.  qsk
 * (rows, C) from oa_gate_fill, when not null, stands in for the kernel's own q . Sk pass (Sk is
 * then not read).
 */
int oa_residual_flash(const void* q, long q_stride, const void* K, const void* V,
                      long kv_stride_b, long kv_stride_s, int rows, int kv_rows, int head_dim,
                      const int32_t* asg, long asg_stride, const int32_t* sel, long sel_stride,
                      int n_sel, const int32_t* exp_idx, int E, const float* quota,
                      const float* n_t, const float* Sk, const float* Sv, int C, float sm_scale,
                      void* out, long out_stride, int out_is_f32, const float* qsk, void* stream);

/*
 * Dense bf16 decode attention over positions [0, n) (the comparator), split-K over nsplit key
 * chunks + combine; workspaces ws_m, ws_l (rows*nsplit) and ws_acc (rows*nsplit*128) fp32.
 * Replaces _k_dense_split + _k_dense_combine (inference/graph_runner.py:259-312).
 */
int oa_dense_decode(const void* q, long q_stride, const void* K, const void* V, long kv_stride_b,
                    long kv_stride_s, int rows, int kv_rows, int head_dim, int Lmax,
                    const int* n_dev, float sm_scale, int nsplit, float* ws_m, float* ws_l,
                    float* ws_acc, void* out, long out_stride, void* stream);

/* ---- prefill index build (one request: kv_rows KV-head rows, rows = G * kv_rows query rows) */

/*
 * QGS codes of tokens [0, T): zc = k U (fp32 fma chain over d), scale = max(max_t |zc| / 127,
 * 1e-12) per (KV row, coordinate), codes = clamp(rint(zc / scale), -127, 127).  K: kv_rows
 * rows of (T, 128) bf16 at k_stride_h / k_stride_t; U (kv_rows, 128, 32) fp32; codes
 * (kv_rows, codes_stride_h / 32, 32) int8; scale (kv_rows, 32); amax_ws (kv_rows * 32) uint32
 * scratch; zc_ws (kv_rows * T * 32) fp32 scratch, 16-byte aligned, or NULL: with it zc is formed
 * once and kept between the two passes, without it the second pass forms it again (same codes).
 * Replaces the code step of inference/ours_fastbuild.py:256-261 and methods_eager.py:519-525
 * (StaticTopKMasker._extend, static_top_k.py:174-181).
 */
int oa_qgs_codes(const void* K, long k_stride_h, long k_stride_t, int kv_rows, int T,
                 const float* U, int8_t* codes, long codes_stride_h, float* scale,
                 uint32_t* amax_ws, float* zc_ws, void* stream);

/*
 * QGC projection bf16(k W) on the bf16 matrix cores and colmean = mean over the T tokens of
 * bf16(k W) (fp64 tile sums in a fixed order); zP = bf16(k W) - colmean.  W (rows, 128, 16)
 * bf16 (per query row); zraw_out (rows, zp_stride) the bf16 bits of k W (what the k-means entry
 * points read), zP (rows, zp_stride) fp32, either may be NULL but not both; zp_stride >= 16 T;
 * colmean (rows, 16); tile_ws (rows * ceil(T/64) * 16) fp64 scratch.  Replaces the projection
 * of inference/ours_fastbuild.py:264-275 and methods_eager.py:526-531.
 */
int oa_qgc_project(const void* K, long k_stride_h, long k_stride_t, int rows, int G, int T,
                   const void* W, float* zP, long zp_stride, float* colmean, double* tile_ws,
                   uint16_t* zraw_out, void* stream);

/*
 * k-means assignment: asg_t = argmax_c bf16(bf16(bf16(zP_t) . bf16(c)) - bf16(|c|^2 / 2)), ties
 * to the lower cluster, written as int32 and uint8; zP_t = zraw_t - colmean (fp32, formed from
 * the stored bf16 projection).  zraw (rows, z_stride) as oa_qgc_project writes it; cent
 * (rows, C, 16) fp32.  Replaces _k_km_assign (inference/ours_fastbuild.py:52-82) and
 * methods_eager.py:536-540.
 */
int oa_kmeans_assign(const uint16_t* zraw, const float* colmean, long z_stride, int rows, int T,
                     const float* cent, int C, int32_t* asg, long asg_stride, uint8_t* asg8,
                     long asg8_stride, void* stream);

/*
 * k-means update: centroid = mean of the members' zP rows (fp64 sum in position order, one
 * rounding), or zP[init_idx[c]] for an empty cluster; zP = zraw - colmean as in
 * oa_kmeans_assign; cnt_out (rows, C) member counts or NULL.  mem_ws (rows, mem_stride >= T),
 * cstart_ws, clen_ws (rows, C) int32 receive the assignment's member lists (the layout
 * oa_cluster_build writes) on the way.  Replaces _k_km_update (inference/ours_fastbuild.py:85-108)
 * and methods_eager.py:541-547.
 */
int oa_kmeans_update(const uint16_t* zraw, const float* colmean, long z_stride, int rows, int T,
                     const uint8_t* asg8, long asg8_stride, int C, const int32_t* init_idx,
                     float* cent, float* cnt_out, int32_t* mem_ws, long mem_stride,
                     int32_t* cstart_ws, int32_t* clen_ws, void* stream);

/*
 * Cluster statistics and CSR member lists: nb = member count, Sk = sum k, Sk2 = sum k*k,
 * Sv = sum v (fp64 sums in position order, one rounding); mem = members by cluster, in position
 * order (the stable argsort of the assignment), cstart / clen per cluster.  K, V: kv_rows rows
 * of (T, 128) bf16; nb (rows, C); Sk, Sk2, Sv (rows, C, 128); mem (rows, mem_stride).
 * Replaces _k_cluster_sums and the CSR build of inference/ours_fastbuild.py:111-139, 293-301
 * (methods_eager.py:548-555).
 */
int oa_cluster_build(const void* K, const void* V, long kv_stride_h, long kv_stride_t, int rows,
                     int G, int T, const uint8_t* asg8, long asg8_stride, int C, float* nb,
                     float* Sk, float* Sk2, float* Sv, int32_t* mem, long mem_stride,
                     int32_t* cstart, int32_t* clen, void* stream);

/*
 * Cluster statistics over member lists already built (the ones oa_kmeans_update leaves for the
 * assignment it was given): nb = clen (as float), Sk = sum k, Sk2 = sum k*k, Sv = sum v (fp64
 * sums in list order, one rounding); the same outputs as oa_cluster_build for that assignment,
 * without sorting it again.  mem (rows, mem_stride), cstart / clen (rows, C) as oa_cluster_build
 * writes them.  Replaces _k_cluster_sums (inference/ours_fastbuild.py:111-139) where the CSR
 * lists of ours_fastbuild.py:293-301 are already at hand.
 */
int oa_cluster_sums(const void* K, const void* V, long kv_stride_h, long kv_stride_t, int rows, int G,
                    int T, int C, float* nb, float* Sk, float* Sk2, float* Sv, const int32_t* mem,
                    long mem_stride, const int32_t* cstart, const int32_t* clen, void* stream);

/*
 * The a10 query metric of rows / G KV rows' G query-head rows each: for query row r, with its P
 * picked question rows q_p (positions pick[p] of q's row r) advanced by their RoPE angles,
 * r_p = scaling (cos_p * q_p + sin_p * rotate_half(q_p)) in fp64, Mq = fp32(sum_p r_p r_p^T / P),
 * M_r = mst_half[r % heads] + 0.5 (Mq / max(tr Mq, 1e-12)), written to m_out[r]; the KV row's
 * mean of its G metrics to gm_out[r / G].  q (rows, Qn, 128) bf16 (q_bf16 = 1) or fp32 with row
 * and position strides in elements; pick (P) int32, 1 <= P <= 64; cosv, sinv (P, 128) fp64;
 * mst_half (heads, 128, 128) fp32 (half the trace-normalised rotated static metric); gm_out
 * (rows / G, 128, 128), m_out (rows, 128, 128) fp32, 16-byte aligned.  Replaces the metric of
 * inference/methods_eager.py:510-519 (question moment static_top_k.py:185-194).
 */
int oa_query_metric(const void* q, int q_bf16, long q_stride_row, long q_stride_pos, int rows, int G,
                    const int32_t* pick, int P, const double* cosv, const double* sinv, double scaling,
                    const float* mst_half, int heads, float* gm_out, float* m_out, void* stream);

/*
 * Top-k eigenpairs of symmetric positive semi-definite 128 x 128 fp32 matrices (one-sided Jacobi,
 * one workgroup per matrix; the lower triangle is read).  M (batch, m_stride >= 128*128) row-major;
 * evals (batch, k) and evecs (batch, 128, k) receive the k largest eigenvalues and their unit
 * eigenvectors in ascending order (the last k of torch.linalg.eigh's order; signs are free);
 * 1 <= k <= 64; n must be 128.  sweeps (batch) int32 or NULL: the Jacobi sweeps each matrix took
 * (negative if it reached the sweep cap unconverged).  Replaces torch.linalg.eigh in the a10
 * bases of inference/methods_eager.py:519-528.
 */
int oa_sym_eig_top(const float* M, long m_stride, int batch, int n, int k, float* evals,
                   float* evecs, int* sweeps, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* OPENATTENTION_AMD_H */
