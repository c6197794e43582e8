// Within-cluster top-q: for every (row, cluster) with quota q_c > 0, the q_c tail members of the
// cluster with the highest QGS score (ties to the lower position) become exact reads.
//
// Reference semantics: the per-token rank within its bin by the selector score
// (multibin.py:2522-2558, trunc_keep = rank < quota) with the deployed tie order of
// ours_graph.py:93-135 / ours_fused.py:228-282 (score, then members before generated tokens,
// then position -- which is position order, since every generated token follows the prefix).
// Members are the prefix members in CSR order (positions ascending) followed by the tokens
// generated since the build (the cluster's generated-token list, or, when that list
// overflowed, a scan of [n0, n) for tokens assigned to the cluster).  Selected tokens carry
// a -inf score and rank last; the quota never reaches them because q_c <= tail count.
//
// exp_idx row layout: cluster c owns slots [base_c, base_c + q_c), base_c = sum_{c'<c} q_c';
// inside a segment the members above the threshold key come first (position order), then
// the tied members at the threshold (position order).  Slots past sum q are -1.
//
// Algorithm: 256 threads per (row, cluster); 4 MSB-first 8-bit radix passes over the
// order-preserving uint32 key of each member's score find the q-th largest key T and how
// many members equal to T are taken; one ordered compaction pass writes the segment.
#include "oa_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxC = 256;

struct TopqArgs {
  const float* S; long s_stride;
  const int32_t* mem; long mem_stride;
  const int32_t* cstart; const int32_t* clen;
  const int32_t* reclist; const int32_t* reccnt; int rmax;
  const int32_t* asg; long asg_stride;
  const float* quota;
  int32_t* exp_idx; int E;
  const int* n_dev; const int* n0_dev;
  int C;
};

struct Members {
  const int32_t* mem; int clen;
  const int32_t* gen; int ngen; bool overflow; int n0;
  const int32_t* asg; int c;
  __device__ __forceinline__ int size() const { return clen + ngen; }
  // virtual index -> position, or -1 when the slot is not a member (overflow scan)
  __device__ __forceinline__ int at(int j) const {
    if (j < clen) return mem[j];
    const int jj = j - clen;
    if (!overflow) return gen[jj];
    const int p = n0 + jj;
    return asg[p] == c ? p : -1;
  }
};

__device__ __forceinline__ int block_excl_scan(int flag, int* s_wave, int* total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const unsigned long long b = __ballot(flag);
  const int below = __popcll(b & ((1ull << lane) - 1ull));
  if (lane == 0) s_wave[wave] = __popcll(b);
  __syncthreads();
  int off = 0, tot = 0;
  for (int w = 0; w < kThreads / 64; ++w) {
    if (w < wave) off += s_wave[w];
    tot += s_wave[w];
  }
  __syncthreads();
  *total = tot;
  return off + below;
}

__global__ void __launch_bounds__(kThreads) topq_kernel(TopqArgs a) {
  __shared__ int hist[256];
  __shared__ int s_bcast[4];
  __shared__ int s_wave[kThreads / 64];
  const int c = blockIdx.x;
  const int row = blockIdx.y;
  const int tid = threadIdx.x;
  const float* qrow = a.quota + (long)row * a.C;
  const int q = (int)qrow[c];
  if (c != 0 && q <= 0) return;
  // segment base and total
  int base = 0, total = 0;
  for (int i = 0; i < a.C; ++i) {
    const int qi = (int)qrow[i];
    if (i < c) base += qi;
    total += qi;
  }
  if (c == 0) {
    for (int j = total + tid; j < a.E; j += kThreads) a.exp_idx[(long)row * a.E + j] = -1;
    if (q <= 0) return;
  }
  const int n = *a.n_dev;
  const int n0 = *a.n0_dev;
  const long rc = (long)row * a.C + c;
  Members mb;
  mb.mem = a.mem + (long)row * a.mem_stride + a.cstart[rc];
  mb.clen = a.clen[rc];
  const int cnt = a.reccnt[rc];
  mb.overflow = cnt > a.rmax;
  mb.gen = a.reclist + rc * a.rmax;
  mb.ngen = mb.overflow ? max(n - n0, 0) : cnt;
  mb.n0 = n0;
  mb.asg = a.asg + (long)row * a.asg_stride;
  mb.c = c;
  const float* srow = a.S + (long)row * a.s_stride;
  const int M = mb.size();

  unsigned prefix = 0u, mask = 0u;
  int k_rem = q;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    hist[tid] = 0;
    __syncthreads();
    for (int j = tid; j < M; j += kThreads) {
      const int p = mb.at(j);
      if (p < 0) continue;
      const unsigned key = oa::float_key(srow[p]);
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1);
    }
    __syncthreads();
    if (tid == 0) {
      int cum = 0, digit = 0;
      for (int d = 255; d >= 0; --d) {
        if (cum + hist[d] >= k_rem) { digit = d; break; }
        cum += hist[d];
      }
      s_bcast[0] = digit;
      s_bcast[1] = k_rem - cum;
    }
    __syncthreads();
    prefix |= ((unsigned)s_bcast[0]) << shift;
    mask |= 255u << shift;
    k_rem = s_bcast[1];
    __syncthreads();
  }
  const unsigned T = prefix;
  const int n_gt = q - k_rem;
  // slots this segment may write (guards against quotas inconsistent with the members)
  const int limit = min(q, a.E - base);
  int32_t* seg = a.exp_idx + (long)row * a.E + base;
  int run_gt = 0, run_eq = 0;
  for (int j0 = 0; j0 < M; j0 += kThreads) {
    const int j = j0 + tid;
    int p = -1;
    unsigned key = 0u;
    if (j < M) {
      p = mb.at(j);
      if (p >= 0) key = oa::float_key(srow[p]);
    }
    const int gt = (p >= 0 && key > T) ? 1 : 0;
    const int eq = (p >= 0 && key == T) ? 1 : 0;
    int tot_gt, tot_eq;
    const int x_gt = block_excl_scan(gt, s_wave, &tot_gt);
    const int x_eq = block_excl_scan(eq, s_wave, &tot_eq);
    const int s_gt = run_gt + x_gt;
    const int s_eq = n_gt + run_eq + x_eq;
    if (gt && s_gt < n_gt && s_gt < limit) seg[s_gt] = p;
    if (eq && run_eq + x_eq < k_rem && s_eq < limit) seg[s_eq] = p;
    run_gt += tot_gt;
    run_eq += tot_eq;
  }
}

}  // namespace

extern "C" int oa_topq(const float* S, long s_stride, const int32_t* mem, long mem_stride,
                       const int32_t* cstart, const int32_t* clen, const int32_t* reclist,
                       const int32_t* reccnt, int rmax, const int32_t* asg, long asg_stride,
                       const float* quota, int rows, int C, int32_t* exp_idx, int E,
                       const int* n_dev, const int* n0_dev, void* stream) {
  if (rows <= 0 || C <= 0 || C > kMaxC || E < 0 || rmax < 0) return OA_EINVAL;
  TopqArgs a;
  a.S = S; a.s_stride = s_stride; a.mem = mem; a.mem_stride = mem_stride;
  a.cstart = cstart; a.clen = clen; a.reclist = reclist; a.reccnt = reccnt; a.rmax = rmax;
  a.asg = asg; a.asg_stride = asg_stride; a.quota = quota; a.exp_idx = exp_idx; a.E = E;
  a.n_dev = n_dev; a.n0_dev = n0_dev; a.C = C;
  hipLaunchKernelGGL(topq_kernel, dim3(C, rows), dim3(kThreads), 0, (hipStream_t)stream, a);
  return OA_LAUNCH_STATUS();
}
