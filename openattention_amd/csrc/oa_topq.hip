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
// a segment lists its chosen members in position order; slots past sum q are -1.
//
// gfx950 decomposition: one 256-thread workgroup per row; its four waves take the row's
// clusters round-robin and skip the ones without quota.  A wave serves a cluster of at most
// 1024 members and a quota of at most 64 from registers: each lane holds 16 members as unique
// 64-bit keys (score key, then the complement of the position), and q rounds of a wave
// butterfly max extract the winners exactly.  Larger clusters or quotas take a wave-level
// radix select: four MSB-first 8-bit passes over the score key with a wave-private LDS
// histogram and a lane-parallel digit search, then ties at the threshold are taken in
// position order by ballot prefix counts.
#include "oa_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxC = 256;
constexpr int KREG = 16;          // member slots per lane on the register path
constexpr int QREG = 64;          // largest quota served by extraction

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

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const unsigned long long o = __shfl_xor(v, m, 64);
    v = o > v ? o : v;
  }
  return v;
}

// number of lanes below this one with flag set, and the wave total
__device__ __forceinline__ int lanes_below(bool flag, int lane, int* total) {
  const unsigned long long b = __ballot(flag);
  *total = __popcll(b);
  return __popcll(b & ((1ull << lane) - 1ull));
}

__device__ void topq_extract(const Members& mb, const float* srow, int q, int32_t* seg, int limit,
                             int lane) {
  const int M = mb.size();
  unsigned long long key[KREG];
#pragma unroll
  for (int j = 0; j < KREG; ++j) {
    const int idx = j * 64 + lane;
    const int p = idx < M ? mb.at(idx) : -1;
    key[j] = p >= 0 ? (((unsigned long long)oa::float_key(srow[p]) << 32) | (0xffffffffu - (unsigned)p))
                    : 0ull;
  }
  unsigned taken = 0u;
  for (int t = 0; t < q; ++t) {
    unsigned long long best = 0ull;
#pragma unroll
    for (int j = 0; j < KREG; ++j)
      if (!((taken >> j) & 1u) && key[j] > best) best = key[j];
    best = wave_max_u64(best);
    if (best == 0ull) break;
#pragma unroll
    for (int j = 0; j < KREG; ++j)
      if (key[j] == best) taken |= 1u << j;
  }
  int run = 0;
#pragma unroll
  for (int j = 0; j < KREG; ++j) {
    const bool f = (taken >> j) & 1u;
    int tot;
    const int below = lanes_below(f, lane, &tot);
    if (f && run + below < limit) seg[run + below] = (int)(0xffffffffu - (unsigned)(key[j] & 0xffffffffull));
    run += tot;
  }
}

__device__ void topq_radix(const Members& mb, const float* srow, int q, int32_t* seg, int limit,
                           int lane, int* hist) {
  const int M = mb.size();
  unsigned prefix = 0u, mask = 0u;
  int k_rem = q;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
#pragma unroll
    for (int i = 0; i < 4; ++i) hist[lane * 4 + i] = 0;
    wave_sync();
    for (int idx = lane; idx < M; idx += 64) {
      const int p = mb.at(idx);
      if (p < 0) continue;
      const unsigned key = oa::float_key(srow[p]);
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1);
    }
    wave_sync();
    int h[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) h[i] = hist[lane * 4 + i];
    const int tot = h[0] + h[1] + h[2] + h[3];
    int incl = tot;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int t = __shfl_down(incl, off, 64);
      if (lane + off < 64) incl += t;
    }
    int cum = incl - tot;            // members whose digit lies in higher lanes
    int found = -1, newk = 0;
#pragma unroll
    for (int i = 3; i >= 0; --i) {
      if (found < 0 && cum < k_rem && cum + h[i] >= k_rem) {
        found = lane * 4 + i;
        newk = k_rem - cum;
      }
      cum += h[i];
    }
    const unsigned long long bl = __ballot(found >= 0);
    const int src = bl ? (int)__builtin_ctzll(bl) : 0;
    const int digit = bl ? __shfl(found, src, 64) : 0;
    k_rem = bl ? __shfl(newk, src, 64) : 0;
    prefix |= ((unsigned)digit) << shift;
    mask |= 255u << shift;
    wave_sync();
  }
  const unsigned T = prefix;
  int run = 0, eq_seen = 0;
  for (int b0 = 0; b0 < M; b0 += 64) {
    const int idx = b0 + lane;
    const int p = idx < M ? mb.at(idx) : -1;
    const unsigned key = p >= 0 ? oa::float_key(srow[p]) : 0u;
    const bool gt = p >= 0 && key > T;
    const bool eq = p >= 0 && key == T;
    int eq_tot, take_tot;
    const int eq_rank = eq_seen + lanes_below(eq, lane, &eq_tot);
    const bool take = gt || (eq && eq_rank < k_rem);
    const int slot = run + lanes_below(take, lane, &take_tot);
    if (take && slot < limit) seg[slot] = p;
    run += take_tot;
    eq_seen += eq_tot;
  }
}

__global__ void __launch_bounds__(kThreads) topq_kernel(TopqArgs a) {
  __shared__ int s_q[kMaxC];
  __shared__ int s_base[kMaxC + 1];
  __shared__ int s_hist[kWaves][256];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const float* qrow = a.quota + (long)row * a.C;
  if (wave == 0) {
    // lane l owns clusters 4l..4l+3: local sums, then an exclusive scan over the lanes
    int v[4], loc = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = lane * 4 + i;
      v[i] = c < a.C ? (int)qrow[c] : 0;
      loc += v[i];
    }
    int incl = loc;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int t = __shfl_up(incl, off, 64);
      if (lane >= off) incl += t;
    }
    int run = incl - loc;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = lane * 4 + i;
      if (c < a.C) { s_q[c] = v[i]; s_base[c] = run; }
      run += v[i];
    }
    if (lane == 63) s_base[a.C] = incl;
  }
  __syncthreads();
  const int total = s_base[a.C];
  int32_t* erow = a.exp_idx + (long)row * a.E;
  for (int j = total + tid; j < a.E; j += kThreads) erow[j] = -1;
  const int n = *a.n_dev;
  const int n0 = *a.n0_dev;
  const float* srow = a.S + (long)row * a.s_stride;
  for (int c = wave; c < a.C; c += kWaves) {
    const int q = s_q[c];
    if (q <= 0) continue;
    const int base = s_base[c];
    const int limit = min(q, a.E - base);
    if (limit <= 0) continue;
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
    if (mb.size() <= 64 * KREG && q <= QREG)
      topq_extract(mb, srow, q, erow + base, limit, lane);
    else
      topq_radix(mb, srow, q, erow + base, limit, lane, s_hist[wave]);
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
  hipLaunchKernelGGL(topq_kernel, dim3(rows), dim3(kThreads), 0, (hipStream_t)stream, a);
  return OA_LAUNCH_STATUS();
}
