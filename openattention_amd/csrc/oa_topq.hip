// Within-cluster top-q: for every (row, cluster) with quota q_c > 0, the q_c tail members of the
// cluster with the highest QGS score (ties to the lower position) become exact reads.
//
// Reference semantics: the per-token rank within its bin by the selector score
// (multibin.py:2522-2558, trunc_keep = rank < quota) with the deployed tie order of
// ours_graph.py:93-135 / ours_fused.py:228-282 (score, then members before generated tokens,
// then position -- i.e. position order, since every generated token follows the prefix).
// Selected, sink, local and unwritten positions carry a -inf score and never qualify.
//
// exp_idx row layout: cluster c owns slots [base_c, base_c + q_c), base_c = sum_{c'<c} q_c';
// a segment lists its chosen members in position order; slots past sum q are -1.
//
// gfx950 decomposition.  About 40 of 64 clusters carry a quota and their members cover most
// of a row, so the row is streamed once instead of gathering member scores:
//   topq_chunk: grid (chunks of 8192 positions, rows).  A workgroup copies its chunk's scores
//     and 8-bit cluster ids into LDS with coalesced loads, then finds, for every cluster at
//     once, the exact top-min(q_c, members) of the chunk by an MSB-first radix select over the
//     unique 48-bit key (order-preserving score key, then the complement of the position inside
//     the chunk): 12 passes of 4-bit digits with per-cluster LDS histograms and per-cluster
//     digit searches.  Candidates go to the caller's workspace as 64-bit keys
//     (score key << 32 | ~position), q_c slots per cluster per chunk.
//   topq_merge: one workgroup per row; each wave takes clusters round-robin and extracts the
//     q_c best candidate keys over the chunks with wave butterflies, then writes the winners in
//     position order.
#include "oa_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxC = 256;
constexpr int kMaxE = 4096;
constexpr int kChunk = 8192;
constexpr int kDigits = 16;     // 4-bit radix digits
constexpr int kPasses = 12;     // 48-bit keys
constexpr int KREG = 16;        // candidate slots per lane in the merge
constexpr unsigned kNegInfKey = 0x007fffffu;   // float_key(-inf)

// dynamic LDS layout of the chunk kernel
struct ChunkLds {
  uint32_t key[kChunk];
  uint8_t cid[kChunk];
};

__global__ void __launch_bounds__(kThreads) topq_chunk_kernel(
    const float* __restrict__ S, long s_stride, const uint8_t* __restrict__ asg8, long a_stride,
    const float* __restrict__ quota, int C, int E, const int* __restrict__ n_dev,
    unsigned long long* __restrict__ cand, int nchunks) {
  extern __shared__ unsigned long long dyn[];
  ChunkLds& L = *reinterpret_cast<ChunkLds*>(dyn);
  // per-cluster arrays after the chunk copy: hist (C x 16), pref, krem, q, base, fill, staging
  int* s_hist = reinterpret_cast<int*>(reinterpret_cast<char*>(dyn) + sizeof(ChunkLds));
  unsigned long long* s_pref = reinterpret_cast<unsigned long long*>(s_hist + C * kDigits);
  int* s_krem = reinterpret_cast<int*>(s_pref + C);
  int* s_q = s_krem + C;
  int* s_base = s_q + C;
  int* s_fill = s_base + C + 1;
  unsigned long long* s_stage = reinterpret_cast<unsigned long long*>(
      (reinterpret_cast<uintptr_t>(s_fill + C) + 7) & ~static_cast<uintptr_t>(7));
  const int chunk = blockIdx.x;
  const int row = blockIdx.y;
  const int tid = threadIdx.x;
  const int n = *n_dev;
  const int p0 = chunk * kChunk;
  const int len = max(0, min(kChunk, n - p0));
  unsigned long long* out = cand + ((long)row * nchunks + chunk) * E;
  if (tid < 64) {
    int v[4], loc = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid * 4 + i;
      v[i] = c < C ? (int)quota[(long)row * C + c] : 0;
      loc += v[i];
    }
    int incl = loc;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int t = __shfl_up(incl, off, 64);
      if (tid >= off) incl += t;
    }
    int run = incl - loc;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid * 4 + i;
      if (c < C) { s_q[c] = v[i]; s_base[c] = run; }
      run += v[i];
    }
    if (tid == 63) s_base[C] = incl;
  }
  for (int i = tid; i < len; i += kThreads) {
    L.key[i] = oa::float_key(S[(long)row * s_stride + p0 + i]);
    L.cid[i] = asg8[(long)row * a_stride + p0 + i];
  }
  for (int e = tid; e < C * kDigits; e += kThreads) s_hist[e] = 0;
  for (int c = tid; c < C; c += kThreads) { s_pref[c] = 0ull; s_fill[c] = 0; }
  __syncthreads();
  const int total = min(s_base[C], E);
  for (int j = tid; j < total; j += kThreads) s_stage[j] = 0ull;
  // qualifying members per cluster -> target count min(q, members)
  for (int i = tid; i < len; i += kThreads) {
    const int c = L.cid[i];
    if (c < C && s_q[c] > 0 && L.key[i] > kNegInfKey) atomicAdd(&s_hist[c * kDigits], 1);
  }
  __syncthreads();
  for (int c = tid; c < C; c += kThreads) {
    s_krem[c] = min(s_q[c], s_hist[c * kDigits]);
    s_hist[c * kDigits] = 0;
  }
  __syncthreads();
  // radix select of the s_krem[c]-th largest 48-bit key of every cluster at once
  for (int pass = 0; pass < kPasses; ++pass) {
    const int shift = 44 - 4 * pass;
    for (int i = tid; i < len; i += kThreads) {
      const int c = L.cid[i];
      if (c >= C || s_krem[c] <= 0 || L.key[i] <= kNegInfKey) continue;
      const unsigned long long k48 = ((unsigned long long)L.key[i] << 16) | (0xffffu - (unsigned)i);
      if ((k48 >> (shift + 4)) == (s_pref[c] >> (shift + 4)))
        atomicAdd(&s_hist[c * kDigits + (int)((k48 >> shift) & 15u)], 1);
    }
    __syncthreads();
    for (int c = tid; c < C; c += kThreads) {
      const int k = s_krem[c];
      if (k > 0) {
        int cum = 0, digit = 0, nk = k;
        for (int d = kDigits - 1; d >= 0; --d) {
          const int h = s_hist[c * kDigits + d];
          if (cum + h >= k) { digit = d; nk = k - cum; break; }
          cum += h;
        }
        s_pref[c] |= ((unsigned long long)digit) << shift;
        s_krem[c] = nk;
      }
      for (int d = 0; d < kDigits; ++d) s_hist[c * kDigits + d] = 0;
    }
    __syncthreads();
  }
  // every qualifying key >= the cluster's threshold is a candidate (keys are unique)
  for (int i = tid; i < len; i += kThreads) {
    const int c = L.cid[i];
    if (c >= C || s_q[c] <= 0 || L.key[i] <= kNegInfKey) continue;
    const unsigned long long k48 = ((unsigned long long)L.key[i] << 16) | (0xffffu - (unsigned)i);
    if (k48 >= s_pref[c]) {
      const int slot = atomicAdd(&s_fill[c], 1);
      if (slot < s_q[c] && s_base[c] + slot < total)
        s_stage[s_base[c] + slot] =
            ((unsigned long long)L.key[i] << 32) | (0xffffffffu - (unsigned)(p0 + i));
    }
  }
  __syncthreads();
  // each cluster's candidates in position order (descending complement), then written out
  for (int c = tid; c < C; c += kThreads) {
    const int b = s_base[c];
    const int m = min(min(s_fill[c], s_q[c]), total - b);
    for (int a = 1; a < m; ++a) {
      const unsigned long long x = s_stage[b + a];
      const unsigned xp = 0xffffffffu - (unsigned)(x & 0xffffffffull);
      int j = a - 1;
      while (j >= 0 && (0xffffffffu - (unsigned)(s_stage[b + j] & 0xffffffffull)) > xp) {
        s_stage[b + j + 1] = s_stage[b + j];
        --j;
      }
      s_stage[b + j + 1] = x;
    }
  }
  __syncthreads();
  for (int j = tid; j < total; j += kThreads) out[j] = s_stage[j];
}

size_t chunk_lds_bytes(int C, int E) {
  return sizeof(ChunkLds) + sizeof(int) * C * kDigits + sizeof(unsigned long long) * C +
         sizeof(int) * (4 * C + 2) + 8 + sizeof(unsigned long long) * (size_t)E;
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const unsigned long long o = __shfl_xor(v, m, 64);
    v = o > v ? o : v;
  }
  return v;
}

__device__ __forceinline__ int lanes_below(bool flag, int lane, int* total) {
  const unsigned long long b = __ballot(flag);
  *total = __popcll(b);
  return __popcll(b & ((1ull << lane) - 1ull));
}

// Candidate slot idx (0 <= idx < nchunks*q) of cluster c: chunk idx / q, entry idx % q.  Over
// idx the non-empty candidates appear in ascending position order.
__global__ void __launch_bounds__(kThreads) topq_merge_kernel(
    const unsigned long long* __restrict__ cand, int nchunks, const float* __restrict__ quota,
    int C, int E, int32_t* __restrict__ exp_idx) {
  __shared__ int s_q[kMaxC];
  __shared__ int s_base[kMaxC + 1];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  if (wave == 0) {
    int v[4], loc = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = lane * 4 + i;
      v[i] = c < C ? (int)quota[(long)row * C + c] : 0;
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
      if (c < C) { s_q[c] = v[i]; s_base[c] = run; }
      run += v[i];
    }
    if (lane == 63) s_base[C] = incl;
  }
  __syncthreads();
  const int total = s_base[C];
  int32_t* erow = exp_idx + (long)row * E;
  for (int j = total + tid; j < E; j += kThreads) erow[j] = -1;
  const unsigned long long* crow = cand + (long)row * nchunks * E;
  for (int c = wave; c < C; c += kWaves) {
    const int q = s_q[c];
    if (q <= 0) continue;
    const int base = s_base[c];
    const int limit = min(q, E - base);
    if (limit <= 0) continue;
    const int M = nchunks * q;
    // threshold T = the limit-th largest candidate key (keys are unique, 0 = empty slot)
    unsigned long long T = 0ull;
    if (M <= 64 * KREG) {
      unsigned long long key[KREG];
#pragma unroll
      for (int j = 0; j < KREG; ++j) {
        const int idx = j * 64 + lane;
        key[j] = idx < M ? crow[(long)(idx / q) * E + base + idx % q] : 0ull;
      }
      unsigned taken = 0u;
      for (int t = 0; t < limit; ++t) {
        unsigned long long best = 0ull;
#pragma unroll
        for (int j = 0; j < KREG; ++j)
          if (!((taken >> j) & 1u) && key[j] > best) best = key[j];
        best = wave_max_u64(best);
        if (best == 0ull) break;
        T = best;
#pragma unroll
        for (int j = 0; j < KREG; ++j)
          if (key[j] == best) taken |= 1u << j;
      }
    } else {
      unsigned long long prev = ~0ull;
      for (int t = 0; t < limit; ++t) {
        unsigned long long best = 0ull;
        for (int idx = lane; idx < M; idx += 64) {
          const unsigned long long kk = crow[(long)(idx / q) * E + base + idx % q];
          if (kk < prev && kk > best) best = kk;
        }
        best = wave_max_u64(best);
        if (best == 0ull) break;
        T = best;
        prev = best;
      }
    }
    if (T == 0ull) continue;
    // emit the candidates >= T in slot order = position order
    int run = 0;
    for (int b0 = 0; b0 < M; b0 += 64) {
      const int idx = b0 + lane;
      const unsigned long long kk = idx < M ? crow[(long)(idx / q) * E + base + idx % q] : 0ull;
      const bool take = kk != 0ull && kk >= T;
      int tot;
      const int below = lanes_below(take, lane, &tot);
      if (take && run + below < limit)
        erow[base + run + below] = (int)(0xffffffffu - (unsigned)(kk & 0xffffffffull));
      run += tot;
    }
  }
}

}  // namespace

extern "C" int oa_topq(const float* S, long s_stride, const uint8_t* asg8, long asg8_stride,
                       const float* quota, int rows, int C, int Lmax, int32_t* exp_idx, int E,
                       const int* n_dev, uint64_t* cand, long cand_elems, void* stream) {
  if (rows <= 0 || C <= 0 || C > kMaxC || E < 0 || E > kMaxE || Lmax <= 0) return OA_EINVAL;
  const int nchunks = (Lmax + kChunk - 1) / kChunk;
  if (!cand || cand_elems < (long)rows * nchunks * (E > 0 ? E : 1)) return OA_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  if (E > 0) {
    const size_t lds = chunk_lds_bytes(C, E);
    if (lds > 65536) {
      const hipError_t e = hipFuncSetAttribute((const void*)topq_chunk_kernel,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return (int)e;
    }
    hipLaunchKernelGGL(topq_chunk_kernel, dim3(nchunks, rows), dim3(kThreads), lds, s, S, s_stride,
                       asg8, asg8_stride, quota, C, E, n_dev, (unsigned long long*)cand, nchunks);
    const int st = OA_LAUNCH_STATUS();
    if (st) return st;
  }
  hipLaunchKernelGGL(topq_merge_kernel, dim3(rows), dim3(kThreads), 0, s,
                     (const unsigned long long*)cand, nchunks, quota, C, E, exp_idx);
  return OA_LAUNCH_STATUS();
}
