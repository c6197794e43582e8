// OpenAttention.flash on gfx950: one online softmax over three streams per query-head row
//   P1 selected tokens  (sink, local, top-k)   -- token indices, -1 = padding
//   P2 expanded tokens  (ErrorGate quotas)      -- token indices, -1 = padding
//   P3 cluster proxies  key kbar_b, value vbar_b, logit s*q.kbar_b + ln n_b (-inf = no proxy)
//
// Mirrors the operator surface of inference/methods_eager.py:161-172 (ours_flash, proxies per
// query-head row) and triton_expand_decode.py:139-165 (decode_expand_attention, proxies per KV
// head).  Kernel semantics follow methods_eager.py:91-158 / triton_expand_decode.py:31-136:
// z = s*log2e*(q.k); p = exp2(z - m); out = acc / l, and out = 0 when no entry is valid.
//
// Work decomposition (not a translation of the Triton program-per-row loop): a 256-thread
// workgroup owns one row (or one chunk of a row in split mode).  Its 16 lane groups of 16
// lanes each stream their own items; a lane holds 8 of the 128 dims, so one item costs one
// 16-byte K load and one 16-byte V load per lane and a 4-step shuffle reduction.  Each lane
// group keeps its own (m, l, acc) and the 16 partial softmaxes are merged once at the end
// in a fixed order.
#include "oa_common.h"

#include <mutex>

namespace {

constexpr int kThreads = 256;
constexpr int kGroups = kThreads / 16;
constexpr float kLog2e = 1.4426950408889634f;

struct FlashArgs {
  const uint16_t* q; long q_stride;
  const uint16_t* k; const uint16_t* v; long kv_sb; long kv_ss;
  const int32_t* sel; long sel_stride; int n_sel;
  const int32_t* exq; long exp_stride; int n_exp;
  const void* kbar; const void* vbar; long kb_sb; long kb_sn; int proxy_per_kv;
  const float* logn; long logn_stride; int n_bins;
  void* out; long out_stride; int out_f32;
  int R; int G; float sm_scale;
  int n_split; int chunk;
  float* ws_m; float* ws_l; float* ws_acc;   // split partials: (R*n_split), (R*n_split), (R*n_split, D)
};

template <typename PT>
__device__ __forceinline__ void load_proxy8(const PT* p, float* x);

template <>
__device__ __forceinline__ void load_proxy8<uint16_t>(const uint16_t* p, float* x) {
  uint4 w = *reinterpret_cast<const uint4*>(p);
  oa::unpack8(w, x);
}
template <>
__device__ __forceinline__ void load_proxy8<float>(const float* p, float* x) {
  float4 a = *reinterpret_cast<const float4*>(p);
  float4 b = *reinterpret_cast<const float4*>(p + 4);
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}

template <typename PT>
__global__ void __launch_bounds__(kThreads) flash_decode_kernel(FlashArgs a) {
  const int row = blockIdx.x;
  const int split = blockIdx.y;
  const int tid = threadIdx.x;
  const int grp = tid >> 4;          // lane group within the workgroup (0..15)
  const int sub = tid & 15;          // lane inside the group: dims [8*sub, 8*sub+8)
  const int kvh = row / a.G;
  const int d0 = sub * 8;

  float qv[8];
  {
    uint4 w = *reinterpret_cast<const uint4*>(a.q + (long)row * a.q_stride + d0);
    oa::unpack8(w, qv);
  }
  const int T = a.n_sel + a.n_exp + a.n_bins;
  const int t_begin = split * a.chunk;
  const int t_end = min(T, t_begin + a.chunk);
  const float qk2 = a.sm_scale * kLog2e;

  const uint16_t* kbase = a.k + (long)kvh * a.kv_sb;
  const uint16_t* vbase = a.v + (long)kvh * a.kv_sb;
  const long prow = a.proxy_per_kv ? (long)kvh : (long)row;
  const PT* kb = reinterpret_cast<const PT*>(a.kbar) + prow * a.kb_sb;
  const PT* vb = reinterpret_cast<const PT*>(a.vbar) + prow * a.kb_sb;

  float m = -INFINITY, l = 0.f;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;

  for (int t = t_begin + grp; t < t_end; t += kGroups) {
    float kx[8], vx[8];
    bool valid;
    float bias = 0.f;
    float zscale;
    if (t < a.n_sel + a.n_exp) {
      int tok = (t < a.n_sel) ? a.sel[(long)row * a.sel_stride + t]
                              : a.exq[(long)row * a.exp_stride + (t - a.n_sel)];
      valid = tok >= 0;
      long off = (long)(valid ? tok : 0) * a.kv_ss + d0;
      uint4 kw = *reinterpret_cast<const uint4*>(kbase + off);
      uint4 vw = *reinterpret_cast<const uint4*>(vbase + off);
      oa::unpack8(kw, kx);
      oa::unpack8(vw, vx);
      zscale = qk2;
    } else {
      int b = t - a.n_sel - a.n_exp;
      float ln = a.logn[(long)row * a.logn_stride + b];
      valid = ln > -INFINITY;           // also false for NaN
      long off = (long)b * a.kb_sn + d0;
      load_proxy8<PT>(kb + off, kx);
      load_proxy8<PT>(vb + off, vx);
      bias = valid ? ln : 0.f;
      zscale = a.sm_scale;
    }
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) part = fmaf(qv[i], kx[i], part);
    float dot = oa::group16_sum(part);
    float z = (t < a.n_sel + a.n_exp) ? dot * zscale : (dot * zscale + bias) * kLog2e;
    if (valid) {
      float m_new = fmaxf(m, z);
      float alpha = exp2f(m - m_new);
      float p = exp2f(z - m_new);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = fmaf(p, vx[i], acc[i] * alpha);
      l = fmaf(l, alpha, p);
      m = m_new;
    }
  }

  // merge the 16 lane-group states in a fixed order
  __shared__ float s_m[kGroups], s_l[kGroups];
  __shared__ float s_acc[kGroups][OA_D];
  if (sub == 0) { s_m[grp] = m; s_l[grp] = l; }
#pragma unroll
  for (int i = 0; i < 8; ++i) s_acc[grp][d0 + i] = acc[i];
  __syncthreads();
  if (tid < OA_D) {
    float M = -INFINITY;
    for (int g = 0; g < kGroups; ++g) M = fmaxf(M, s_m[g]);
    float L = 0.f, A = 0.f;
    if (M > -INFINITY) {
      for (int g = 0; g < kGroups; ++g) {
        if (s_m[g] > -INFINITY) {
          float w = exp2f(s_m[g] - M);
          L = fmaf(s_l[g], w, L);
          A = fmaf(s_acc[g][tid], w, A);
        }
      }
    }
    if (a.n_split == 1) {
      float o = (L > 0.f) ? A / L : 0.f;
      oa::store_out(a.out, a.out_f32, (long)row * a.out_stride + tid, o);
    } else {
      long pr = (long)row * a.n_split + split;
      if (tid == 0) { a.ws_m[pr] = M; a.ws_l[pr] = L; }
      a.ws_acc[pr * OA_D + tid] = A;
    }
  }
}

__global__ void __launch_bounds__(OA_D) flash_combine_kernel(const float* ws_m, const float* ws_l,
                                                             const float* ws_acc, int n_split,
                                                             void* out, long out_stride,
                                                             int out_f32) {
  const int row = blockIdx.x;
  const int d = threadIdx.x;
  const long base = (long)row * n_split;
  float M = -INFINITY;
  for (int s = 0; s < n_split; ++s) M = fmaxf(M, ws_m[base + s]);
  float L = 0.f, A = 0.f;
  if (M > -INFINITY) {
    for (int s = 0; s < n_split; ++s) {
      float ms = ws_m[base + s];
      if (ms > -INFINITY) {
        float w = exp2f(ms - M);
        L = fmaf(ws_l[base + s], w, L);
        A = fmaf(ws_acc[(base + s) * OA_D + d], w, A);
      }
    }
  }
  float o = (L > 0.f) ? A / L : 0.f;
  oa::store_out(out, out_f32, (long)row * out_stride + d, o);
}

}  // namespace

namespace {

// Launches the flash kernel (plus the combine when n_split > 1) with the split partials in
// ws_m, ws_l (rows * n_split) and ws_acc (rows * n_split * 128); the arguments are checked.
int flash_launch(const void* q, long q_stride, const void* k, const void* v, long kv_stride_b,
                 long kv_stride_s, const int32_t* sel, long sel_stride, int n_sel,
                 const int32_t* exp_idx, long exp_stride, int n_exp, const void* kbar,
                 const void* vbar, long kbar_stride_b, long kbar_stride_n, int kbar_is_f32,
                 int proxy_per_kv, const float* log_n, long log_n_stride, int n_bins, void* out,
                 long out_stride, int out_is_f32, int rows, int kv_rows, float sm_scale,
                 int n_split, float* ws_m, float* ws_l, float* ws_acc, hipStream_t s) {
  FlashArgs a;
  a.q = (const uint16_t*)q; a.q_stride = q_stride;
  a.k = (const uint16_t*)k; a.v = (const uint16_t*)v; a.kv_sb = kv_stride_b; a.kv_ss = kv_stride_s;
  a.sel = sel; a.sel_stride = sel_stride; a.n_sel = n_sel;
  a.exq = exp_idx; a.exp_stride = exp_stride; a.n_exp = n_exp;
  a.kbar = kbar; a.vbar = vbar; a.kb_sb = kbar_stride_b; a.kb_sn = kbar_stride_n;
  a.proxy_per_kv = proxy_per_kv;
  a.logn = log_n; a.logn_stride = log_n_stride; a.n_bins = n_bins;
  a.out = out; a.out_stride = out_stride; a.out_f32 = out_is_f32 ? 1 : 0;
  a.R = rows; a.G = rows / kv_rows; a.sm_scale = sm_scale;
  a.n_split = n_split;
  const int T = n_sel + n_exp + n_bins;
  int chunk = (T + n_split - 1) / n_split;
  chunk = ((chunk + 15) / 16) * 16;
  if (chunk < 16) chunk = 16;
  a.chunk = chunk;
  a.ws_m = ws_m; a.ws_l = ws_l; a.ws_acc = ws_acc;
  dim3 grid(rows, n_split);
  if (kbar_is_f32)
    hipLaunchKernelGGL(flash_decode_kernel<float>, grid, dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL(flash_decode_kernel<uint16_t>, grid, dim3(kThreads), 0, s, a);
  int st = OA_LAUNCH_STATUS();
  if (st || n_split == 1) return st;
  hipLaunchKernelGGL(flash_combine_kernel, dim3(rows), dim3(OA_D), 0, s, ws_m, ws_l, ws_acc,
                     n_split, out, out_stride, a.out_f32);
  return OA_LAUNCH_STATUS();
}

int flash_check(int rows, int kv_rows, int head_dim, int n_sel, int n_exp, int n_bins,
                int n_split, const void* kbar, const void* vbar, const float* log_n) {
  if (head_dim != OA_D || rows <= 0 || kv_rows <= 0 || rows % kv_rows != 0) return OA_EINVAL;
  if (n_sel < 0 || n_exp < 0 || n_bins < 0 || n_split < 1) return OA_EINVAL;
  if (n_bins > 0 && (!kbar || !vbar || !log_n)) return OA_EINVAL;
  return 0;
}

// ---- no-allocation variant: the split partials live in a fixed device array ----------------
// Each GPU holds its own copy of `scratch` for the life of the process.  Host code never uses
// the array's name as an address: the device address comes from hipGetSymbolAddress, taken
// once per device (with that device current) on the first call there, and kept in
// g_scratch_dev.  Every call on one GPU shares that GPU's array, so calls that overlap on one
// GPU (concurrent streams) race on it.  Each (row, split) slot is written in full by the flash
// kernel before the combine reads it, so nothing needs clearing between calls.
constexpr long kScratchFloats = 1L << 20;          // 4 MiB per GPU
constexpr int kMaxDevices = 64;
static __device__ __align__(256) float scratch[kScratchFloats];
float* g_scratch_dev[kMaxDevices] = {};
std::mutex g_scratch_mu;

int scratch_address(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return OA_EINVAL;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return (int)hipErrorInvalidSymbol;
    g_scratch_dev[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_dev[dev];
  return 0;
}

}  // namespace

extern "C" int oa_flash_decode(const void* q, long q_stride,
                               const void* k, const void* v, long kv_stride_b, long kv_stride_s,
                               const int32_t* sel, long sel_stride, int n_sel,
                               const int32_t* exp_idx, long exp_stride, int n_exp,
                               const void* kbar, const void* vbar, long kbar_stride_b,
                               long kbar_stride_n, int kbar_is_f32, int proxy_per_kv,
                               const float* log_n, long log_n_stride, int n_bins,
                               void* out, long out_stride, int out_is_f32,
                               int rows, int kv_rows, int head_dim, float sm_scale,
                               int n_split, float* ws_m, float* ws_l, float* ws_acc,
                               void* stream) {
  int st = flash_check(rows, kv_rows, head_dim, n_sel, n_exp, n_bins, n_split, kbar, vbar, log_n);
  if (st) return st;
  if (n_split > 1 && (!ws_m || !ws_l || !ws_acc)) return OA_EINVAL;
  return flash_launch(q, q_stride, k, v, kv_stride_b, kv_stride_s, sel, sel_stride, n_sel,
                      exp_idx, exp_stride, n_exp, kbar, vbar, kbar_stride_b, kbar_stride_n,
                      kbar_is_f32, proxy_per_kv, log_n, log_n_stride, n_bins, out, out_stride,
                      out_is_f32, rows, kv_rows, sm_scale, n_split, ws_m, ws_l, ws_acc,
                      (hipStream_t)stream);
}

extern "C" int oa_flash_decode_noalloc(const void* q, long q_stride, const void* k, const void* v,
                                       long kv_stride_b, long kv_stride_s, const int32_t* sel,
                                       long sel_stride, int n_sel, const int32_t* exp_idx,
                                       long exp_stride, int n_exp, const void* kbar,
                                       const void* vbar, long kbar_stride_b, long kbar_stride_n,
                                       int kbar_is_f32, int proxy_per_kv, const float* log_n,
                                       long log_n_stride, int n_bins, void* out, long out_stride,
                                       int out_is_f32, int rows, int kv_rows, int head_dim,
                                       float sm_scale, int n_split, void* stream) {
  int st = flash_check(rows, kv_rows, head_dim, n_sel, n_exp, n_bins, n_split, kbar, vbar, log_n);
  if (st) return st;
  const long slots = (long)rows * (long)n_split;
  if (slots * (OA_D + 2) > kScratchFloats) return OA_ENOSPC;
  float* ws_acc = nullptr;
  float* ws_m = nullptr;
  float* ws_l = nullptr;
  if (n_split > 1) {
    float* base = nullptr;
    st = scratch_address(&base);
    if (st) return st;
    ws_acc = base;                       // slots * 128, 512-byte aligned rows
    ws_m = base + slots * OA_D;
    ws_l = ws_m + slots;
  }
  return flash_launch(q, q_stride, k, v, kv_stride_b, kv_stride_s, sel, sel_stride, n_sel,
                      exp_idx, exp_stride, n_exp, kbar, vbar, kbar_stride_b, kbar_stride_n,
                      kbar_is_f32, proxy_per_kv, log_n, log_n_stride, n_bins, out, out_stride,
                      out_is_f32, rows, kv_rows, sm_scale, n_split, ws_m, ws_l, ws_acc,
                      (hipStream_t)stream);
}
