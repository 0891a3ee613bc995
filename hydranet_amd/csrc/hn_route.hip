// MoE routing and token dispatch kernels (gfx950).
//
//  * router logits   : TopKRouter.gate (model/router.py:102, fp16 Linear, logits
//                      rounded to fp16 then .float()) and GLM4SigmoidRouter
//                      (model/glm4.py:279, fp32 F.linear).
//  * top-k           : mode 0 = Mixtral softmax over the selected logits and
//                      renormalisation (model/router.py:109-120);
//                      mode 1 = GLM sigmoid, top-k, normalise with +eps, scale
//                      (model/glm4.py:282-309), plus an optional per-expert
//                      selection bias (scores + bias pick the experts, the
//                      unbiased scores weight them).
//                      Ties go to the lower expert index.  exp() is evaluated
//                      in double and rounded once to fp32, so the fp32 scores
//                      are reproducible on any host.
//  * permute         : stable counting sort of the flattened [T*k] assignments
//                      by expert id, ties in assignment order.  This is the
//                      order of torch.where(flat_indices == e) row-major in
//                      MixtralMoELayer.forward (model/mixtral.py:327-338) over
//                      unique() experts in ascending order (:296).
//  * unpermute       : out[t] = sum over the token's experts, in ascending
//                      expert order, of fp16(y * w), accumulated in fp16 as
//                      output.index_add_ does on an fp16 buffer
//                      (model/mixtral.py:365-368); optional fp16 "shared"
//                      addend as in GLM4MoELayer (model/glm4.py:473).
#include "hn_common.h"

namespace {

constexpr int kPermThreads = 1024;
constexpr int kPermWaves = kPermThreads / 64;
constexpr int kMaxExperts = 256;
constexpr int kMaxTopK = 16;

template <typename TW>
__device__ __forceinline__ void load8f(const TW* p, float out[8]);
template <>
__device__ __forceinline__ void load8f<h16>(const h16* p, float out[8]) {
  const half8_t v = *reinterpret_cast<const half8_t*>(p);
#pragma unroll
  for (int j = 0; j < 8; ++j) out[j] = (float)v[j];
}
template <>
__device__ __forceinline__ void load8f<float>(const float* p, float out[8]) {
  const float4_t a = *reinterpret_cast<const float4_t*>(p);
  const float4_t b = *reinterpret_cast<const float4_t*>(p + 4);
#pragma unroll
  for (int j = 0; j < 4; ++j) { out[j] = a[j]; out[4 + j] = b[j]; }
}

// One wave per (token, expert) dot product of length H; fp32 accumulation.
template <typename TW, bool ROUND16>
__global__ __launch_bounds__(256) void router_logits_kernel(const h16* __restrict__ h, long ld_h,
                                                            const TW* __restrict__ w, long ld_w,
                                                            float* __restrict__ logits, int T,
                                                            int E, int H) {
  const int lane = threadIdx.x & 63;
  const long wid = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wid >= (long)T * E) return;
  const int t = (int)(wid / E);
  const int e = (int)(wid - (long)t * E);
  const h16* hr = h + (long)t * ld_h;
  const TW* wr = w + (long)e * ld_w;
  float acc = 0.f;
  for (int k = lane * 8; k < H; k += 512) {
    float a[8], b[8];
    load8f<h16>(hr + k, a);
    load8f<TW>(wr + k, b);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc = __builtin_fmaf(a[j], b[j], acc);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (lane == 0) logits[(long)t * E + e] = ROUND16 ? (float)(h16)acc : acc;
}

__device__ __forceinline__ float sigmoid_f32(float l) {
  return (float)(1.0 / (1.0 + exp(-(double)l)));
}

// One thread per token.
__global__ __launch_bounds__(256) void router_topk_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, int T, int E, int k,
    int mode, float eps, float scaling, int* __restrict__ idx_out, h16* __restrict__ w_out) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= T) return;
  const float* l = logits + (long)t * E;
  float key[kMaxTopK];
  int sel[kMaxTopK];
  int n = 0;
  for (int e = 0; e < E; ++e) {
    float v = l[e];
    if (mode == 1) {
      v = sigmoid_f32(v);
      if (bias) v = v + bias[e];
    }
    // insert if strictly greater than the current k-th (ties keep lower index)
    if (n < k || v > key[n - 1]) {
      int p = (n < k) ? n : k - 1;
      while (p > 0 && v > key[p - 1]) {
        key[p] = key[p - 1];
        sel[p] = sel[p - 1];
        --p;
      }
      key[p] = v;
      sel[p] = e;
      if (n < k) ++n;
    }
  }
  float wt[kMaxTopK];
  if (mode == 0) {
    // softmax over the selected logits (fp32 result per element), then
    // divide by the fp32 sum (model/router.py:114-117)
    const double mx = (double)l[sel[0]];
    double z = 0.0;
    for (int i = 0; i < n; ++i) z += exp((double)l[sel[i]] - mx);
    float s = 0.f;
    for (int i = 0; i < n; ++i) {
      wt[i] = (float)(exp((double)l[sel[i]] - mx) / z);
      s += wt[i];
    }
    for (int i = 0; i < n; ++i) wt[i] = wt[i] / s;
  } else {
    float s = 0.f;
    for (int i = 0; i < n; ++i) {
      wt[i] = sigmoid_f32(l[sel[i]]);
      s += wt[i];
    }
    const float d = s + eps;
    for (int i = 0; i < n; ++i) wt[i] = (wt[i] / d) * scaling;
  }
  for (int i = 0; i < k; ++i) {
    idx_out[(long)t * k + i] = (i < n) ? sel[i] : -1;
    w_out[(long)t * k + i] = (i < n) ? (h16)wt[i] : (h16)0.0f;
  }
}

// Single-workgroup stable counting sort.  Entries outside [0, E) are ignored
// (they get no position; inv[j] = -1).
__global__ __launch_bounds__(kPermThreads) void moe_permute_kernel(
    const int* __restrict__ idx, int n, int E, int* __restrict__ offsets,
    int* __restrict__ perm, int* __restrict__ inv, int* __restrict__ active,
    int* __restrict__ n_active) {
  __shared__ int cnt[kMaxExperts];
  __shared__ int off[kMaxExperts];
  __shared__ int running[kMaxExperts];
  __shared__ int wtab[kPermWaves][kMaxExperts];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  for (int e = tid; e < kMaxExperts; e += kPermThreads) {
    cnt[e] = 0;
    running[e] = 0;
  }
  for (int i = tid; i < kPermWaves * kMaxExperts; i += kPermThreads) (&wtab[0][0])[i] = 0;
  __syncthreads();
  for (int j = tid; j < n; j += kPermThreads) {
    const int e = idx[j];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int acc = 0, na = 0;
    for (int e = 0; e < E; ++e) {
      off[e] = acc;
      offsets[e] = acc;
      if (cnt[e] > 0) active[na++] = e;
      acc += cnt[e];
    }
    offsets[E] = acc;
    *n_active = na;
  }
  __syncthreads();
  for (int base = 0; base < n; base += kPermThreads) {
    const int j = base + tid;
    int e = (j < n) ? idx[j] : -1;
    if (e < 0 || e >= E) e = -1;
    // rank among earlier lanes of this wave with the same expert
    int rank = 0;
    for (int l2 = 0; l2 < 64; ++l2) {
      const int e2 = __shfl(e, l2, 64);
      rank += (l2 < lane && e2 == e) ? 1 : 0;
    }
    if (e >= 0) atomicAdd(&wtab[wave][e], 1);
    __syncthreads();
    if (e >= 0) {
      int before = 0;
      for (int w2 = 0; w2 < wave; ++w2) before += wtab[w2][e];
      const int pos = off[e] + running[e] + before + rank;
      perm[pos] = j;
      inv[j] = pos;
    } else if (j < n) {
      inv[j] = -1;
    }
    __syncthreads();
    for (int e2 = tid; e2 < E; e2 += kPermThreads) {
      int s = 0;
      for (int w2 = 0; w2 < kPermWaves; ++w2) {
        s += wtab[w2][e2];
        wtab[w2][e2] = 0;
      }
      running[e2] += s;
    }
    __syncthreads();
  }
}

// x_perm[p] = x[perm[p] / k]
__global__ __launch_bounds__(256) void moe_gather_kernel(const h16* __restrict__ x, long ld_x,
                                                         const int* __restrict__ perm, int k,
                                                         const int* __restrict__ offsets, int E,
                                                         h16* __restrict__ xp, long ld_p, int H) {
  const int p = blockIdx.x;
  if (p >= offsets[E]) return;
  const int t = perm[p] / k;
  const h16* src = x + (long)t * ld_x;
  h16* dst = xp + (long)p * ld_p;
  for (int c = threadIdx.x * 8; c < H; c += blockDim.x * 8)
    *reinterpret_cast<half8_t*>(dst + c) = *reinterpret_cast<const half8_t*>(src + c);
}

// One workgroup per token; each thread owns 8 consecutive columns.
__global__ __launch_bounds__(256) void moe_unpermute_kernel(
    const h16* __restrict__ y, long ld_y, const int* __restrict__ inv,
    const int* __restrict__ idx, const h16* __restrict__ w, int k, const h16* __restrict__ shared,
    long ld_sh, h16* __restrict__ out, long ld_o, int H) {
  const int t = blockIdx.x;
  int pos[kMaxTopK];
  int ex[kMaxTopK];
  float wt[kMaxTopK];
  int n = 0;
  for (int s = 0; s < k; ++s) {
    const int j = t * k + s;
    const int p = inv[j];
    if (p < 0) continue;
    const int e = idx[j];
    // insertion by expert id (ascending): the reference visits experts in
    // unique() order and accumulates into an fp16 buffer
    int q = n;
    while (q > 0 && ex[q - 1] > e) {
      ex[q] = ex[q - 1];
      pos[q] = pos[q - 1];
      wt[q] = wt[q - 1];
      --q;
    }
    ex[q] = e;
    pos[q] = p;
    wt[q] = (float)w[j];
    ++n;
  }
  for (int c = threadIdx.x * 8; c < H; c += blockDim.x * 8) {
    half8_t acc = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int s = 0; s < n; ++s) {
      const half8_t v = *reinterpret_cast<const half8_t*>(y + (long)pos[s] * ld_y + c);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const h16 prod = (h16)((float)v[j] * wt[s]);
        acc[j] = (h16)((float)acc[j] + (float)prod);
      }
    }
    if (shared) {
      const half8_t sv = *reinterpret_cast<const half8_t*>(shared + (long)t * ld_sh + c);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = (h16)((float)sv[j] + (float)acc[j]);
    }
    *reinterpret_cast<half8_t*>(out + (long)t * ld_o + c) = acc;
  }
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

// logits[T, E] fp32.  w_dtype: 0 = fp16 gate (logits rounded to fp16, Mixtral),
// 1 = fp32 weight (fp32 logits, GLM).
extern "C" int hn_router_logits(const void* h, long ld_h, const void* w, long ld_w, int w_dtype,
                                void* logits, long T, long E, long H, void* stream) {
  HN_ARG_CHECK(T >= 0 && E > 0 && H > 0, "hn_router_logits: bad dims");
  HN_ARG_CHECK(H % 8 == 0 && ld_h % 8 == 0 && al16(h), "hn_router_logits: h rows must be "
               "16-byte aligned with H %% 8 == 0");
  HN_ARG_CHECK(al16(w) && (w_dtype == 0 ? ld_w % 8 == 0 : ld_w % 4 == 0),
               "hn_router_logits: weight rows must be 16-byte aligned");
  if (T == 0) return 0;
  const long waves = T * E;
  dim3 grid(hn_cdiv(waves, 4)), block(256);
  hipStream_t s = (hipStream_t)stream;
  if (w_dtype == 0)
    hipLaunchKernelGGL((router_logits_kernel<h16, true>), grid, block, 0, s, (const h16*)h, ld_h,
                       (const h16*)w, ld_w, (float*)logits, (int)T, (int)E, (int)H);
  else
    hipLaunchKernelGGL((router_logits_kernel<float, false>), grid, block, 0, s, (const h16*)h,
                       ld_h, (const float*)w, ld_w, (float*)logits, (int)T, (int)E, (int)H);
  HN_LAUNCH_CHECK("hn_router_logits");
  return 0;
}

// mode 0: softmax top-k (Mixtral); mode 1: sigmoid top-k (GLM), bias may be null.
extern "C" int hn_router_topk(const void* logits, const void* bias, long T, long E, long k,
                              int mode, float eps, float scaling, int* idx_out, void* w_out,
                              void* stream) {
  HN_ARG_CHECK(T >= 0 && E > 0 && k > 0 && k <= kMaxTopK && k <= E,
               "hn_router_topk: need 0 < k <= min(E, %d)", kMaxTopK);
  HN_ARG_CHECK(mode == 0 || mode == 1, "hn_router_topk: mode must be 0 or 1");
  if (T == 0) return 0;
  hipLaunchKernelGGL(router_topk_kernel, dim3(hn_cdiv(T, 256)), dim3(256), 0, (hipStream_t)stream,
                     (const float*)logits, (const float*)bias, (int)T, (int)E, (int)k, mode, eps,
                     scaling, idx_out, (h16*)w_out);
  HN_LAUNCH_CHECK("hn_router_topk");
  return 0;
}

extern "C" int hn_moe_permute(const int* idx, long T, long k, long E, int* offsets, int* perm,
                              int* inv, int* active, int* n_active, void* stream) {
  HN_ARG_CHECK(T >= 0 && k > 0 && E > 0 && E <= kMaxExperts,
               "hn_moe_permute: need 0 < E <= %d", kMaxExperts);
  HN_ARG_CHECK(T * k < (1L << 30), "hn_moe_permute: too many assignments");
  hipLaunchKernelGGL(moe_permute_kernel, dim3(1), dim3(kPermThreads), 0, (hipStream_t)stream,
                     idx, (int)(T * k), (int)E, offsets, perm, inv, active, n_active);
  HN_LAUNCH_CHECK("hn_moe_permute");
  return 0;
}

// rows = T*k upper bound of permuted rows (grid size); rows past offsets[E] exit.
extern "C" int hn_moe_gather(const void* x, long ld_x, const int* perm, long k,
                             const int* offsets, long E, void* x_perm, long ld_p, long rows,
                             long H, void* stream) {
  HN_ARG_CHECK(H % 8 == 0 && al16(x) && al16(x_perm) && ld_x % 8 == 0 && ld_p % 8 == 0,
               "hn_moe_gather: rows must be 16-byte aligned");
  if (rows <= 0) return 0;
  hipLaunchKernelGGL(moe_gather_kernel, dim3((unsigned)rows), dim3(256), 0, (hipStream_t)stream,
                     (const h16*)x, ld_x, perm, (int)k, offsets, (int)E, (h16*)x_perm, ld_p,
                     (int)H);
  HN_LAUNCH_CHECK("hn_moe_gather");
  return 0;
}

extern "C" int hn_moe_unpermute(const void* y_perm, long ld_y, const int* inv, const int* idx,
                                const void* w, long T, long k, const void* shared, long ld_sh,
                                void* out, long ld_o, long H, void* stream) {
  HN_ARG_CHECK(k > 0 && k <= kMaxTopK, "hn_moe_unpermute: k must be in (0, %d]", kMaxTopK);
  HN_ARG_CHECK(H % 8 == 0 && al16(y_perm) && al16(out) && ld_y % 8 == 0 && ld_o % 8 == 0 &&
                   (!shared || (al16(shared) && ld_sh % 8 == 0)),
               "hn_moe_unpermute: rows must be 16-byte aligned");
  if (T <= 0) return 0;
  hipLaunchKernelGGL(moe_unpermute_kernel, dim3((unsigned)T), dim3(256), 0, (hipStream_t)stream,
                     (const h16*)y_perm, ld_y, inv, idx, (const h16*)w, (int)k,
                     (const h16*)shared, ld_sh, (h16*)out, ld_o, (int)H);
  HN_LAUNCH_CHECK("hn_moe_unpermute");
  return 0;
}
