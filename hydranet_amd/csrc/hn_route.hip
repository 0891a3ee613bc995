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
#include "hn_topk.h"
#include "hn_unpermute.h"

#include <algorithm>

namespace {

constexpr int kPermThreads = 1024;
constexpr int kPermWaves = kPermThreads / 64;
constexpr int kMaxExperts = 256;

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

// One wave's dot product of length H (fp32 accumulation, lane-strided, then a
// butterfly over the wave; every lane returns the sum).
template <typename TW, bool ROUND16>
__device__ __forceinline__ float logit_dot(const h16* hr, const TW* wr, int H, int lane) {
  float acc = 0.f;
#pragma unroll 4
  for (int k = lane * 8; k < H; k += 512) {
    float a[8], b[8];
    load8f<h16>(hr + k, a);
    load8f<TW>(wr + k, b);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc = __builtin_fmaf(a[j], b[j], acc);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  return ROUND16 ? (float)(h16)acc : acc;
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
  const float acc = logit_dot<TW, ROUND16>(h + (long)t * ld_h, w + (long)e * ld_w, H, lane);
  if (lane == 0) logits[(long)t * E + e] = acc;
}

// One wave per token (more than 16 experts) or one thread per token.
// Group-limited selection of GLM4SigmoidRouter (model/glm4.py:285-298), one
// wave per token: the experts' sigmoids (sigmoid_f32, as the top-k) go to
// LDS, lane g < n_group takes the max over its group of E / n_group
// consecutive experts, the topk_group largest group scores are kept (equal
// scores: the lower group), and the row is written back with -inf for every
// expert of the other groups (their sigmoid is then exactly 0, the
// reference's masked score).
__global__ __launch_bounds__(256) void router_group_limit_kernel(
    const float* __restrict__ logits, int T, int E, int n_group, int topk_group,
    float* __restrict__ out) {
  __shared__ float s_sc[4][kMaxExperts];
  __shared__ float s_gs[4][64];
  __shared__ int s_keep[4][64];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wv;
  if (t >= T) return;  // uniform per wave; no block-wide barrier below
  const float* l = logits + (long)t * E;
  for (int e = lane; e < E; e += 64) s_sc[wv][e] = sigmoid_f32(l[e]);
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  const int gsz = E / n_group;
  float gmax = -__builtin_inff();
  if (lane < n_group)
    for (int j = 0; j < gsz; ++j) gmax = fmaxf(gmax, s_sc[wv][lane * gsz + j]);
  s_gs[wv][lane] = gmax;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  int rank = 0;
  for (int g = 0; g < n_group; ++g) {
    const float o = s_gs[wv][g];
    rank += (o > gmax || (o == gmax && g < lane)) ? 1 : 0;
  }
  s_keep[wv][lane] = (lane < n_group && rank < topk_group) ? 1 : 0;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  for (int e = lane; e < E; e += 64)
    out[(long)t * E + e] = s_keep[wv][e / gsz] ? l[e] : -__builtin_inff();
}

__global__ __launch_bounds__(256) void router_topk_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, int T, int E, int k,
    int mode, float eps, float scaling, int* __restrict__ idx_out, h16* __restrict__ w_out) {
  if (E <= 16) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= T) return;
    topk_small<16>(logits + (long)t * E, bias, E, k, mode, eps, scaling, idx_out + (long)t * k,
                   w_out + (long)t * k);
    return;
  }
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= T) return;
  const TopkBias tb = topk_wave_bias(bias, E, threadIdx.x & 63);
  topk_wave(logits + (long)t * E, tb, E, k, mode, eps, scaling, threadIdx.x & 63,
            idx_out + (long)t * k, w_out + (long)t * k);
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
    // rank among earlier lanes of this wave with the same expert, from nine
    // ballots over the bits of e (E <= 256; -1 sets bit 8); the rank-0 lane
    // of each expert writes the wave's count
    uint64_t same = ~0ull;
#pragma unroll
    for (int b = 0; b < 9; ++b) {
      const uint64_t bal = __ballot((e >> b) & 1);
      same &= ((e >> b) & 1) ? bal : ~bal;
    }
    const int rank = __popcll(same & ((1ull << lane) - 1));
    if (e >= 0 && rank == 0) wtab[wave][e] = __popcll(same);
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

// Workgroup (token, column block): each thread owns 8 consecutive columns
// per pass (blockDim.x * 8 columns per block and pass, gridDim.y blocks
// interleaved over H); the sum is unp_select / unp_cols (hn_unpermute.h).
// KS = 0: y is fp16 [rows, ld_y]; KS > 0: y is given as KS fp32 partial sums
// part[j * ks_stride + row * ld_y] (a K-split down projection), added in
// slice order and rounded to fp16 once: the expert output the unsplit kernel
// would write, up to fp32 summation order.  A shared expert's row, when
// given, is added last: out = fp16(shared + acc).
template <int KS>
__global__ __launch_bounds__(256) void moe_unpermute_kernel(
    const h16* __restrict__ y, const float* __restrict__ part, long ks_stride, long ld_y,
    const int* __restrict__ inv, const int* __restrict__ idx, const h16* __restrict__ w, int k,
    const h16* __restrict__ shared, long ld_sh, h16* __restrict__ out, long ld_o, int H) {
  const int t = blockIdx.x;
  int pos[kMaxTopK];
  float wt[kMaxTopK];
  const int n = unp_select(t, inv, idx, w, k, pos, wt);
  for (int c = (blockIdx.y * blockDim.x + threadIdx.x) * 8; c < H;
       c += gridDim.y * blockDim.x * 8) {
    // the shared expert's row is loaded with the first batch of rows
    half8_t sv = {0, 0, 0, 0, 0, 0, 0, 0};
    if (shared) sv = *reinterpret_cast<const half8_t*>(shared + (long)t * ld_sh + c);
    half8_t acc = unp_cols<KS>(y, part, ks_stride, ld_y, pos, wt, n, c);
    if (shared) {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = (h16)((float)sv[j] + (float)acc[j]);
    }
    *reinterpret_cast<half8_t*>(out + (long)t * ld_o + c) = acc;
  }
}

// Decode routing in one launch.  Every workgroup computes the routing of all
// T tokens into LDS (logits unless given, top-k, the stable order by expert),
// then copies its share of the permuted rows x_perm[p] = h[perm[p] / k];
// workgroup 0 also writes the routing outputs.  Top-k and the order are those
// of router_topk_kernel / moe_permute_kernel.  Logits (LG):
//  * 1, 2, 4: MFMA (fp16 gate, T <= 16 / 32 / 64 tokens, E <= 16, T * E <= 512,
//    H % 512 == 0):
//    each of the 16 waves multiplies one 1/16 slice of H (all its loads in
//    flight together), the 16 partial 16x16 tiles are summed in wave order,
//    then rounded to fp16 (the fp16 Linear of the reference);
//  * 0: one wave per (token, expert) dot product, as router_logits_kernel.
constexpr int kRouteThreads = 1024;
constexpr int kRouteWaves = kRouteThreads / 64;
constexpr int kRouteMaxLogits = 8192;  // T * E
constexpr int kRouteMaxAssign = 1024;  // T * k (one thread per assignment)

template <typename TW, bool ROUND16, int LG, int TK>
__global__ __launch_bounds__(kRouteThreads) void moe_route_kernel(
    const h16* __restrict__ h, long ld_h, const TW* __restrict__ w, long ld_w,
    const float* __restrict__ logits_in, const float* __restrict__ bias, int T, int E, int H,
    int k, int mode, float eps, float scaling, float* __restrict__ logits_out,
    int* __restrict__ idx_out, h16* __restrict__ w_out, int* __restrict__ offsets,
    int* __restrict__ perm, int* __restrict__ inv, int* __restrict__ active,
    int* __restrict__ n_active, long long* __restrict__ usage, h16* __restrict__ x_perm,
    long ld_p) {
  // logits, or the MFMA partial tiles (16 waves x 16 LG tokens x 16 experts)
  __shared__ __align__(16) float s_buf[LG == 4 ? 16 * 64 * 16 : kRouteMaxLogits];
  __shared__ float s_lg[512];               // MFMA logits (T * E <= 512)
  __shared__ int s_sel[kRouteMaxAssign];
  __shared__ h16 s_w[kRouteMaxAssign];
  __shared__ int s_perm[kRouteMaxAssign];
  __shared__ int s_wcnt[kRouteWaves][kMaxExperts];  // per wave, per expert
  __shared__ int s_off[kMaxExperts + 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nw = blockDim.x >> 6;
  const bool lead = blockIdx.x == 0;
  const int n = T * k;
  // the selection bias (E > 16: one wave per token) goes out with the logits
  const TopkBias tb = topk_wave_bias(E > 16 ? bias : nullptr, E, lane);

  for (int i = tid; i < kRouteWaves * kMaxExperts; i += blockDim.x) (&s_wcnt[0][0])[i] = 0;

  // 1. logits
  const float* lg = s_buf;
  if (logits_in) {
    copy_to_lds_f32(logits_in, s_buf, T * E);
  } else if constexpr (LG > 0) {
    const int ksl = H >> 4, kb0 = wave * ksl, steps = ksl >> 5;
    const int tl = lane & 15, kq = (lane >> 4) * 8;
    // lanes past the T tokens / E experts load nothing (their products are
    // never read): their MFMA operand is zero
    const h16* ap[LG];
    bool a_on[LG];
#pragma unroll
    for (int u = 0; u < LG; ++u) {
      ap[u] = h + (long)min(16 * u + tl, T - 1) * ld_h + kb0 + kq;
      a_on[u] = 16 * u + tl < T;
    }
    const h16* bp = reinterpret_cast<const h16*>(w) + (long)min(tl, E - 1) * ld_w + kb0 + kq;
    const bool b_on = tl < E;
    const half8_t z8 = {};
    float4_t acc[LG];
#pragma unroll
    for (int u = 0; u < LG; ++u) acc[u] = float4_t{0.f, 0.f, 0.f, 0.f};
    // passes of up to KST steps whose loads go out together (steps past the
    // slice repeat the last one and are not multiplied)
    constexpr int KST = LG == 1 ? 8 : 4;
    for (int s0 = 0; s0 < steps; s0 += KST) {
      half8_t bv[KST], av[KST][LG];
#pragma unroll
      for (int i = 0; i < KST; ++i) {
        const int st = min(s0 + i, steps - 1);
        bv[i] = b_on ? *reinterpret_cast<const half8_t*>(bp + 32 * st) : z8;
#pragma unroll
        for (int u = 0; u < LG; ++u)
          av[i][u] = a_on[u] ? *reinterpret_cast<const half8_t*>(ap[u] + 32 * st) : z8;
      }
#pragma unroll
      for (int i = 0; i < KST; ++i) {
        if (s0 + i < steps) {  // uniform
#pragma unroll
          for (int u = 0; u < LG; ++u)
            acc[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i][u], bv[i], acc[u], 0, 0, 0);
        }
      }
    }
    // lane: expert tl, tokens 16 u + 4 (lane >> 4) + r; a wave's partial
    // tile holds TS tokens
    constexpr int TS = LG == 4 ? 64 : 32;
#pragma unroll
    for (int u = 0; u < LG; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        s_buf[(wave * TS + 16 * u + 4 * (lane >> 4) + r) * 16 + tl] = acc[u][r];
    __syncthreads();
    for (int i = tid; i < T * E; i += blockDim.x) {
      const int t = i / E, e = i - t * E;
      float v = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < kRouteWaves; ++w2) v += s_buf[(w2 * TS + t) * 16 + e];
      s_lg[i] = ROUND16 ? (float)(h16)v : v;
    }
    lg = s_lg;
  } else {
    for (int pr = wave; pr < T * E; pr += nw) {
      const int t = pr / E, e = pr - t * E;
      const float v = logit_dot<TW, ROUND16>(h + (long)t * ld_h, w + (long)e * ld_w, H, lane);
      if (lane == 0) s_buf[pr] = v;
    }
  }
  __syncthreads();
  if (lead && logits_out)
    for (int i = tid; i < T * E; i += blockDim.x) logits_out[i] = lg[i];

  // 2. top-k: one thread per token up to 16 experts, else one wave per token
  if constexpr (TK == 1) {  // E <= 8, k == 2, softmax (Mixtral)
    for (int t = tid; t < T; t += blockDim.x)
      topk_small<8, 2, 0>(lg + t * E, bias, E, 2, 0, eps, scaling, s_sel + t * 2, s_w + t * 2);
  } else if (E <= 16) {
    for (int t = tid; t < T; t += blockDim.x)
      topk_small<16>(lg + t * E, bias, E, k, mode, eps, scaling, s_sel + t * k, s_w + t * k);
  } else {
    for (int t = wave; t < T; t += nw)
      topk_wave(lg + t * E, tb, E, k, mode, eps, scaling, lane, s_sel + t * k, s_w + t * k);
  }
  __syncthreads();
  if (lead)
    for (int j = tid; j < n; j += blockDim.x) {
      idx_out[j] = s_sel[j];
      w_out[j] = s_w[j];
    }

  // 3. stable order by expert: one thread per assignment j (n <= blockDim);
  //    rank among equal experts in the wave from nine ballots over the bits
  //    of e (-1 for none), then the per-wave counts before this wave
  const int j = tid;
  int e = j < n ? s_sel[j] : -1;
  if (e < 0 || e >= E) e = -1;
  uint64_t same = ~0ull;
#pragma unroll
  for (int b = 0; b < 9; ++b) {
    const uint64_t bal = __ballot((e >> b) & 1);
    same &= ((e >> b) & 1) ? bal : ~bal;
  }
  const int rank = __popcll(same & ((1ull << lane) - 1));
  if (e >= 0 && rank == 0) s_wcnt[wave][e] = __popcll(same);
  __syncthreads();
  if (wave == 0) {  // counts, offsets and the active list: 4 experts per lane, wave scans
    int c[4], f[4], cs = 0, fs = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int ex = 4 * lane + q;
      c[q] = 0;
      if (ex < E)
        for (int w2 = 0; w2 < kRouteWaves; ++w2) c[q] += s_wcnt[w2][ex];
      f[q] = c[q] > 0 ? 1 : 0;
      cs += c[q];
      fs += f[q];
    }
    int ci = cs, fi = fs;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int oc = __shfl_up(ci, off, 64), of = __shfl_up(fi, off, 64);
      if (lane >= off) { ci += oc; fi += of; }
    }
    int co = ci - cs, fo = fi - fs;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int ex = 4 * lane + q;
      if (ex < E) {
        s_off[ex] = co;
        if (lead) {
          offsets[ex] = co;
          if (f[q]) active[fo] = ex;
          if (usage && c[q]) usage[ex] += c[q];
        }
      }
      co += c[q];
      fo += f[q];
    }
    if (lane == 63) {
      s_off[E] = ci;
      if (lead) {
        offsets[E] = ci;
        *n_active = fi;
      }
    }
  }
  __syncthreads();
  if (j < n) {
    if (e >= 0) {
      int pos = s_off[e] + rank;
      for (int w2 = 0; w2 < wave; ++w2) pos += s_wcnt[w2][e];
      s_perm[pos] = j;
      if (lead) {
        perm[pos] = j;
        inv[j] = pos;
      }
    } else if (lead) {
      inv[j] = -1;
    }
  }
  __syncthreads();

  // 4. this workgroup's rows of x_perm (16-byte pieces, 4 in flight per thread)
  const int rows = s_off[E];
  const int per_row = H >> 3;
  const int pieces = rows * per_row;  // < 2^31: T*k <= 1024 rows, checked H
  for (int base = blockIdx.x * blockDim.x * 4 + tid; base < pieces;
       base += gridDim.x * blockDim.x * 4) {
    half8_t v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = min(base + u * (int)blockDim.x, pieces - 1);
      const int p = i / per_row, c = i - p * per_row;
      v[u] = *reinterpret_cast<const half8_t*>(h + (long)(s_perm[p] / k) * ld_h + c * 8);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = base + u * (int)blockDim.x;
      if (i < pieces) {
        const int p = i / per_row, c = i - p * per_row;
        *reinterpret_cast<half8_t*>(x_perm + (long)p * ld_p + c * 8) = v[u];
      }
    }
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

// mode 0: softmax top-k (Mixtral); mode 1: sigmoid top-k (GLM), bias may be
// null; mode 2: sigmoid top-k without the normalisation (norm_topk_prob=False).
extern "C" int hn_router_topk(const void* logits, const void* bias, long T, long E, long k,
                              int mode, float eps, float scaling, int* idx_out, void* w_out,
                              void* stream) {
  HN_ARG_CHECK(T >= 0 && E > 0 && k > 0 && k <= kMaxTopK && k <= E,
               "hn_router_topk: need 0 < k <= min(E, %d)", kMaxTopK);
  // one wave per token holds at most 4 x 64 candidates
  HN_ARG_CHECK(E <= kMaxExperts, "hn_router_topk: need E <= %d (got %ld)", kMaxExperts, E);
  HN_ARG_CHECK(mode >= 0 && mode <= 2, "hn_router_topk: mode must be 0, 1 or 2");
  if (T == 0) return 0;
  hipLaunchKernelGGL(router_topk_kernel, dim3(E <= 16 ? hn_cdiv(T, 256) : hn_cdiv(T, 4)), dim3(256),
                     0, (hipStream_t)stream,
                     (const float*)logits, (const float*)bias, (int)T, (int)E, (int)k, mode, eps,
                     scaling, idx_out, (h16*)w_out);
  HN_LAUNCH_CHECK("hn_router_topk");
  return 0;
}

// Group-limited routing: out [T, E] = logits with the experts outside each
// token's topk_group best groups set to -inf (then hn_router_topk mode 1/2).
extern "C" int hn_router_group_limit(const void* logits, long T, long E, long n_group,
                                     long topk_group, void* out, void* stream) {
  const char* who = "hn_router_group_limit";
  HN_ARG_CHECK(T >= 0 && E > 0 && E <= kMaxExperts, "%s: need 0 < E <= %d", who, kMaxExperts);
  HN_ARG_CHECK(n_group >= 1 && n_group <= 64 && E % n_group == 0,
               "%s: n_group must divide E and be <= 64 (E=%ld n_group=%ld)", who, E, n_group);
  HN_ARG_CHECK(topk_group >= 1 && topk_group <= n_group,
               "%s: need 1 <= topk_group <= n_group (got %ld)", who, topk_group);
  if (T == 0) return 0;
  hipLaunchKernelGGL(router_group_limit_kernel, dim3(hn_cdiv(T, 4)), dim3(256), 0,
                     (hipStream_t)stream, (const float*)logits, (int)T, (int)E, (int)n_group,
                     (int)topk_group, (float*)out);
  HN_LAUNCH_CHECK(who);
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

// Unpermute grid: (token, column block) workgroups of 8 columns per thread;
// batches under 64 tokens use 64-thread workgroups (512 columns each) so
// that a small batch still spreads over the CUs.  At most 8 blocks per token.
static unsigned unpermute_threads(long T) { return T < 64 ? 64u : 256u; }
static unsigned unpermute_blocks(long H, long T) {
  const long cols = 8L * unpermute_threads(T);
  const long b = (H + cols - 1) / cols;
  return (unsigned)(b < 1 ? 1 : (b > 8 ? 8 : b));
}

extern "C" int hn_moe_unpermute(const void* y_perm, long ld_y, const int* inv, const int* idx,
                                const void* w, long T, long k, const void* shared, long ld_sh,
                                void* out, long ld_o, long H, void* stream) {
  HN_ARG_CHECK(k > 0 && k <= kMaxTopK, "hn_moe_unpermute: k must be in (0, %d]", kMaxTopK);
  HN_ARG_CHECK(H % 8 == 0 && al16(y_perm) && al16(out) && ld_y % 8 == 0 && ld_o % 8 == 0 &&
                   (!shared || (al16(shared) && ld_sh % 8 == 0)),
               "hn_moe_unpermute: rows must be 16-byte aligned");
  if (T <= 0) return 0;
  hipLaunchKernelGGL(moe_unpermute_kernel<0>, dim3((unsigned)T, unpermute_blocks(H, T)),
                     dim3(unpermute_threads(T)), 0,
                     (hipStream_t)stream, (const h16*)y_perm, (const float*)nullptr, 0L, ld_y,
                     inv, idx, (const h16*)w, (int)k, (const h16*)shared, ld_sh, (h16*)out, ld_o,
                     (int)H);
  HN_LAUNCH_CHECK("hn_moe_unpermute");
  return 0;
}

// Decode routing in one launch (logits unless logits_in is given, top-k,
// permutation, gather).  See include/hn_int4.h.
extern "C" int hn_moe_route(const void* h, long ld_h, const void* w, long ld_w, int w_dtype,
                            const void* logits_in, const void* bias, long T, long E, long H,
                            long k, int mode, float eps, float scaling, void* logits_out,
                            int* idx_out, void* w_out, int* offsets, int* perm, int* inv,
                            int* active, int* n_active, long long* usage, void* x_perm,
                            long ld_p, void* stream) {
  const char* who = "hn_moe_route";
  HN_ARG_CHECK(T >= 0 && E > 0 && E <= kMaxExperts && H > 0,
               "%s: need 0 < E <= %d", who, kMaxExperts);
  HN_ARG_CHECK(k > 0 && k <= kMaxTopK && k <= E, "%s: need 0 < k <= min(E, %d)", who, kMaxTopK);
  HN_ARG_CHECK(mode >= 0 && mode <= 2, "%s: mode must be 0, 1 or 2", who);
  HN_ARG_CHECK(T * E <= kRouteMaxLogits && T * k <= kRouteMaxAssign,
               "%s: T*E <= %d and T*k <= %d (decode sizes; use the separate kernels above)",
               who, kRouteMaxLogits, kRouteMaxAssign);
  HN_ARG_CHECK(H % 8 == 0 && ld_h % 8 == 0 && al16(h) && al16(x_perm) && ld_p % 8 == 0,
               "%s: h and x_perm rows must be 16-byte aligned with H %% 8 == 0", who);
  HN_ARG_CHECK(logits_in || (w && al16(w) && (w_dtype == 0 ? ld_w % 8 == 0 : ld_w % 4 == 0)),
               "%s: weight rows must be 16-byte aligned (or pass logits_in)", who);
  HN_ARG_CHECK(!logits_in || al16(logits_in), "%s: logits_in must be 16-byte aligned", who);
  if (T == 0) return 0;
  // about 64 KiB of rows per workgroup; every workgroup repeats the routing
  const long bytes = T * k * H * 2;
  const int grid = (int)std::min(128L, std::max(1L, (bytes + 65535) / 65536));
  hipStream_t s = (hipStream_t)stream;
  // logits by MFMA for an fp16 gate with T <= 64, T * E <= 512, E <= 16, H % 512 == 0
  const int lgv = (logits_in || w_dtype != 0 || E > 16 || H % 512 != 0 || T * E > 512)
                      ? 0 : (T <= 16 ? 1 : (T <= 32 ? 2 : (T <= 64 ? 4 : 0)));
  const bool mix = E <= 8 && k == 2 && mode == 0;
#define HN_ROUTE_LAUNCH(TW, R16, LGV, TKV)                                                          \
  hipLaunchKernelGGL((moe_route_kernel<TW, R16, LGV, TKV>), dim3(grid), dim3(kRouteThreads), 0, s, \
                     (const h16*)h, ld_h, (const TW*)w, ld_w, (const float*)logits_in,           \
                     (const float*)bias, (int)T, (int)E, (int)H, (int)k, mode, eps, scaling,      \
                     (float*)logits_out, idx_out, (h16*)w_out, offsets, perm, inv, active,        \
                     n_active, usage, (h16*)x_perm, ld_p)
  if (w_dtype == 0) {
    if (lgv == 1 && mix) HN_ROUTE_LAUNCH(h16, true, 1, 1);
    else if (lgv == 2 && mix) HN_ROUTE_LAUNCH(h16, true, 2, 1);
    else if (lgv == 4 && mix) HN_ROUTE_LAUNCH(h16, true, 4, 1);
    else if (lgv == 1) HN_ROUTE_LAUNCH(h16, true, 1, 0);
    else if (lgv == 2) HN_ROUTE_LAUNCH(h16, true, 2, 0);
    else if (lgv == 4) HN_ROUTE_LAUNCH(h16, true, 4, 0);
    // given logits (or no MFMA logits) with Mixtral's top-2: the top-2
    // specialisation, not the generic top-k (whose unrolled guards for up
    // to 16 picks and every mode cost a thread about 5 us of branches)
    else if (mix) HN_ROUTE_LAUNCH(h16, true, 0, 1);
    else HN_ROUTE_LAUNCH(h16, true, 0, 0);
  } else {
    HN_ROUTE_LAUNCH(float, false, 0, 0);
  }
#undef HN_ROUTE_LAUNCH
  HN_LAUNCH_CHECK(who);
  return 0;
}

// Unpermute from the kHnDownSplit = 4 fp32 K-slice partials of the down
// projection (hn_stream_down_split_impl): part[j * ks_stride + row * H], j < 4.
extern "C" int hn_moe_unpermute_split4_impl(const float* part, long ks_stride, const int* inv,
                                            const int* idx, const void* w, long T, long k,
                                            const void* shared, long ld_sh, void* out,
                                            long ld_o, long H, void* stream) {
  HN_ARG_CHECK(k > 0 && k <= kMaxTopK, "hn_moe_unpermute: k must be in (0, %d]", kMaxTopK);
  HN_ARG_CHECK(H % 8 == 0 && al16(part) && al16(out) && ks_stride % 4 == 0 && ld_o % 8 == 0 &&
                   (!shared || (al16(shared) && ld_sh % 8 == 0)),
               "hn_moe_unpermute: rows must be 16-byte aligned");
  if (T <= 0) return 0;
  hipLaunchKernelGGL(moe_unpermute_kernel<kHnDownSplit>,
                     dim3((unsigned)T, unpermute_blocks(H, T)), dim3(unpermute_threads(T)), 0,
                     (hipStream_t)stream, (const h16*)nullptr, part, ks_stride, H, inv, idx,
                     (const h16*)w, (int)k, (const h16*)shared, ld_sh, (h16*)out, ld_o, (int)H);
  HN_LAUNCH_CHECK("hn_moe_unpermute");
  return 0;
}
