// Decoder-step kernels around the MoE layer (the whole-model decode harness):
// residual add + RMSNorm, and RoPE on the query/key projections with the
// KV-cache append.  Each replaces a chain of stock elementwise kernels of the
// reference's torch formulation (model/mixtral.py:23-37, 82-101, 150-190)
// with one launch and reproduces its fp16 rounding steps:
//
//   add:      x' = fp16(float(x) + float(r))                 (torch fp16 add)
//   RMSNorm:  v = mean(float(x')^2); t = float(x') * rsqrt(v + eps);
//             out = fp16(float(w) * t)                       (fp32 math, one cast)
//   RoPE:     c, s = fp16(cos[pos]), fp16(sin[pos]);
//             y[d] = fp16(fp16(x[d] * c[d]) + fp16(rh(x)[d] * s[d])),
//             rh(x) = (-x[hd/2:], x[:hd/2])                  (rotate_half)
//
// The mean's fp32 summation order differs from torch's reduction tree, so
// RMSNorm outputs can differ from the torch formulation by an fp16 ulp;
// add and RoPE are exact replicas.
#include "hn_common.h"

namespace {

constexpr int kNormThreads = 256;

constexpr int kMaxGate = 16;  // router experts the norm kernel can score

// One workgroup per row; 8 fp16 per vector access.  LG > 0: also the router
// logits of the normalised row against E <= LG gate rows, logits[row, e] =
// fp16(sum_k out[k] gate[e, k]) (fp32 sums: per thread, then the wave, then
// the waves in order) stored as fp32 -- the fp16 Linear of TopKRouter
// (model/router.py:102) on this row.  Every expert's gate loads of a thread
// go out together and the E wave reductions are interleaved.
template <int LG>
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(
    const h16* __restrict__ x, long ld_x, const h16* __restrict__ res, long ld_r,
    h16* __restrict__ x_out, long ld_xo, const h16* __restrict__ w, h16* __restrict__ out,
    long ld_o, int H, float eps, const h16* __restrict__ gate, long ld_g, int E,
    float* __restrict__ logits) {
  __shared__ float s_part[kNormThreads / 64];
  __shared__ float s_lg[kNormThreads / 64][kMaxGate];
  const int row = blockIdx.x, tid = threadIdx.x;
  const half8_t* xr = reinterpret_cast<const half8_t*>(x + (long)row * ld_x);
  const half8_t* rr = res ? reinterpret_cast<const half8_t*>(res + (long)row * ld_r) : nullptr;
  half8_t* xo = x_out ? reinterpret_cast<half8_t*>(x_out + (long)row * ld_xo) : nullptr;
  const int nv = H >> 3;
  // H <= 8 * 256 * 4 = 8192: a thread keeps at most 4 vectors in registers
  half8_t v[4];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int j = tid + i * kNormThreads;
    if (j < nv) {
      half8_t a = xr[j];
      if (rr) {
        const half8_t b = rr[j];
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = (h16)((float)a[e] + (float)b[e]);
        if (xo) xo[j] = a;
      }
      v[i] = a;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += (float)a[e] * (float)a[e];
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
  if ((tid & 63) == 0) s_part[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) tot += s_part[i];
  const float r = rsqrtf(tot / (float)H + eps);
  const half8_t* wr = reinterpret_cast<const half8_t*>(w);
  half8_t* orow = reinterpret_cast<half8_t*>(out + (long)row * ld_o);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int j = tid + i * kNormThreads;
    if (j < nv) {
      const half8_t wv = wr[j];
      half8_t o;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float t = (float)v[i][e] * r;
        o[e] = (h16)((float)wv[e] * t);
      }
      orow[j] = o;
      if constexpr (LG > 0) v[i] = o;
    }
  }
  if constexpr (LG > 0) {
    const int lane = tid & 63, wave = tid >> 6;
    float d[LG];
#pragma unroll
    for (int e = 0; e < LG; ++e) d[e] = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = tid + i * kNormThreads;
      if (j < nv) {
        half8_t gv[LG];
#pragma unroll
        for (int e = 0; e < LG; ++e)
          if (e < E) gv[e] = reinterpret_cast<const half8_t*>(gate + (long)e * ld_g)[j];
#pragma unroll
        for (int e = 0; e < LG; ++e)
          if (e < E)
#pragma unroll
            for (int q = 0; q < 8; ++q) d[e] = __builtin_fmaf((float)v[i][q], (float)gv[e][q], d[e]);
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1)
#pragma unroll
      for (int e = 0; e < LG; ++e) d[e] += __shfl_xor(d[e], off, 64);
    if (lane == 0)
#pragma unroll
      for (int e = 0; e < LG; ++e)
        if (e < E) s_lg[wave][e] = d[e];
    __syncthreads();
    if (tid < E) {
      float t = 0.f;
#pragma unroll
      for (int wv = 0; wv < kNormThreads / 64; ++wv) t += s_lg[wv][tid];
      logits[(long)row * E + tid] = (float)(h16)t;
    }
  }
}

// Attention probabilities of a decode step, one wave per row of scores:
//   a = fp16(float(s) * inv_scale);  a = fp16(float(a) + float(mask))  (mask given)
//   p = fp16(exp(a - max) / sum exp(a - max))   (fp32)
// The torch formulation's steps (model/mixtral.py:193-203): a Half tensor
// divided by a Python scalar is multiplied by the fp32 reciprocal
// (div_true_kernel_cuda's scalar path) and rounded; the mask add rounds;
// F.softmax(dtype=float32) of a row of L <= 1024 runs softmax_warp_forward,
// whose element order this kernel keeps: ws = min(2^ceil(log2 L), 64) lanes,
// lane l holding elements l + ws * it, each lane's exps summed in it order,
// then butterflies from ws / 2 down (max, then sum), exp by the same libm
// expf; the .to(fp16) rounds the fp32 quotient.  Rows (b, g, r, s) take mask
// row s = row % mask_rows.
template <int IT>
__global__ __launch_bounds__(256) void attn_softmax_kernel(const h16* __restrict__ s, long ld_s,
                                                           const h16* __restrict__ mask,
                                                           long ld_m, int mask_rows, int rows,
                                                           int L, int ws, float inv_scale,
                                                           h16* __restrict__ out, long ld_o) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole wave
  const h16* sr = s + (long)row * ld_s;
  const h16* mr = mask ? mask + (long)(row % mask_rows) * ld_m : nullptr;
  float x[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int i = it * ws + lane;
    if (lane < ws && i < L) {
      h16 a = (h16)((float)sr[i] * inv_scale);
      if (mr) a = (h16)((float)a + (float)mr[i]);
      x[it] = (float)a;
    } else {
      x[it] = -__builtin_inff();
    }
  }
  float mx = x[0];
#pragma unroll
  for (int it = 1; it < IT; ++it) mx = mx > x[it] ? mx : x[it];
  for (int off = ws >> 1; off > 0; off >>= 1) {
    const float o = __shfl_xor(mx, off, 64);
    mx = mx < o ? o : mx;
  }
  float sum = 0.f;
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    x[it] = expf(x[it] - mx);
    sum += x[it];
  }
  for (int off = ws >> 1; off > 0; off >>= 1) sum = sum + __shfl_xor(sum, off, 64);
  h16* orow = out + (long)row * ld_o;
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int i = it * ws + lane;
    if (lane < ws && i < L) orow[i] = (h16)(x[it] / sum);
  }
}

// Grid (rows = B * S, nh + nkv): one workgroup of hd threads per (token,
// head).  Heads below nh are query heads, written rotated to
// q_out[b][h / rep][h % rep][s][:]; the others are KV heads g: the rotated
// key goes to kt[b][g][:][pos[s]] (keys transposed), the value to
// vc[b][g][pos[s]][:].
__global__ void rope_append_kernel(const h16* __restrict__ q, long ld_q, const h16* __restrict__ k,
                                   long ld_k, const h16* __restrict__ v, long ld_v,
                                   const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                                   const long* __restrict__ pos, int S, int nh, int nkv, int hd,
                                   h16* __restrict__ q_out, h16* __restrict__ kt,
                                   h16* __restrict__ vc, long max_len) {
  // each product is rounded to fp16 before the sum (no fused multiply-add)
#pragma clang fp contract(off)
  const int row = blockIdx.x, head = blockIdx.y, d = threadIdx.x;
  const int b = row / S, s = row - b * S;
  const long p = pos[s];
  if (p < 0 || p >= max_len) return;  // callers check positions on the host too
  const int half = hd >> 1;
  const h16 c = (h16)cos_t[p * hd + d];
  const h16 sn = (h16)sin_t[p * hd + d];
  const int dp = d < half ? d + half : d - half;
  auto rot = [&](const h16* src) -> h16 {
    const h16 xd = src[d];
    const h16 xr = d < half ? (h16)(-(float)src[dp]) : src[dp];
    const h16 a = (h16)((float)xd * (float)c);
    const h16 bb = (h16)((float)xr * (float)sn);
    return (h16)((float)a + (float)bb);
  };
  const int rep = nh / nkv;
  if (head < nh) {
    const h16* src = q + (long)row * ld_q + (long)head * hd;
    const int g = head / rep, r = head - g * rep;
    q_out[((((long)b * nkv + g) * rep + r) * S + s) * hd + d] = rot(src);
  } else {
    const int g = head - nh;
    const h16* src = k + (long)row * ld_k + (long)g * hd;
    kt[(((long)b * nkv + g) * hd + d) * max_len + p] = rot(src);
    vc[(((long)b * nkv + g) * max_len + p) * hd + d] = v[(long)row * ld_v + (long)g * hd + d];
  }
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

// out[t] = RMSNorm(x[t] (+ res[t])) * w, rows t < T of H fp16; with res, the
// sum x + res is also written to x_out (the updated residual stream; may
// alias x).  See include/hn_int4.h.
extern "C" int hn_add_rmsnorm(const void* x, long ld_x, const void* res, long ld_r, void* x_out,
                              long ld_xo, const void* w, void* out, long ld_o, long T, long H,
                              float eps, void* stream) {
  HN_ARG_CHECK(T >= 0 && H > 0 && H % 8 == 0 && H <= 8 * kNormThreads * 4,
               "hn_add_rmsnorm: need 0 < H <= %d, H %% 8 == 0", 8 * kNormThreads * 4);
  HN_ARG_CHECK(al16(x) && ld_x % 8 == 0 && al16(w) && al16(out) && ld_o % 8 == 0 &&
                   (!res || (al16(res) && ld_r % 8 == 0)) &&
                   (!x_out || (al16(x_out) && ld_xo % 8 == 0)),
               "hn_add_rmsnorm: rows must be 16-byte aligned");
  if (T == 0) return 0;
  hipLaunchKernelGGL(add_rmsnorm_kernel<0>, dim3((unsigned)T), dim3(kNormThreads), 0,
                     (hipStream_t)stream, (const h16*)x, ld_x, (const h16*)res, ld_r,
                     (h16*)x_out, ld_xo, (const h16*)w, (h16*)out, ld_o, (int)H, eps,
                     (const h16*)nullptr, 0L, 0, (float*)nullptr);
  HN_LAUNCH_CHECK("hn_add_rmsnorm");
  return 0;
}

// hn_add_rmsnorm, then the router logits of each normalised row against an
// fp16 gate [E, H] (E <= 16): logits [T, E] fp32 holding fp16-rounded values.
// See include/hn_int4.h.
extern "C" int hn_add_rmsnorm_router(const void* x, long ld_x, const void* res, long ld_r,
                                     void* x_out, long ld_xo, const void* w, void* out,
                                     long ld_o, long T, long H, float eps, const void* gate,
                                     long ld_g, long E, float* logits, void* stream) {
  HN_ARG_CHECK(T >= 0 && H > 0 && H % 8 == 0 && H <= 8 * kNormThreads * 4,
               "hn_add_rmsnorm_router: need 0 < H <= %d, H %% 8 == 0", 8 * kNormThreads * 4);
  HN_ARG_CHECK(E > 0 && E <= kMaxGate, "hn_add_rmsnorm_router: need 0 < E <= %d", kMaxGate);
  HN_ARG_CHECK(al16(x) && ld_x % 8 == 0 && al16(w) && al16(out) && ld_o % 8 == 0 &&
                   (!res || (al16(res) && ld_r % 8 == 0)) &&
                   (!x_out || (al16(x_out) && ld_xo % 8 == 0)) && gate && al16(gate) &&
                   ld_g % 8 == 0 && ld_g >= H && logits,
               "hn_add_rmsnorm_router: rows must be 16-byte aligned (gate and logits given)");
  if (T == 0) return 0;
  auto kern = E <= 8 ? add_rmsnorm_kernel<8> : add_rmsnorm_kernel<kMaxGate>;
  hipLaunchKernelGGL(kern, dim3((unsigned)T), dim3(kNormThreads), 0, (hipStream_t)stream,
                     (const h16*)x, ld_x, (const h16*)res, ld_r, (h16*)x_out, ld_xo,
                     (const h16*)w, (h16*)out, ld_o, (int)H, eps, (const h16*)gate, ld_g, (int)E,
                     logits);
  HN_LAUNCH_CHECK("hn_add_rmsnorm_router");
  return 0;
}

// Scale, mask, fp32 softmax and fp16 cast of attention scores in one
// launch.  See include/hn_int4.h.
extern "C" int hn_attn_softmax(const void* scores, long ld_s, const void* mask, long ld_m,
                               long mask_rows, long rows, long L, float inv_scale, void* out,
                               long ld_o, void* stream) {
  HN_ARG_CHECK(rows >= 0 && L >= 1 && L <= 1024 && (!mask || mask_rows >= 1),
               "hn_attn_softmax: need 1 <= L <= 1024 (L=%ld) and mask_rows >= 1 with a mask", L);
  HN_ARG_CHECK(ld_s >= L && ld_o >= L && (!mask || ld_m >= L),
               "hn_attn_softmax: row strides below L");
  if (rows == 0) return 0;
  int p2 = 1;
  while (p2 < L) p2 <<= 1;
  const int ws = p2 < 64 ? p2 : 64;
  const int it = p2 / ws;
  const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
  hipStream_t st = (hipStream_t)stream;
#define HN_SOFTMAX(N)                                                                          \
  hipLaunchKernelGGL(attn_softmax_kernel<N>, grid, block, 0, st, (const h16*)scores, ld_s,     \
                     (const h16*)mask, ld_m, (int)(mask ? mask_rows : 1), (int)rows, (int)L,   \
                     ws, inv_scale, (h16*)out, ld_o)
  switch (it) {
    case 1: HN_SOFTMAX(1); break;
    case 2: HN_SOFTMAX(2); break;
    case 4: HN_SOFTMAX(4); break;
    case 8: HN_SOFTMAX(8); break;
    default: HN_SOFTMAX(16); break;
  }
#undef HN_SOFTMAX
  HN_LAUNCH_CHECK("hn_attn_softmax");
  return 0;
}

// RoPE on the query / key projections of B * S tokens and the KV-cache
// append at positions pos[S].  See include/hn_int4.h.
extern "C" int hn_rope_append(const void* q, long ld_q, const void* k, long ld_k, const void* v,
                              long ld_v, const float* cos_t, const float* sin_t, const long* pos,
                              long B, long S, long nh, long nkv, long hd, void* q_out, void* kt,
                              void* vc, long max_len, void* stream) {
  HN_ARG_CHECK(B >= 0 && S >= 0 && nkv > 0 && nh % nkv == 0 && hd % 2 == 0 && hd <= 1024 &&
                   max_len > 0,
               "hn_rope_append: need nh %% nkv == 0, even head_dim <= 1024");
  if (B == 0 || S == 0) return 0;
  hipLaunchKernelGGL(rope_append_kernel, dim3((unsigned)(B * S), (unsigned)(nh + nkv)),
                     dim3((unsigned)hd), 0, (hipStream_t)stream, (const h16*)q, ld_q,
                     (const h16*)k, ld_k, (const h16*)v, ld_v, cos_t, sin_t, pos, (int)S,
                     (int)nh, (int)nkv, (int)hd, (h16*)q_out, (h16*)kt, (h16*)vc, max_len);
  HN_LAUNCH_CHECK("hn_rope_append");
  return 0;
}
