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
#include "hn_unpermute.h"

namespace {

constexpr int kNormThreads = 256;

constexpr int kMaxGate = 16;  // router experts the norm kernel can score

// One workgroup per row; 8 fp16 per vector access.  LG > 0: also the router
// logits of the normalised row against E <= LG gate rows, logits[row, e] =
// fp16(sum_k out[k] gate[e, k]) (fp32 sums: per thread, then the wave, then
// the waves in order) stored as fp32 -- the fp16 Linear of TopKRouter
// (model/router.py:102) on this row.  Every expert's gate loads of a thread
// go out together and the E wave reductions are interleaved.
// UNP: the residual res is the row's MoE output, computed here from the
// down projection's four fp32 K-slice partials and the routing (the ordered
// weighted sum of moe_unpermute_kernel<4>, unp_select / unp_cols), instead of
// read: the MoE block's last launch and the next RMSNorm in one.
struct UnpSrc {
  const float* part;  // [kHnDownSplit][rows][ld_y] fp32
  long ks_stride;     // floats between slices
  long ld_y;
  const int* inv;
  const int* idx;
  const h16* w;
  int k;
};

template <int LG, bool UNP = false>
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(
    const h16* __restrict__ x, long ld_x, const h16* __restrict__ res, long ld_r,
    h16* __restrict__ x_out, long ld_xo, const h16* __restrict__ w, h16* __restrict__ out,
    long ld_o, int H, float eps, const h16* __restrict__ gate, long ld_g, int E,
    float* __restrict__ logits, UnpSrc U) {
  __shared__ float s_part[kNormThreads / 64];
  __shared__ float s_lg[kNormThreads / 64][kMaxGate];
  const int row = blockIdx.x, tid = threadIdx.x;
  int upos[kMaxTopK];
  float uwt[kMaxTopK];
  int un = 0;
  if constexpr (UNP) un = unp_select(row, U.inv, U.idx, U.w, U.k, upos, uwt);
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
      if (UNP || rr) {
        half8_t b;
        if constexpr (UNP)
          b = unp_cols<kHnDownSplit>(nullptr, U.part, U.ks_stride, U.ld_y, upos, uwt, un, 8 * j);
        else
          b = rr[j];
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
// RoPE of element d of one head's row at position p (model/mixtral.py:82-101):
// c, s = fp16(cos[p][d]), fp16(sin[p][d]); y = fp16(fp16(x[d] c) + fp16(rh(x)[d]
// s)), rh(x) = (-x[hd/2:], x[:hd/2]).  Each product is rounded to fp16
// before the sum (no fused multiply-add); one function for every kernel that
// rotates, so they agree bit for bit.
__device__ __forceinline__ h16 rope_rot(const h16* src, const float* cos_t, const float* sin_t,
                                        long p, int d, int hd) {
#pragma clang fp contract(off)
  const int half = hd >> 1;
  const h16 c = (h16)cos_t[p * hd + d];
  const h16 sn = (h16)sin_t[p * hd + d];
  const int dp = d < half ? d + half : d - half;
  const h16 xd = src[d];
  const h16 xr = d < half ? (h16)(-(float)src[dp]) : src[dp];
  const h16 a = (h16)((float)xd * (float)c);
  const h16 bb = (h16)((float)xr * (float)sn);
  return (h16)((float)a + (float)bb);
}

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
  auto rot = [&](const h16* src) -> h16 { return rope_rot(src, cos_t, sin_t, p, d, hd); };
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


// ---------------------------------------------------------------------------
// Decode attention: one query token per sequence, grouped-query heads.
// One workgroup of 16 waves per (sequence b, KV head g) reads that head's
// keys and values once and computes, for the REP query heads of the group,
// the reference's formulation (model/mixtral.py:193-207):
//   s16 = fp16(sum_d q[r][d] k[d][l])            (fp16 product, fp32 sums)
//   a = fp16(s16 * inv_scale); a = fp16(a + mask[l]) with a mask row
//   p = fp16(softmax_fp32(a))                    (F.softmax(dtype=float32))
//   o[r][d] = fp16(sum_l p[r][l] v[l][d])        (fp16 product, fp32 sums)
// Keys are stored transposed, kt[b][g][d][max_len]; values v[b][g][l][d].
//  * scores: thread (position group pg = tid / 8, d slice ds = tid % 8)
//    loads keys d = 16 ds .. 16 ds + 15 at positions 8 pg .. 8 pg + 7 (16
//    loads of 16 bytes, all in flight: the head's whole K in one round
//    trip) and accumulates the REP x 8 partial sums in fp32 with v_dot2
//    (fp16 pairs of d, the keys of two rows packed per position by
//    v_perm: 2.5 instructions per key element instead of 4 mixed FMAs);
//    a three-step reduce-scatter over the 8 lanes of a group (DPP) leaves
//    lane ds the sums of position 8 pg + ds; waves wholly past L skip it;
//  * the values' loads go out next (thread: 8 d columns dg, positions
//    ls + 64 i), before the softmax, whose reductions hide their latency;
//  * softmax per row over LDS (row max, then exp sums: per lane in index
//    order, then the wave's butterfly, then the waves in order);
//  * values: per-thread fp32 sums over its positions (v_dot2 over position
//    pairs), a reduce-scatter over the wave's 4 position slices, then the 16
//    waves added in order.
// The fp32 sums run in another order than a library GEMM's, so outputs
// agree with the two-product formulation within fp16 rounding.
constexpr int kAttnHd = 128;
constexpr int kAttnWaves = 16;

template <int CTL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTL, 0xf, 0xf, false));
}
// v from lane ^ 4 (within a row of 16 lanes)
__device__ __forceinline__ float xor4_f32(float v, bool hi) {
  const float up = dpp_f32<0x104>(v);  // row_shl:4: lane + 4
  const float dn = dpp_f32<0x114>(v);  // row_shr:4: lane - 4
  return hi ? dn : up;
}

// ROPE: the step's own query, key and value come unrotated from the fused
// q/k/v projection (qkv[b][ld_qkv]: nh query heads, nkv keys, nkv values);
// the workgroup rotates its REP query heads and its key (rope_rot, the same
// arithmetic as hn_rope_append), writes the key and value to the cache at
// the step's position p = pos[0], and uses them directly: the cache loads
// go out first, and the lanes holding position p take the new key and value
// in registers (the loaded copies are from before the write).
template <int REP, int LMAX, bool ROPE>
__global__ __launch_bounds__(1024) void attn_decode_kernel(
    const h16* __restrict__ q, h16* __restrict__ kt, h16* __restrict__ vc, long max_len,
    int nkv, int L, const h16* __restrict__ mask, float inv_scale, h16* __restrict__ out,
    long ld_o, const h16* __restrict__ qkv, long ld_qkv, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, const long* __restrict__ pos) {
  constexpr int HD = kAttnHd;
  constexpr int NV = LMAX / 64;  // value positions per thread
  // the query pairs are read as four scalars: read as one 16-byte vector
  // and split by element extracts into v_dot2, the compiler fed element 0
  // to every head's dot products (all heads got head 0's scores)
  __shared__ uint32_t s_q2[HD / 2][4];  // [i][r] = (q[r][2 i], q[r][2 i + 1])
  // scaled scores, then probabilities, [l][r]; 1024 rows whatever LMAX, so
  // every lane's position (8 pg + ds < 1024) has a row and the store after
  // the DPP exchanges needs no branch
  __shared__ float4_t s_x[1024];
  __shared__ float s_red[2][kAttnWaves];
  __shared__ __align__(16) float s_o[kAttnWaves][REP][HD];
  __shared__ uint32_t s_knew[HD / 2];  // ROPE: the step's rotated key, d pairs
  __shared__ uint32_t s_vnew[HD / 2];  // ROPE: the step's value, d pairs
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform
  const int bg = blockIdx.x;  // b * nkv + g
  const int b = bg / nkv, g = bg - b * nkv;
  const h16* qb = q + (long)bg * REP * HD;
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(kt + (long)bg * HD * max_len), (short)0, (int)(HD * max_len * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(vc + (long)bg * max_len * HD), (short)0, (int)(max_len * HD * 2), 0x00020000);
  constexpr uint32_t kOOB = 0x7ffffff0u;

  // 1. keys: all 16 loads of the thread in flight (positions past the
  //    groups of L read nothing; waves wholly past them skip the scores)
  const int pg = tid >> 3, ds = tid & 7;
  const int npg = (L + 7) >> 3;
  const bool kwave = 64 * wave < L;  // uniform
  const uint32_t ko = pg < npg ? (uint32_t)(((16 * ds) * max_len + 8 * pg) * 2) : kOOB;
  u32x4 kr[16];
  if (kwave) {
#pragma unroll
    for (int dd = 0; dd < 16; ++dd)
      kr[dd] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     rk, ko == kOOB ? kOOB : ko + (uint32_t)(dd * max_len * 2), 0, 0));
  }
  // this lane's score position and its mask entry (loaded with the keys)
  const int lpos = 8 * pg + ds;
  const bool lon = lpos < L;
  const float mv = mask ? (float)mask[lon ? lpos : L - 1] : 0.f;
  long pnew = -1;  // ROPE: the step's position
  if (ROPE) {
    // threads (row r <= REP, pair i): rows < REP the query heads, row REP the
    // key; the next HD / 2 threads the value pairs
    pnew = pos[0];
    // a position outside the cache writes nothing and patches nothing (the
    // callers check it on the host too)
    const bool pok = pnew >= 0 && pnew < max_len;
    const long prot = pok ? pnew : 0;  // the tables' row the rotation reads
    if (!pok) pnew = -1;
    const int nh = nkv * REP;
    const h16* rowp = qkv + (long)b * ld_qkv;
    if (tid < (REP + 1) * (HD / 2)) {
      const int r = tid / (HD / 2), i = tid - r * (HD / 2);
      const h16* src = r < REP ? rowp + (long)(g * REP + r) * HD : rowp + (long)(nh + g) * HD;
      const h16 y0 = rope_rot(src, cos_t, sin_t, prot, 2 * i, HD);
      const h16 y1 = rope_rot(src, cos_t, sin_t, prot, 2 * i + 1, HD);
      const uint32_t pr = (uint32_t)__builtin_bit_cast(uint16_t, y0) |
                          ((uint32_t)__builtin_bit_cast(uint16_t, y1) << 16);
      if (r < REP) {
        s_q2[i][r] = pr;
      } else {
        s_knew[i] = pr;
        if (pok) {
          h16* kcol = kt + ((long)bg * HD + 2 * i) * max_len + pnew;
          kcol[0] = y0;
          kcol[max_len] = y1;
        }
      }
    } else if (tid < (REP + 2) * (HD / 2)) {
      const int i = tid - (REP + 1) * (HD / 2);
      const uint32_t pr =
          *reinterpret_cast<const uint32_t*>(rowp + (long)(nh + nkv + g) * HD + 2 * i);
      s_vnew[i] = pr;
      if (pok) *reinterpret_cast<uint32_t*>(vc + ((long)bg * max_len + pnew) * HD + 2 * i) = pr;
    }
  } else if (tid < REP * HD / 2) {
    const int r = tid / (HD / 2), i = tid - r * (HD / 2);
    s_q2[i][r] = *reinterpret_cast<const uint32_t*>(qb + r * HD + 2 * i);
  }
  __syncthreads();
  if (ROPE && kwave) {
    // the lanes of position pnew take the new key (the loaded one is from
    // before this step's write)
    const int jp = (int)(pnew - 8 * pg);
    if (jp >= 0 && jp < 8) {
#pragma unroll
      for (int dd = 0; dd < 16; ++dd) {
        const int d = 16 * ds + dd;
        const uint32_t kn = (s_knew[d >> 1] >> (16 * (d & 1))) & 0xffffu;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          if ((jp >> 1) == w) {
            const uint32_t cur = kr[dd][w];
            kr[dd][w] = (jp & 1) ? ((cur & 0xffffu) | (kn << 16)) : ((cur & 0xffff0000u) | kn);
          }
        }
      }
    }
  }

  // 2. scores: fp32 sums over the thread's 16 d (v_dot2: pairs of d, the
  //    keys of two rows packed per position), then over the 8 d slices
  float acc[REP][8];
#pragma unroll
  for (int r = 0; r < REP; ++r)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[r][j] = 0.f;
  if (kwave) {
#pragma unroll
    for (int dd = 0; dd < 16; dd += 2) {
      uint32_t q2[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) q2[r] = s_q2[8 * ds + dd / 2][r];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        // (k[d][2 w], k[d + 1][2 w]) and (k[d][2 w + 1], k[d + 1][2 w + 1])
        const uint32_t lo = __builtin_amdgcn_perm(kr[dd + 1][w], kr[dd][w], 0x05040100u);
        const uint32_t hi = __builtin_amdgcn_perm(kr[dd + 1][w], kr[dd][w], 0x07060302u);
#pragma unroll
        for (int r = 0; r < REP; ++r) {
          const half2_t qa = __builtin_bit_cast(half2_t, q2[r]);
          acc[r][2 * w] = __builtin_amdgcn_fdot2(qa, __builtin_bit_cast(half2_t, lo),
                                                 acc[r][2 * w], false);
          acc[r][2 * w + 1] = __builtin_amdgcn_fdot2(qa, __builtin_bit_cast(half2_t, hi),
                                                     acc[r][2 * w + 1], false);
        }
      }
    }
  }
  if (kwave) {
  // reduce-scatter over ds (lane bits 2, 1, 0): keep positions of bit 2 = h
  // (4 of 8), then bit 1 (2 of 4), then bit 0 (1 of 2); each step adds the
  // kept half of this lane and the partner's copy of the same positions
  float r4[REP][4], r2[REP][2], r1[REP];
  {
    const bool h = (ds >> 2) & 1;
#pragma unroll
    for (int r = 0; r < REP; ++r)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const float keep = h ? acc[r][4 + jj] : acc[r][jj];
        const float send = h ? acc[r][jj] : acc[r][4 + jj];
        r4[r][jj] = keep + xor4_f32(send, h);
      }
  }
  {
    const bool h = (ds >> 1) & 1;
#pragma unroll
    for (int r = 0; r < REP; ++r)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const float keep = h ? r4[r][2 + jj] : r4[r][jj];
        const float send = h ? r4[r][jj] : r4[r][2 + jj];
        r2[r][jj] = keep + dpp_f32<0x4E>(send);  // quad_perm [2,3,0,1]: lane ^ 2
      }
  }
  {
    const bool h = ds & 1;
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      const float keep = h ? r2[r][1] : r2[r][0];
      const float send = h ? r2[r][0] : r2[r][1];
      r1[r] = keep + dpp_f32<0xB1>(send);  // quad_perm [1,0,3,2]: lane ^ 1
    }
  }
  // lane ds holds position l = 8 pg + ds: scale and mask with the
  // reference's fp16 roundings (straight-line code: the exchanged sums are
  // not consumed under a lane-dependent branch)
  {
    const int l = lpos;
    const bool on = lon;
    float4_t xs;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float xv = -__builtin_inff();
      if (r < REP) {
        h16 a = (h16)((float)(h16)r1[r] * inv_scale);
        a = (h16)((float)a + mv);  // + 0 without a mask: the same value
        xv = on ? (float)a : -__builtin_inff();
      }
      xs[r] = xv;
    }
    s_x[l] = xs;
  }
  }

  // 3. values: thread (8 columns dg, positions ls + 64 i); loads out now
  const int dg = tid & 15, ls = tid >> 4;
  u32x4 vr[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int l = ls + 64 * i;
    const uint32_t vo = l < L ? (uint32_t)((l * HD + 8 * dg) * 2) : kOOB;
    vr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, vo, 0, 0));
  }
  __syncthreads();

  // 4. softmax of row r: wave w takes row w % REP, part w / REP of the
  //    positions (lane + 64 i within the part)
  {
    constexpr int PARTS = kAttnWaves / REP;
    constexpr int PER = LMAX / PARTS;  // positions per part
    constexpr int IT = (PER + 63) / 64;
    const int r = wave % REP, part = wave / REP;
    float x[IT];
    float mx = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int l = part * PER + lane + 64 * i;
      x[i] = (lane + 64 * i < PER && l < L) ? s_x[l][r] : -__builtin_inff();
      mx = mx > x[i] ? mx : x[i];
    }
    for (int off = 32; off > 0; off >>= 1) {
      const float o = __shfl_xor(mx, off, 64);
      mx = mx < o ? o : mx;
    }
    if (lane == 0) s_red[0][wave] = mx;
    __syncthreads();
    mx = s_red[0][r];
#pragma unroll
    for (int p2 = 1; p2 < PARTS; ++p2) mx = mx < s_red[0][r + REP * p2] ? s_red[0][r + REP * p2] : mx;
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      x[i] = expf(x[i] - mx);
      sum += x[i];
    }
    for (int off = 32; off > 0; off >>= 1) sum = sum + __shfl_xor(sum, off, 64);
    if (lane == 0) s_red[1][wave] = sum;
    __syncthreads();
    sum = s_red[1][r];
#pragma unroll
    for (int p2 = 1; p2 < PARTS; ++p2) sum += s_red[1][r + REP * p2];
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int l = part * PER + lane + 64 * i;
      if (lane + 64 * i < PER) s_x[l][r] = l < L ? (float)(h16)(x[i] / sum) : 0.f;
    }
  }
  __syncthreads();

  // 5. values: o[r][8 dg + j] over the thread's positions, v_dot2 over
  //    position pairs (i, i + 1): the values of two rows packed per column,
  //    the probabilities (fp16 values held in fp32, so the packing is exact)
  float oa[REP][8];
#pragma unroll
  for (int r = 0; r < REP; ++r)
#pragma unroll
    for (int j = 0; j < 8; ++j) oa[r][j] = 0.f;
#pragma unroll
  for (int i = 0; i < NV; i += 2) {
    if (64 * i < L) {  // uniform: past L the loads returned zero
      const float4_t pa = s_x[ls + 64 * i];
      const float4_t pb = s_x[ls + 64 * (i + 1)];
      u32x4 va = vr[i], vb = vr[i + 1];
      if (ROPE) {
        // the lanes of position pnew take the step's value
        u32x4 vn;
#pragma unroll
        for (int w = 0; w < 4; ++w) vn[w] = s_vnew[4 * dg + w];
        if (ls + 64 * i == pnew) va = vn;
        if (ls + 64 * (i + 1) == pnew) vb = vn;
      }
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t lo = __builtin_amdgcn_perm(vb[w], va[w], 0x05040100u);
        const uint32_t hi = __builtin_amdgcn_perm(vb[w], va[w], 0x07060302u);
#pragma unroll
        for (int r = 0; r < REP; ++r) {
          const half2_t p2 = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_pkrtz(pa[r], pb[r]));
          oa[r][2 * w] = __builtin_amdgcn_fdot2(p2, __builtin_bit_cast(half2_t, lo),
                                                oa[r][2 * w], false);
          oa[r][2 * w + 1] = __builtin_amdgcn_fdot2(p2, __builtin_bit_cast(half2_t, hi),
                                                    oa[r][2 * w + 1], false);
        }
      }
    }
  }
  // reduce-scatter over the wave's 4 position slices (lane bits 5, 4):
  // lane keeps columns 8 dg + 4 h5 + 2 h4 + {0, 1}
  float o4[REP][4], o2[REP][2];
  {
    const bool h = (lane >> 5) & 1;
#pragma unroll
    for (int r = 0; r < REP; ++r)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const float keep = h ? oa[r][4 + jj] : oa[r][jj];
        const float send = h ? oa[r][jj] : oa[r][4 + jj];
        o4[r][jj] = keep + __shfl_xor(send, 32, 64);
      }
  }
  {
    const bool h = (lane >> 4) & 1;
#pragma unroll
    for (int r = 0; r < REP; ++r)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const float keep = h ? o4[r][2 + jj] : o4[r][jj];
        const float send = h ? o4[r][jj] : o4[r][2 + jj];
        o2[r][jj] = keep + __shfl_xor(send, 16, 64);
      }
  }
  {
    const int c0 = 8 * dg + 4 * ((lane >> 5) & 1) + 2 * ((lane >> 4) & 1);
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      s_o[wave][r][c0] = o2[r][0];
      s_o[wave][r][c0 + 1] = o2[r][1];
    }
  }
  __syncthreads();
  if (tid < REP * HD) {
    const int r = tid / HD, d = tid - r * HD;
    float o = s_o[0][r][d];
#pragma unroll
    for (int w2 = 1; w2 < kAttnWaves; ++w2) o += s_o[w2][r][d];
    out[(long)b * ld_o + (long)(g * REP + r) * HD + d] = (h16)o;
  }
}
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
                     (const h16*)nullptr, 0L, 0, (float*)nullptr, UnpSrc{});
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
                     logits, UnpSrc{});
  HN_LAUNCH_CHECK("hn_add_rmsnorm_router");
  return 0;
}

// The MoE block's ordered unpermute (from the four fp32 K-slice partials of
// the down projection) + residual add + RMSNorm of the next block, one
// launch.  See include/hn_int4.h.
extern "C" int hn_unpermute_add_rmsnorm(const float* part, long ks_stride, long ld_y,
                                        const int* inv, const int* idx, const void* rw, long T,
                                        long k, const void* x, long ld_x, void* x_out,
                                        long ld_xo, const void* w, void* out, long ld_o, long H,
                                        float eps, void* stream) {
  const char* who = "hn_unpermute_add_rmsnorm";
  HN_ARG_CHECK(T >= 0 && H > 0 && H % 8 == 0 && H <= 8 * kNormThreads * 4,
               "%s: need 0 < H <= %d, H %% 8 == 0", who, 8 * kNormThreads * 4);
  HN_ARG_CHECK(k > 0 && k <= kMaxTopK, "%s: k must be in (0, %d]", who, kMaxTopK);
  HN_ARG_CHECK(al16(part) && ld_y % 4 == 0 && ks_stride % 4 == 0 && al16(x) && ld_x % 8 == 0 &&
                   al16(x_out) && ld_xo % 8 == 0 && al16(w) && al16(out) && ld_o % 8 == 0 &&
                   part && inv && idx && rw && x_out,
               "%s: partials, rows and weights must be 16-byte aligned (x_out given)", who);
  if (T == 0) return 0;
  const UnpSrc U = {part, ks_stride, ld_y, inv, idx, (const h16*)rw, (int)k};
  hipLaunchKernelGGL((add_rmsnorm_kernel<0, true>), dim3((unsigned)T), dim3(kNormThreads), 0,
                     (hipStream_t)stream, (const h16*)x, ld_x, (const h16*)nullptr, 0L,
                     (h16*)x_out, ld_xo, (const h16*)w, (h16*)out, ld_o, (int)H, eps,
                     (const h16*)nullptr, 0L, 0, (float*)nullptr, U);
  HN_LAUNCH_CHECK(who);
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

// Decode attention over the KV cache (one query token per sequence); with
// qkv, the step's RoPE and cache append too.
static int attn_decode(const char* who, const void* q, const void* qkv, long ld_qkv,
                       const float* cos_t, const float* sin_t, const long* pos, void* kt, void* v,
                       long max_len, long B, long nkv, long rep, long hd, long L,
                       const void* mask, float inv_scale, void* out, long ld_o, void* stream) {
  HN_ARG_CHECK(B >= 0 && nkv > 0 && (rep == 1 || rep == 2 || rep == 4) && hd == kAttnHd,
               "%s: need head_dim %d and 1, 2 or 4 query heads per KV head (rep=%ld hd=%ld)",
               who, kAttnHd, rep, hd);
  HN_ARG_CHECK(L >= 1 && L <= 1024 && max_len >= (L + 7) / 8 * 8,
               "%s: need 1 <= L <= 1024 and max_len >= L rounded up to 8 (L=%ld max_len=%ld)",
               who, L, max_len);
  HN_ARG_CHECK(hd * max_len * 2 < 0x7ffffff0L, "%s: one head's cache must stay below 2 GiB",
               who);
  HN_ARG_CHECK(al16(q) && al16(kt) && al16(v) && max_len % 8 == 0 && al16(out) && ld_o % 8 == 0 &&
                   ld_o >= nkv * rep * hd,
               "%s: q, caches and out must be 16-byte aligned (max_len %% 8 == 0)", who);
  HN_ARG_CHECK(!qkv || (((uintptr_t)qkv & 3) == 0 && ld_qkv % 2 == 0 &&
                        ld_qkv >= (nkv * rep + 2 * nkv) * hd && cos_t && sin_t && pos),
               "%s: qkv rows must be 4-byte aligned and hold q, k and v (with the RoPE "
               "tables and the position)", who);
  if (B == 0) return 0;
  const dim3 grid((unsigned)(B * nkv)), block(64 * kAttnWaves);
  hipStream_t st = (hipStream_t)stream;
#define HN_ATTN(R, LM)                                                                         \
  do {                                                                                       \
    if (qkv)                                                                                 \
      hipLaunchKernelGGL((attn_decode_kernel<R, LM, true>), grid, block, 0, st,              \
                         (const h16*)nullptr, (h16*)kt, (h16*)v, max_len, (int)nkv, (int)L,  \
                         (const h16*)mask, inv_scale, (h16*)out, ld_o, (const h16*)qkv,      \
                         ld_qkv, cos_t, sin_t, pos);                                         \
    else                                                                                     \
      hipLaunchKernelGGL((attn_decode_kernel<R, LM, false>), grid, block, 0, st,             \
                         (const h16*)q, (h16*)kt, (h16*)v, max_len, (int)nkv, (int)L,        \
                         (const h16*)mask, inv_scale, (h16*)out, ld_o, (const h16*)nullptr,  \
                         0L, (const float*)nullptr, (const float*)nullptr,                   \
                         (const long*)nullptr);                                              \
  } while (0)
#define HN_ATTN_L(R)             \
  if (L <= 256) HN_ATTN(R, 256);      \
  else if (L <= 512) HN_ATTN(R, 512); \
  else if (L <= 768) HN_ATTN(R, 768); \
  else HN_ATTN(R, 1024)
  if (rep == 1) { HN_ATTN_L(1); }
  else if (rep == 2) { HN_ATTN_L(2); }
  else { HN_ATTN_L(4); }
#undef HN_ATTN_L
#undef HN_ATTN
  HN_LAUNCH_CHECK(who);
  return 0;
}

// See include/hn_int4.h.
extern "C" int hn_attn_decode(const void* q, const void* kt, const void* v, long max_len, long B,
                              long nkv, long rep, long hd, long L, const void* mask,
                              float inv_scale, void* out, long ld_o, void* stream) {
  return attn_decode("hn_attn_decode", q, nullptr, 0, nullptr, nullptr, nullptr, (void*)kt,
                     (void*)v, max_len, B, nkv, rep, hd, L, mask, inv_scale, out, ld_o, stream);
}

// See include/hn_int4.h.
extern "C" int hn_attn_decode_rope(const void* qkv, long ld_qkv, const float* cos_t,
                                   const float* sin_t, const long* pos, void* kt, void* v,
                                   long max_len, long B, long nkv, long rep, long hd, long L,
                                   const void* mask, float inv_scale, void* out, long ld_o,
                                   void* stream) {
  const char* who = "hn_attn_decode_rope";
  HN_ARG_CHECK(qkv != nullptr, "%s: qkv is required", who);
  return attn_decode(who, nullptr, qkv, ld_qkv, cos_t, sin_t, pos, kt, v, max_len, B, nkv, rep,
                     hd, L, mask, inv_scale, out, ld_o, stream);
}
