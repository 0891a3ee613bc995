// W4A16 skinny GEMM for decode (a handful of tokens per weight matrix), gfx950.
//
//   out[m, n] = sum_k x[m, k] * W[n, k],  W[n, k] = (nibble - 8) * scale[n, k / group]
//
// Replaces the Triton int4_matmul_kernel (kernels/int4_gemm.py:25-121,
// kernels/int4_expert_mlp.py:15-96) for M <= 16 per token chunk, and fuses the
// SwiGLU epilogue of fused_silu_mul (kernels/int4_gemm.py:175-193):
//   h = fp16( silu(float(fp16(gate))) * float(fp16(up)) ).
//
// Mapping onto CDNA4:
//  * One workgroup owns a tile of 16 weight rows (the N side of one
//    v_mfma_f32_16x16x32_f16) and a chunk of up to 16 tokens (the M side).
//  * Its NW waves split K: wave w streams a contiguous range of 128-k groups.
//    Per group each lane issues ONE 16-byte load: row (n0 + lane%16), bytes
//    [16*(lane/16), +16) of the group's 64 bytes.  That 16 bytes is exactly
//    the B operand of four MFMA steps (4 x 8 k), so packed weights go from HBM
//    to registers once, are unpacked in registers and never touch LDS.
//  * Activations are staged once per workgroup into LDS, each 8-block permuted
//    to the unpack order, and read as the A operand with ds_read_b128.
//  * Group scales are applied to the fp32 MFMA partial of each 128-k group
//    (one fma per accumulator) when group % 128 == 0.  Otherwise (group 32/64)
//    the unpacked fp16 values are multiplied by the per-lane scale before the
//    MFMA, which reproduces the reference's fp16 dequantised weight exactly.
//  * Waves reduce through LDS; the epilogue writes fp16 (optionally SiLU*up).
#include "hn_common.h"

namespace {

constexpr int kTileN = 16;
constexpr int kTileM = 16;
constexpr int kLdsXBytes = 48 * 1024;  // x staging; + reduction stays <= 64 KB

struct W4Mat {
  const uint8_t* q;  // [N, K/2] packed nibbles
  const h16* s;      // [N, K/group] fp16 scales
  long ld_q;         // row stride in bytes
  long ld_s;         // row stride in elements
};

// Per-expert weight table entry used by the grouped launch (device memory).
struct ExpertW4 {
  const uint8_t* gate_q; const h16* gate_s;
  const uint8_t* up_q;   const h16* up_s;
  const uint8_t* down_q; const h16* down_s;
};

template <int MATS, int NW, int EPI, bool PREMUL, int LPB>
__device__ __forceinline__ void skinny_body(const h16* __restrict__ x, long ld_x, int Mc,
                                            const W4Mat* mats, h16* __restrict__ out, long ld_o,
                                            int n0, int N, int K, int group, int kc_groups,
                                            int lds_rows, unsigned char* smem) {
  constexpr int BATCH = LPB / MATS;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 15;  // weight row in the tile (B/D) and token (A)
  const int q = lane >> 4;    // 32-k sub-block of a 128-k group
  const int row = n0 + col;
  const bool row_ok = row < N;
  const int G = (K + 127) >> 7;
  const int ldx = kc_groups * 128 + 8;  // padded LDS row stride (halves)
  h16* xs = reinterpret_cast<h16*>(smem);
  float* red = reinterpret_cast<float*>(smem + (size_t)lds_rows * ldx * sizeof(h16));

  float4_t acc[MATS];
#pragma unroll
  for (int mt = 0; mt < MATS; ++mt) acc[mt] = float4_t{0.f, 0.f, 0.f, 0.f};

  for (int gc0 = 0; gc0 < G; gc0 += kc_groups) {
    const int gcn = min(kc_groups, G - gc0);
    __syncthreads();  // previous chunk's readers are done with xs
    {
      const int blocks8 = gcn * 16;
      for (int i = tid; i < Mc * blocks8; i += NW * 64) {
        const int m = i / blocks8;
        const int b = i - m * blocks8;
        const int k = gc0 * 128 + b * 8;
        half8_t v = {0, 0, 0, 0, 0, 0, 0, 0};
        if (k < K) v = *reinterpret_cast<const half8_t*>(x + (long)m * ld_x + k);
        half8_t p;
#pragma unroll
        for (int j = 0; j < 8; ++j) p[j] = v[hn_perm8(j)];
        *reinterpret_cast<half8_t*>(xs + m * ldx + b * 8) = p;
      }
    }
    __syncthreads();

    const int gw0 = (gcn * wave) / NW;
    const int gw1 = (gcn * (wave + 1)) / NW;
    for (int gb = gw0; gb < gw1; gb += BATCH) {
      const int nb = min(BATCH, gw1 - gb);
      u32x4 wq[MATS][BATCH];
      h16 sc[MATS][BATCH];
#pragma unroll
      for (int i = 0; i < BATCH; ++i) {
        const int g = gc0 + gb + i;
        const int kk = g * 128 + 32 * q;
        const bool ok = (i < nb) && row_ok && (kk < K);
#pragma unroll
        for (int mt = 0; mt < MATS; ++mt) {
          if (ok) {
            wq[mt][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
                mats[mt].q + (long)row * mats[mt].ld_q + (long)g * 64 + 16 * q));
            sc[mt][i] = mats[mt].s[(long)row * mats[mt].ld_s + (PREMUL ? kk : g * 128) / group];
          } else {
            wq[mt][i] = u32x4{0u, 0u, 0u, 0u};
            sc[mt][i] = (h16)0.0f;
          }
        }
      }
#pragma unroll
      for (int i = 0; i < BATCH; ++i) {
        if (i < nb) {
          const int gl = gb + i;
          half8_t a[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            if (col < Mc)
              a[t] = *reinterpret_cast<const half8_t*>(xs + col * ldx + gl * 128 + 32 * q + 8 * t);
            else
              a[t] = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
          }
#pragma unroll
          for (int mt = 0; mt < MATS; ++mt) {
            if (PREMUL) {
              const half2_t s2 = {sc[mt][i], sc[mt][i]};
#pragma unroll
              for (int t = 0; t < 4; ++t) {
                half2_t p[4];
                hn_unpack8_centered(wq[mt][i][t], p);
#pragma unroll
                for (int j = 0; j < 4; ++j) p[j] = p[j] * s2;
                acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[t], hn_cat4(p), acc[mt], 0, 0, 0);
              }
            } else {
              float4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
              for (int t = 0; t < 4; ++t) {
                half2_t p[4];
                hn_unpack8_centered(wq[mt][i][t], p);
                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[t], hn_cat4(p), c, 0, 0, 0);
              }
              const float s = (float)sc[mt][i];
#pragma unroll
              for (int r = 0; r < 4; ++r) acc[mt][r] = __builtin_fmaf(s, c[r], acc[mt][r]);
            }
          }
        }
      }
    }
  }

  // Cross-wave reduction: red[wave][mat][token][row]
#pragma unroll
  for (int mt = 0; mt < MATS; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      red[((wave * MATS + mt) * kTileM + 4 * q + r) * kTileN + col] = acc[mt][r];
  __syncthreads();
  if (tid < kTileM * kTileN) {
    const int m = tid >> 4;
    const int r = tid & 15;
    float v[MATS];
#pragma unroll
    for (int mt = 0; mt < MATS; ++mt) {
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) s += red[((w * MATS + mt) * kTileM + m) * kTileN + r];
      v[mt] = s;
    }
    if (m < Mc && n0 + r < N) {
      h16 o;
      if (EPI == 1) {
        const float g = (float)(h16)v[0];
        const float u = (float)(h16)v[MATS - 1];
        o = (h16)(hn_silu(g) * u);
      } else {
        o = (h16)v[0];
      }
      out[(long)m * ld_o + n0 + r] = o;
    }
  }
}

template <int MATS, int NW, int EPI, bool PREMUL, int LPB>
__global__ __launch_bounds__(NW * 64) void skinny_kernel(const h16* __restrict__ x, long ld_x,
                                                         int M, W4Mat w0, W4Mat w1,
                                                         h16* __restrict__ out, long ld_o, int N,
                                                         int K, int group, int kc_groups,
                                                         int lds_rows) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int m0 = blockIdx.y * kTileM;
  const int Mc = min(kTileM, M - m0);
  if (Mc <= 0) return;
  const W4Mat mats[2] = {w0, w1};
  skinny_body<MATS, NW, EPI, PREMUL, LPB>(x + (long)m0 * ld_x, ld_x, Mc, mats,
                                          out + (long)m0 * ld_o, ld_o, blockIdx.x * kTileN, N, K,
                                          group, kc_groups, lds_rows, smem);
}

// Grouped launch over the experts of one MoE layer.  Tokens are already
// permuted so that expert e owns rows [offsets[e], offsets[e+1]) of x.
// blockIdx.z walks the active-expert list; blockIdx.y walks 16-token chunks.
// PHASE 0: gate+up+SiLU (x = hidden, K = H, N = I); PHASE 1: down (K = I, N = H).
template <int PHASE, int NW, bool PREMUL, int LPB>
__global__ __launch_bounds__(NW * 64) void grouped_kernel(
    const h16* __restrict__ x, long ld_x, const ExpertW4* __restrict__ table,
    const int* __restrict__ active, const int* __restrict__ n_active,
    const int* __restrict__ offsets, h16* __restrict__ out, long ld_o, int H, int I, int group,
    int kc_groups, int lds_rows) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int a = blockIdx.z;
  if (a >= *n_active) return;
  const int e = active[a];
  const int t0 = offsets[e];
  const int Me = offsets[e + 1] - t0;
  const int m0 = blockIdx.y * kTileM;
  const int Mc = min(kTileM, Me - m0);
  if (Mc <= 0) return;
  const ExpertW4 ew = table[e];
  const long rowoff = (long)t0 + m0;
  if (PHASE == 0) {
    const W4Mat mats[2] = {{ew.gate_q, ew.gate_s, H / 2, H / group},
                           {ew.up_q, ew.up_s, H / 2, H / group}};
    skinny_body<2, NW, 1, PREMUL, LPB>(x + rowoff * ld_x, ld_x, Mc, mats, out + rowoff * ld_o,
                                       ld_o, blockIdx.x * kTileN, I, H, group, kc_groups,
                                       lds_rows, smem);
  } else {
    const W4Mat mats[2] = {{ew.down_q, ew.down_s, I / 2, I / group},
                           {ew.down_q, ew.down_s, I / 2, I / group}};
    skinny_body<1, NW, 0, PREMUL, LPB>(x + rowoff * ld_x, ld_x, Mc, mats, out + rowoff * ld_o,
                                       ld_o, blockIdx.x * kTileN, H, I, group, kc_groups,
                                       lds_rows, smem);
  }
}

__global__ __launch_bounds__(256) void silu_mul_kernel(const h16* __restrict__ g, long ld_g,
                                                       const h16* __restrict__ u, long ld_u,
                                                       h16* __restrict__ o, long ld_o, int M,
                                                       int N) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)M * N) return;
  const int m = (int)(i / N);
  const int n = (int)(i - (long)m * N);
  const float gv = (float)g[(long)m * ld_g + n];
  const float uv = (float)u[(long)m * ld_u + n];
  o[(long)m * ld_o + n] = (h16)(hn_silu(gv) * uv);
}

// Host-side launch configuration shared by the single and grouped paths.
struct SkinnyCfg {
  int kc_groups;
  int lds_rows;
  size_t lds_bytes;
};

SkinnyCfg skinny_cfg(int rows, int K, int mats, int nw) {
  SkinnyCfg c;
  const int G = (K + 127) / 128;
  c.lds_rows = rows < 1 ? 1 : (rows > kTileM ? kTileM : rows);
  int kc = kLdsXBytes / (c.lds_rows * 256 + 16);
  if (kc < 1) kc = 1;
  if (kc > G) kc = G;
  c.kc_groups = kc;
  c.lds_bytes = (size_t)c.lds_rows * (kc * 128 + 8) * 2 + (size_t)nw * mats * kTileM * kTileN * 4;
  return c;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

#define HN_SKINNY_LAUNCH(MATS, NW, EPI, PREMUL)                                                 \
  hipLaunchKernelGGL((skinny_kernel<MATS, NW, EPI, PREMUL, 16>), grid, dim3(NW * 64),           \
                     cfg.lds_bytes, s, (const h16*)x, ld_x, (int)M, w0, w1, (h16*)out, ld_o,     \
                     (int)N, (int)K, (int)group, cfg.kc_groups, cfg.lds_rows)

static int skinny_launch(int mats, int epi, const void* x, long ld_x, W4Mat w0, W4Mat w1,
                         void* out, long ld_o, long M, long N, long K, long group,
                         hipStream_t s, const char* who) {
  HN_ARG_CHECK(M >= 0 && N >= 0 && K >= 0, "%s: negative dims", who);
  HN_ARG_CHECK(K % 32 == 0, "%s: K=%ld must be a multiple of 32", who, K);
  HN_ARG_CHECK(group >= 32 && group % 32 == 0 && K % group == 0,
               "%s: group=%ld must be a multiple of 32 dividing K=%ld", who, group, K);
  HN_ARG_CHECK(aligned16(x) && ld_x % 8 == 0, "%s: x rows must be 16-byte aligned", who);
  HN_ARG_CHECK(aligned16(w0.q) && w0.ld_q % 16 == 0 && aligned16(w1.q) && w1.ld_q % 16 == 0,
               "%s: packed weight rows must be 16-byte aligned", who);
  if (M == 0 || N == 0) return 0;
  const bool premul = (group % 128) != 0;
  constexpr int NW = 8;
  const SkinnyCfg cfg = skinny_cfg((int)M, (int)K, mats, NW);
  dim3 grid(hn_cdiv(N, kTileN), hn_cdiv(M, kTileM));
  if (mats == 2) {
    if (premul) HN_SKINNY_LAUNCH(2, NW, 1, true);
    else HN_SKINNY_LAUNCH(2, NW, 1, false);
  } else {
    if (premul) HN_SKINNY_LAUNCH(1, NW, 0, true);
    else HN_SKINNY_LAUNCH(1, NW, 0, false);
  }
  (void)epi;
  HN_LAUNCH_CHECK(who);
  return 0;
}

// out[M, N] = x[M, K] @ deq(W)^T   (fp16 in/out, fp32 accumulation)
extern "C" int hn_int4_linear(const void* x, long ld_x, const void* wq, long ld_q,
                              const void* ws, long ld_s, void* out, long ld_o, long M, long N,
                              long K, long group, void* stream) {
  const W4Mat w = {(const uint8_t*)wq, (const h16*)ws, ld_q, ld_s};
  return skinny_launch(1, 0, x, ld_x, w, w, out, ld_o, M, N, K, group, (hipStream_t)stream,
                       "hn_int4_linear");
}

// h[M, N] = fp16(silu(fp16(x @ deq(Wg)^T)) * fp16(x @ deq(Wu)^T))
extern "C" int hn_int4_gate_up_silu(const void* x, long ld_x, const void* gq, const void* gs,
                                    const void* uq, const void* us, long ld_q, long ld_s,
                                    void* h, long ld_h, long M, long N, long K, long group,
                                    void* stream) {
  const W4Mat g = {(const uint8_t*)gq, (const h16*)gs, ld_q, ld_s};
  const W4Mat u = {(const uint8_t*)uq, (const h16*)us, ld_q, ld_s};
  return skinny_launch(2, 1, x, ld_x, g, u, h, ld_h, M, N, K, group, (hipStream_t)stream,
                       "hn_int4_gate_up_silu");
}

// Fused SwiGLU expert: out = down(silu(gate(x)) * up(x)); h is a caller-owned
// [T, I] fp16 workspace.  Two launches on the caller's stream.
extern "C" int hn_expert_mlp_int4(const void* x, const void* gq, const void* gs, const void* uq,
                                  const void* us, const void* dq, const void* ds, void* out,
                                  long T, long H, long I, long group, void* h_ws,
                                  void* stream) {
  HN_ARG_CHECK(H % 2 == 0 && I % 2 == 0, "hn_expert_mlp_int4: odd dims");
  HN_ARG_CHECK(group > 0 && H % group == 0 && I % group == 0,
               "hn_expert_mlp_int4: group=%ld must divide H=%ld and I=%ld", group, H, I);
  int rc = hn_int4_gate_up_silu(x, H, gq, gs, uq, us, H / 2, H / group, h_ws, I, T, I, H, group,
                                stream);
  if (rc) return rc;
  return hn_int4_linear(h_ws, I, dq, I / 2, ds, I / group, out, H, T, H, I, group, stream);
}

extern "C" int hn_silu_mul(const void* g, long ld_g, const void* u, long ld_u, void* out,
                           long ld_o, long M, long N, void* stream) {
  HN_ARG_CHECK(M >= 0 && N >= 0, "hn_silu_mul: negative dims");
  if (M == 0 || N == 0) return 0;
  hipLaunchKernelGGL(silu_mul_kernel, dim3(hn_cdiv(M * N, 256)), dim3(256), 0,
                     (hipStream_t)stream, (const h16*)g, ld_g, (const h16*)u, ld_u, (h16*)out,
                     ld_o, (int)M, (int)N);
  HN_LAUNCH_CHECK("hn_silu_mul");
  return 0;
}

// Grouped decode over one MoE layer.
//   x_perm [rows, H] fp16 (rows sorted by expert), table: E entries (device),
//   active[E_max], n_active[1], offsets[E+1] (device, from hn_moe_permute),
//   h_ws [rows, I] fp16 workspace, y_perm [rows, H] fp16 output.
//   max_rows_per_expert bounds the token chunks walked per expert.
extern "C" int hn_grouped_expert_mlp_int4(const void* x_perm, const void* table,
                                          const int* active, const int* n_active,
                                          const int* offsets, long E_max,
                                          long max_rows_per_expert, long H, long I, long group,
                                          void* h_ws, void* y_perm, void* stream) {
  HN_ARG_CHECK(E_max >= 0 && max_rows_per_expert >= 0, "hn_grouped_expert_mlp_int4: bad sizes");
  HN_ARG_CHECK(H % 128 == 0 && I % 32 == 0, "hn_grouped_expert_mlp_int4: H=%ld must be a "
               "multiple of 128 and I=%ld of 32", H, I);
  HN_ARG_CHECK(group >= 32 && group % 32 == 0 && H % group == 0 && I % group == 0,
               "hn_grouped_expert_mlp_int4: bad group=%ld", group);
  HN_ARG_CHECK(aligned16(x_perm) && aligned16(h_ws), "hn_grouped_expert_mlp_int4: misaligned");
  HN_ARG_CHECK((I / 2) % 16 == 0, "hn_grouped_expert_mlp_int4: down rows (I/2=%ld bytes) must "
               "be 16-byte aligned", I / 2);
  if (E_max == 0 || max_rows_per_expert == 0) return 0;
  hipStream_t s = (hipStream_t)stream;
  const bool premul = (group % 128) != 0;
  constexpr int NW = 8;
  const int chunks = hn_cdiv(max_rows_per_expert, kTileM);
  {
    const SkinnyCfg cfg = skinny_cfg((int)max_rows_per_expert, (int)H, 2, NW);
    dim3 grid(hn_cdiv(I, kTileN), chunks, (int)E_max);
    if (premul)
      hipLaunchKernelGGL((grouped_kernel<0, NW, true, 16>), grid, dim3(NW * 64), cfg.lds_bytes, s,
                         (const h16*)x_perm, H, (const ExpertW4*)table, active, n_active, offsets,
                         (h16*)h_ws, I, (int)H, (int)I, (int)group, cfg.kc_groups, cfg.lds_rows);
    else
      hipLaunchKernelGGL((grouped_kernel<0, NW, false, 16>), grid, dim3(NW * 64), cfg.lds_bytes,
                         s, (const h16*)x_perm, H, (const ExpertW4*)table, active, n_active,
                         offsets, (h16*)h_ws, I, (int)H, (int)I, (int)group, cfg.kc_groups,
                         cfg.lds_rows);
    HN_LAUNCH_CHECK("hn_grouped_expert_mlp_int4(gate_up)");
  }
  {
    const SkinnyCfg cfg = skinny_cfg((int)max_rows_per_expert, (int)I, 1, NW);
    dim3 grid(hn_cdiv(H, kTileN), chunks, (int)E_max);
    if (premul)
      hipLaunchKernelGGL((grouped_kernel<1, NW, true, 16>), grid, dim3(NW * 64), cfg.lds_bytes, s,
                         (const h16*)h_ws, I, (const ExpertW4*)table, active, n_active, offsets,
                         (h16*)y_perm, H, (int)H, (int)I, (int)group, cfg.kc_groups,
                         cfg.lds_rows);
    else
      hipLaunchKernelGGL((grouped_kernel<1, NW, false, 16>), grid, dim3(NW * 64), cfg.lds_bytes,
                         s, (const h16*)h_ws, I, (const ExpertW4*)table, active, n_active,
                         offsets, (h16*)y_perm, H, (int)H, (int)I, (int)group, cfg.kc_groups,
                         cfg.lds_rows);
    HN_LAUNCH_CHECK("hn_grouped_expert_mlp_int4(down)");
  }
  return 0;
}
