// W4A16 skinny GEMM for decode (a few tokens per weight matrix), gfx950.
//
//   out[m, n] = sum_k x[m, k] * W[n, k],  W[n, k] = (nibble - 8) * scale[n, k / group]
//
// Replaces the Triton int4_matmul_kernel (kernels/int4_gemm.py:25-121,
// kernels/int4_expert_mlp.py:15-96) for up to 64 tokens per weight matrix and
// fuses the SwiGLU epilogue of fused_silu_mul (kernels/int4_gemm.py:175-193):
//   h = fp16( silu(float(fp16(gate))) * float(fp16(up)) ).
//
// Decode is HBM-bound: the design goal is that every packed byte is requested
// from HBM as early as possible and exactly once.
//  * Work unit of one wave = (tile of 16 weight rows, k-chunk of <= 16/MATS
//    groups of 128 k).  Per group each lane issues ONE 16-byte load: row
//    (n0 + lane%16), bytes [16*(lane/16), +16) of the group's 64 bytes.  Those
//    16 bytes are the B operand of four v_mfma_f32_16x16x32_f16 steps.  All of
//    a wave's loads are in flight at once (no branches around loads; invalid
//    lanes read a clamped address and get scale 0).
//  * A workgroup = 4 waves on 4 consecutive tiles sharing one k-chunk; the
//    activations of that k-chunk are loaded FIRST (so waiting for them, in
//    vmcnt order, does not wait for the weights), permuted to the unpack order
//    and staged in LDS for the A operand.
//  * Tokens beyond 16 (up to 64) reuse the unpacked B operand with another
//    MFMA per 16-token chunk.
//  * K is split over blockIdx.y.  Each split writes fp32 partials; the last
//    split to finish a tile (atomic counter, which it resets to 0) sums the
//    partials in split order — deterministic — and runs the epilogue.
//  * Group scales multiply the fp32 MFMA partial of each 128-k group when
//    group % 128 == 0; for group 32/64 the unpacked fp16 values are multiplied
//    by the per-lane scale first, which is the reference's fp16 dequantised
//    weight exactly.
#include "hn_common.h"

namespace {

constexpr int kTileN = 16;
constexpr int kWaves = 4;                // waves (tiles) per workgroup
constexpr int kLoadsPerLane = 16;        // 16-byte weight loads in flight per lane
constexpr int kXChunkBytes = 32 * 1024;  // LDS activation chunk budget

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

struct SkinnyArgs {
  // single-problem operands (grouped launches resolve these per expert)
  const h16* x; long ld_x; int M;
  W4Mat w[2];
  h16* out; long ld_o;
  int N, K, group;
  int ks;          // k-splits (gridDim.y)
  int gpc;         // groups per k-chunk
  int ldx;         // LDS row stride of the x chunk (halves)
  float* partial;  // [ks][MATS][part_rows][N] fp32 when ks > 1
  int* counters;   // [E?][tiles] zero on entry, left zero on exit
  long part_rows;  // row capacity of one (split, mat) partial plane
  // grouped mode
  const ExpertW4* table;
  const int* active;
  const int* n_active;
  const int* offsets;
  int phase;       // 0 = gate/up (+SiLU), 1 = down
  int H, I;
};

template <int MATS, int EPI, bool PREMUL, int NCH, int XR>
__device__ __forceinline__ void skinny_unit(const SkinnyArgs& A, const h16* __restrict__ x,
                                            int Mc, const W4Mat* mats, h16* __restrict__ out,
                                            float* __restrict__ part, int* __restrict__ ctr,
                                            int tile0, unsigned char* smem) {
  constexpr int BATCH = kLoadsPerLane / MATS;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 15;  // weight row in the tile (B/D), token in a 16-chunk (A)
  const int q = lane >> 4;    // 32-k sub-block of a 128-k group
  const int N = A.N, K = A.K, group = A.group;
  const int G = (K + 127) >> 7;
  const int ks = blockIdx.y;
  const int g0 = ks * A.gpc;
  const int gn = min(A.gpc, G - g0);  // groups in this k-chunk (>= 1)
  const int tile = tile0 + wave;
  const int tiles = (N + kTileN - 1) / kTileN;
  const bool tile_ok = tile < tiles;
  const int n0 = tile * kTileN;
  const int row = n0 + col;
  const bool row_ok = tile_ok && row < N;
  const int row_c = min(row, N - 1);
  const int ldx = A.ldx;
  h16* xs = reinterpret_cast<h16*>(smem);

  // ---- 1. activation chunk -> registers (issued before the weights; branch-free
  //         so the wait for them lands after the weight loads are issued)
  constexpr int kXRegs = XR;  // XR x 16 B of activations per thread
  const int blocks8 = gn * 16;
  const int nblk = Mc * blocks8;
  half8_t xr[kXRegs];
#pragma unroll
  for (int j = 0; j < kXRegs; ++j) {
    const int i = min(tid + j * kWaves * 64, nblk - 1);
    const int m = i / blocks8;
    const int b = i - m * blocks8;
    const int k = min(g0 * 128 + b * 8, K - 8);
    xr[j] = *reinterpret_cast<const half8_t*>(x + (long)m * A.ld_x + k);
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the activation loads ahead of the weights

  // ---- 2. weights and scales of this wave's unit, all in flight
  u32x4 wq[MATS][BATCH];
  h16 sc[MATS][BATCH];
#pragma unroll
  for (int i = 0; i < BATCH; ++i) {
    const int g = min(g0 + i, G - 1);
    const int kk_c = min(g * 128 + 32 * q, K - 32);
#pragma unroll
    for (int mt = 0; mt < MATS; ++mt) {
      wq[mt][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
          mats[mt].q + (long)row_c * mats[mt].ld_q + (long)(kk_c >> 1)));
      sc[mt][i] = mats[mt].s[(long)row_c * mats[mt].ld_s + (PREMUL ? kk_c : g * 128) / group];
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- 3. stage the activations (waits for them only), permuted to unpack order
#pragma unroll
  for (int j = 0; j < kXRegs; ++j) {
    const int i = tid + j * kWaves * 64;
    if (i < nblk) {
      const int m = i / blocks8;
      const int b = i - m * blocks8;
      const bool in_k = g0 * 128 + b * 8 < K;
      half8_t p;
#pragma unroll
      for (int t = 0; t < 8; ++t) p[t] = in_k ? xr[j][hn_perm8(t)] : (h16)0.0f;
      *reinterpret_cast<half8_t*>(xs + m * ldx + b * 8) = p;
    }
  }
  __syncthreads();

  // ---- 4. unpack + MFMA
  float4_t acc[NCH][MATS];
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int mt = 0; mt < MATS; ++mt) acc[c][mt] = float4_t{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int i = 0; i < BATCH; ++i) {
    if (i < gn) {  // uniform
      const bool ok = row_ok && ((g0 + i) * 128 + 32 * q < K);
#pragma unroll
      for (int mt = 0; mt < MATS; ++mt) {
        const h16 s16 = ok ? sc[mt][i] : (h16)0.0f;
        half8_t b[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          half2_t p[4];
          hn_unpack8_centered(wq[mt][i][t], p);
          if (PREMUL) {
            const half2_t s2 = {s16, s16};
#pragma unroll
            for (int j = 0; j < 4; ++j) p[j] = p[j] * s2;
          }
          b[t] = hn_cat4(p);
        }
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
          const int tok = c * 16 + col;
          float4_t cc = {0.f, 0.f, 0.f, 0.f};
          if (PREMUL) cc = acc[c][mt];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            half8_t a = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
            if (tok < Mc)
              a = *reinterpret_cast<const half8_t*>(xs + tok * ldx + i * 128 + 32 * q + 8 * t);
            cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[t], cc, 0, 0, 0);
          }
          if (PREMUL) {
            acc[c][mt] = cc;
          } else {
            const float s = (float)s16;
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[c][mt][r] = __builtin_fmaf(s, cc[r], acc[c][mt][r]);
          }
        }
      }
    }
  }

  // ---- 5. output: D lane layout is row (n0 + col), tokens 16c + 4q + r
  if (!tile_ok) return;
  if (A.ks == 1) {
    if (row_ok) {
#pragma unroll
      for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = c * 16 + 4 * q + r;
          if (m < Mc) {
            h16 o;
            if (EPI == 1) {
              o = (h16)(hn_silu((float)(h16)acc[c][0][r]) * (float)(h16)acc[c][MATS - 1][r]);
            } else {
              o = (h16)acc[c][0][r];
            }
            out[(long)m * A.ld_o + row] = o;
          }
        }
    }
    return;
  }
  // split-K: write partials, last split of this tile reduces in split order.
  // Partials and counters are relaxed agent-scope atomics (sc1 accesses,
  // coherent across XCDs without writing back or invalidating the L2); the
  // s_waitcnt orders "partials stored" before "counter incremented".
  const long plane = A.part_rows * (long)N;
  if (row_ok) {
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = c * 16 + 4 * q + r;
        if (m < Mc)
#pragma unroll
          for (int mt = 0; mt < MATS; ++mt)
            __hip_atomic_store(part + (long)(ks * MATS + mt) * plane + (long)m * N + row,
                               acc[c][mt][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
  }
  __builtin_amdgcn_s_waitcnt(0);
  int last = 0;
  if (lane == 0)
    last = __hip_atomic_fetch_add(ctr + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           A.ks - 1;
  last = __shfl(last, 0, 64);
  if (!last) return;
  if (lane == 0) __hip_atomic_store(ctr + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // this wave now owns the tile's 16 rows x Mc tokens: lanes walk (token, row)
  for (int e = lane; e < Mc * kTileN; e += 64) {
    const int m = e / kTileN;
    const int rr = n0 + (e % kTileN);
    if (rr >= N) continue;
    float v[MATS];
#pragma unroll
    for (int mt = 0; mt < MATS; ++mt) {
      float s = 0.f;
      for (int k2 = 0; k2 < A.ks; ++k2)
        s += __hip_atomic_load(part + (long)(k2 * MATS + mt) * plane + (long)m * N + rr,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      v[mt] = s;
    }
    h16 o;
    if (EPI == 1) o = (h16)(hn_silu((float)(h16)v[0]) * (float)(h16)v[MATS - 1]);
    else o = (h16)v[0];
    out[(long)m * A.ld_o + rr] = o;
  }
}

template <int MATS, int EPI, bool PREMUL, int NCH, int XR>
__global__ __launch_bounds__(kWaves * 64) void skinny_kernel(SkinnyArgs A) {
  extern __shared__ __align__(16) unsigned char smem[];
  const W4Mat mats[2] = {A.w[0], A.w[1]};
  skinny_unit<MATS, EPI, PREMUL, NCH, XR>(A, A.x, A.M, mats, A.out, A.partial, A.counters,
                                      blockIdx.x * kWaves, smem);
}

// Grouped launch over the experts of one MoE layer; tokens are permuted so
// expert e owns rows [offsets[e], offsets[e+1]).  blockIdx.z walks the
// active-expert list (device), so no host sync is needed.
template <int PHASE, bool PREMUL, int NCH, int XR>
__global__ __launch_bounds__(kWaves * 64) void grouped_kernel(SkinnyArgs A) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int a = blockIdx.z;
  if (a >= *A.n_active) return;
  const int e = A.active[a];
  const int t0 = A.offsets[e];
  const int Me = min(A.offsets[e + 1] - t0, A.M);  // A.M: rows the plan was sized for
  if (Me <= 0) return;
  const ExpertW4 ew = A.table[e];
  const int H = A.H, I = A.I, g = A.group;
  const int tmax = max((H + kTileN - 1) / kTileN, (I + kTileN - 1) / kTileN);
  int* ctr = A.counters + (long)e * tmax;
  float* part = A.partial + (long)t0 * A.N;  // row offset inside each plane
  if (PHASE == 0) {
    const W4Mat mats[2] = {{ew.gate_q, ew.gate_s, H / 2, H / g}, {ew.up_q, ew.up_s, H / 2, H / g}};
    skinny_unit<2, 1, PREMUL, NCH, XR>(A, A.x + (long)t0 * A.ld_x, Me, mats,
                                   A.out + (long)t0 * A.ld_o, part, ctr, blockIdx.x * kWaves, smem);
  } else {
    const W4Mat mats[2] = {{ew.down_q, ew.down_s, I / 2, I / g},
                           {ew.down_q, ew.down_s, I / 2, I / g}};
    skinny_unit<1, 0, PREMUL, NCH, XR>(A, A.x + (long)t0 * A.ld_x, Me, mats,
                                   A.out + (long)t0 * A.ld_o, part, ctr, blockIdx.x * kWaves, smem);
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

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// k-split plan: groups per chunk limited by the load budget and the LDS chunk.
struct Plan {
  int ks, gpc, ldx, nch, xr;
  size_t lds;
};

Plan make_plan(int rows, int K, int mats) {
  Plan p;
  const int G = (K + 127) / 128;
  int gpc = kLoadsPerLane / mats;
  const int by_lds = kXChunkBytes / (rows * 256 + 16 * rows);
  if (by_lds < gpc) gpc = by_lds < 1 ? 1 : by_lds;
  // the x staging registers hold at most 8 x 16 B per thread
  while (gpc > 1 && rows * gpc * 16 > 8 * kWaves * 64) --gpc;
  if (gpc > G) gpc = G;
  p.gpc = gpc;
  p.ks = (G + gpc - 1) / gpc;
  p.ldx = gpc * 128 + 8;
  p.nch = rows <= 16 ? 1 : rows <= 32 ? 2 : 4;
  // activation registers per thread (variants 1, 2, 8; 8 whenever NCH > 1)
  const int need = (rows * gpc * 16 + kWaves * 64 - 1) / (kWaves * 64);
  p.xr = (p.nch == 1 && need <= 1) ? 1 : (p.nch == 1 && need <= 2) ? 2 : 8;
  p.lds = (size_t)rows * p.ldx * 2;
  return p;
}

#define HN_SKINNY_VARIANTS(KERNEL, ...)                                                    \
  do {                                                                                     \
    if (p.nch == 1 && p.xr == 1)                                                           \
      hipLaunchKernelGGL((KERNEL<__VA_ARGS__, 1, 1>), grid, block, p.lds, s, A);           \
    else if (p.nch == 1 && p.xr == 2)                                                      \
      hipLaunchKernelGGL((KERNEL<__VA_ARGS__, 1, 2>), grid, block, p.lds, s, A);           \
    else if (p.nch == 1)                                                                   \
      hipLaunchKernelGGL((KERNEL<__VA_ARGS__, 1, 8>), grid, block, p.lds, s, A);           \
    else if (p.nch == 2)                                                                   \
      hipLaunchKernelGGL((KERNEL<__VA_ARGS__, 2, 8>), grid, block, p.lds, s, A);           \
    else                                                                                   \
      hipLaunchKernelGGL((KERNEL<__VA_ARGS__, 4, 8>), grid, block, p.lds, s, A);           \
  } while (0)

template <int MATS, int EPI, bool PREMUL>
int launch_single(SkinnyArgs& A, const Plan& p, hipStream_t s) {
  dim3 grid(hn_cdiv(hn_cdiv(A.N, kTileN), kWaves), p.ks, 1), block(kWaves * 64);
  HN_SKINNY_VARIANTS(skinny_kernel, MATS, EPI, PREMUL);
  return 0;
}

template <int PHASE, bool PREMUL>
void launch_grouped(SkinnyArgs& A, const Plan& p, int E_max, hipStream_t s) {
  dim3 grid(hn_cdiv(hn_cdiv(A.N, kTileN), kWaves), p.ks, E_max), block(kWaves * 64);
  HN_SKINNY_VARIANTS(grouped_kernel, PHASE, PREMUL);
}

constexpr int kMaxRows = 64;  // tokens per weight matrix handled per launch

// workspace layout: [counters: one region shared by every launch of a call][partials]
size_t ctr_bytes(long counters) { return ((size_t)counters * 4 + 255) & ~(size_t)255; }

size_t part_bytes(int ks, int mats, long rows, long N) {
  return ks > 1 ? (size_t)ks * mats * rows * N * 4 : 0;
}

}  // namespace

// Bytes of workspace hn_int4_linear / hn_int4_gate_up_silu / hn_expert_mlp_int4 /
// hn_grouped_expert_mlp_int4 need.  kind: 0 linear (M,N,K), 1 gate_up (M,N=I,K=H),
// 2 expert mlp (M=T, N=H, K=I), 3 grouped (M=rows=T*k, N=H, K=I, E).
extern "C" long hn_skinny_workspace_bytes(int kind, long M, long N, long K, long E) {
  const long rows = M < 1 ? 1 : M;
  const int r = (int)(rows > kMaxRows ? kMaxRows : rows);
  if (kind == 0 || kind == 1) {
    const int mats = kind == 0 ? 1 : 2;
    const Plan p = make_plan(r, (int)K, mats);
    return (long)(ctr_bytes(hn_cdiv(N, kTileN)) + part_bytes(p.ks, mats, r, N));
  }
  // kind 2: expert MLP, N = H, K = I.  kind 3: grouped over E experts, M = all rows.
  const long H = N, I = K;
  const long ctr = (kind == 3 ? E : 1) * (long)(hn_cdiv(I, kTileN) > hn_cdiv(H, kTileN)
                                                  ? hn_cdiv(I, kTileN) : hn_cdiv(H, kTileN));
  const long prow = kind == 3 ? rows : r;
  const Plan pg = make_plan(r, (int)H, 2);
  const Plan pd = make_plan(r, (int)I, 1);
  const size_t a = part_bytes(pg.ks, 2, prow, I);
  const size_t b = part_bytes(pd.ks, 1, prow, H);
  return (long)(ctr_bytes(ctr) + (a > b ? a : b));
}

static int check_common(const char* who, long M, long N, long K, long group, const void* x,
                        long ld_x) {
  HN_ARG_CHECK(M >= 0 && N >= 0 && K >= 0, "%s: negative dims", who);
  HN_ARG_CHECK(K % 32 == 0 && K > 0, "%s: K=%ld must be a positive multiple of 32", who, K);
  HN_ARG_CHECK(group >= 32 && group % 32 == 0 && K % group == 0,
               "%s: group=%ld must be a multiple of 32 dividing K=%ld", who, group, K);
  HN_ARG_CHECK(aligned16(x) && ld_x % 8 == 0, "%s: x rows must be 16-byte aligned", who);
  return 0;
}

static int run_single(int mats, const void* x, long ld_x, W4Mat w0, W4Mat w1, void* out,
                      long ld_o, long M, long N, long K, long group, void* ws, long ws_size,
                      long n_counters, hipStream_t s, const char* who) {
  if (int rc = check_common(who, M, N, K, group, x, ld_x)) return rc;
  HN_ARG_CHECK(aligned16(w0.q) && w0.ld_q % 16 == 0 && aligned16(w1.q) && w1.ld_q % 16 == 0,
               "%s: packed weight rows must be 16-byte aligned", who);
  if (M == 0 || N == 0) return 0;
  const bool premul = (group % 128) != 0;
  const int tiles = hn_cdiv(N, kTileN);
  for (long m0 = 0; m0 < M; m0 += kMaxRows) {
    const int rows = (int)((M - m0) > kMaxRows ? kMaxRows : (M - m0));
    const Plan p = make_plan(rows, (int)K, mats);
    const size_t cb = ctr_bytes(n_counters < tiles ? tiles : n_counters);
    const size_t need = cb + part_bytes(p.ks, mats, rows, N);
    HN_ARG_CHECK(p.ks == 1 || (ws && (size_t)ws_size >= need),
                 "%s: workspace too small (%ld < %zu bytes)", who, ws_size, need);
    SkinnyArgs A = {};
    A.x = (const h16*)x + m0 * ld_x;
    A.ld_x = ld_x;
    A.M = rows;
    A.w[0] = w0;
    A.w[1] = w1;
    A.out = (h16*)out + m0 * ld_o;
    A.ld_o = ld_o;
    A.N = (int)N;
    A.K = (int)K;
    A.group = (int)group;
    A.ks = p.ks;
    A.gpc = p.gpc;
    A.ldx = p.ldx;
    A.counters = (int*)ws;
    A.partial = ws ? (float*)((char*)ws + cb) : nullptr;
    A.part_rows = rows;
    if (mats == 2) {
      if (premul) launch_single<2, 1, true>(A, p, s);
      else launch_single<2, 1, false>(A, p, s);
    } else {
      if (premul) launch_single<1, 0, true>(A, p, s);
      else launch_single<1, 0, false>(A, p, s);
    }
    HN_LAUNCH_CHECK(who);
  }
  return 0;
}

// out[M, N] = x[M, K] @ deq(W)^T   (fp16 in/out, fp32 accumulation)
extern "C" int hn_int4_linear(const void* x, long ld_x, const void* wq, long ld_q,
                              const void* ws, long ld_s, void* out, long ld_o, long M, long N,
                              long K, long group, void* work, long work_bytes, void* stream) {
  const W4Mat w = {(const uint8_t*)wq, (const h16*)ws, ld_q, ld_s};
  return run_single(1, x, ld_x, w, w, out, ld_o, M, N, K, group, work, work_bytes, 0,
                    (hipStream_t)stream, "hn_int4_linear");
}

// h[M, N] = fp16(silu(fp16(x @ deq(Wg)^T)) * fp16(x @ deq(Wu)^T))
extern "C" int hn_int4_gate_up_silu(const void* x, long ld_x, const void* gq, const void* gs,
                                    const void* uq, const void* us, long ld_q, long ld_s,
                                    void* h, long ld_h, long M, long N, long K, long group,
                                    void* work, long work_bytes, void* stream) {
  const W4Mat g = {(const uint8_t*)gq, (const h16*)gs, ld_q, ld_s};
  const W4Mat u = {(const uint8_t*)uq, (const h16*)us, ld_q, ld_s};
  return run_single(2, x, ld_x, g, u, h, ld_h, M, N, K, group, work, work_bytes, 0,
                    (hipStream_t)stream, "hn_int4_gate_up_silu");
}

// Fused SwiGLU expert: out = down(silu(gate(x)) * up(x)); h is a caller-owned
// [T, I] fp16 buffer; work is hn_skinny_workspace_bytes(2, T, H, I, 0) bytes.
extern "C" int hn_expert_mlp_int4(const void* x, const void* gq, const void* gs, const void* uq,
                                  const void* us, const void* dq, const void* ds, void* out,
                                  long T, long H, long I, long group, void* h_ws, void* work,
                                  long work_bytes, void* stream) {
  HN_ARG_CHECK(H % 2 == 0 && I % 2 == 0, "hn_expert_mlp_int4: odd dims");
  HN_ARG_CHECK(group > 0 && H % group == 0 && I % group == 0,
               "hn_expert_mlp_int4: group=%ld must divide H=%ld and I=%ld", group, H, I);
  // both launches share one counter region (each leaves its counters at zero)
  const long nctr = hn_cdiv(I, kTileN) > hn_cdiv(H, kTileN) ? hn_cdiv(I, kTileN)
                                                            : hn_cdiv(H, kTileN);
  const W4Mat g = {(const uint8_t*)gq, (const h16*)gs, H / 2, H / group};
  const W4Mat u = {(const uint8_t*)uq, (const h16*)us, H / 2, H / group};
  const W4Mat d = {(const uint8_t*)dq, (const h16*)ds, I / 2, I / group};
  int rc = run_single(2, x, H, g, u, h_ws, I, T, I, H, group, work, work_bytes, nctr,
                      (hipStream_t)stream, "hn_expert_mlp_int4(gate_up)");
  if (rc) return rc;
  return run_single(1, h_ws, I, d, d, out, H, T, H, I, group, work, work_bytes, nctr,
                    (hipStream_t)stream, "hn_expert_mlp_int4(down)");
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

// Grouped decode over one MoE layer (<= 64 rows per expert).
//   x_perm [rows, H] fp16 sorted by expert; table: E x ExpertW4 (device);
//   active[E], n_active[1], offsets[E+1] from hn_moe_permute; h_ws [rows, I];
//   y_perm [rows, H]; work = hn_skinny_workspace_bytes(3, rows, H, I, E) bytes.
extern "C" int hn_grouped_expert_mlp_int4(const void* x_perm, const void* table,
                                          const int* active, const int* n_active,
                                          const int* offsets, long E, long max_rows_per_expert,
                                          long rows, long H, long I, long group, void* h_ws,
                                          void* y_perm, void* work, long work_bytes,
                                          void* stream) {
  const char* who = "hn_grouped_expert_mlp_int4";
  HN_ARG_CHECK(E > 0 && max_rows_per_expert >= 0 && rows >= 0, "%s: bad sizes", who);
  HN_ARG_CHECK(max_rows_per_expert <= kMaxRows, "%s: at most %d rows per expert (got %ld); "
               "use the grouped prefill GEMM", who, kMaxRows, max_rows_per_expert);
  HN_ARG_CHECK(H % 128 == 0 && I % 32 == 0, "%s: H=%ld must be a multiple of 128, I=%ld of 32",
               who, H, I);
  HN_ARG_CHECK(group >= 32 && group % 32 == 0 && H % group == 0 && I % group == 0,
               "%s: bad group=%ld", who, group);
  HN_ARG_CHECK(aligned16(x_perm) && aligned16(h_ws) && aligned16(y_perm), "%s: misaligned", who);
  HN_ARG_CHECK((I / 2) % 16 == 0, "%s: down rows (I/2=%ld bytes) must be 16-byte aligned", who,
               I / 2);
  if (max_rows_per_expert == 0 || rows == 0) return 0;
  const long need = hn_skinny_workspace_bytes(3, rows, H, I, E);
  HN_ARG_CHECK(work && work_bytes >= need, "%s: workspace too small (%ld < %ld)", who, work_bytes,
               need);
  hipStream_t s = (hipStream_t)stream;
  const bool premul = (group % 128) != 0;
  const int rmax = (int)max_rows_per_expert;
  SkinnyArgs A = {};
  A.table = (const ExpertW4*)table;
  A.active = active;
  A.n_active = n_active;
  A.offsets = offsets;
  A.H = (int)H;
  A.I = (int)I;
  A.group = (int)group;
  A.counters = (int*)work;
  A.part_rows = rows;
  A.M = rmax;
  const long tmax = hn_cdiv(I, kTileN) > hn_cdiv(H, kTileN) ? hn_cdiv(I, kTileN)
                                                            : hn_cdiv(H, kTileN);
  float* partial = (float*)((char*)work + ctr_bytes(E * tmax));
  {
    const Plan p = make_plan(rmax, (int)H, 2);
    A.x = (const h16*)x_perm; A.ld_x = H;
    A.out = (h16*)h_ws; A.ld_o = I;
    A.N = (int)I; A.K = (int)H;
    A.ks = p.ks; A.gpc = p.gpc; A.ldx = p.ldx;
    A.partial = partial;
    A.phase = 0;
    if (premul) launch_grouped<0, true>(A, p, (int)E, s);
    else launch_grouped<0, false>(A, p, (int)E, s);
    HN_LAUNCH_CHECK("hn_grouped_expert_mlp_int4(gate_up)");
  }
  {
    const Plan p = make_plan(rmax, (int)I, 1);
    A.x = (const h16*)h_ws; A.ld_x = I;
    A.out = (h16*)y_perm; A.ld_o = H;
    A.N = (int)H; A.K = (int)I;
    A.ks = p.ks; A.gpc = p.gpc; A.ldx = p.ldx;
    A.partial = partial;
    A.phase = 1;
    if (premul) launch_grouped<1, true>(A, p, (int)E, s);
    else launch_grouped<1, false>(A, p, (int)E, s);
    HN_LAUNCH_CHECK("hn_grouped_expert_mlp_int4(down)");
  }
  return 0;
}
