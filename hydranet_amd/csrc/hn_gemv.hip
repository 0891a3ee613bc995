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
//  * Work unit of one wave = (tile of 16 weight rows, gpw <= 16/MATS groups of
//    128 k).  Per group each lane issues ONE 16-byte load: row (n0 + lane%16),
//    bytes [16*(lane/16), +16) of the group's 64 bytes.  Those 16 bytes are the
//    B operand of four v_mfma_f32_16x16x32_f16 steps.  All of a wave's loads
//    are in flight at once (no branches around loads; invalid lanes read a
//    clamped address and get scale 0).
//  * A workgroup = TG tiles x KW waves per tile.  The KW waves of a tile split
//    its k-chunk and reduce through LDS (fixed order), so a tile is finished
//    on chip and the epilogue writes the result directly.  The activations of
//    the workgroup's k-chunk are staged once in LDS (permuted to the unpack
//    order) for the A operand.
//  * Only when the activation chunk would not fit in LDS is K also split over
//    workgroups (blockIdx.y): each split writes fp32 partials, the last split
//    of a tile (tagged counter, hn_arrive; acquire at agent scope)
//    sums them in split order — deterministic — and runs the epilogue.
//  * Tokens beyond 16 (up to 64) reuse the unpacked B operand with another
//    MFMA per 16-token chunk.
//  * Group scales multiply the fp32 MFMA partial of each 128-k group when
//    group % 128 == 0; for group 32/64 the unpacked fp16 values are multiplied
//    by the per-lane scale first, which is the reference's fp16 dequantised
//    weight exactly.
#include "hn_common.h"

namespace {

constexpr int kTileN = 16;
constexpr int kMaxWaves = 8;             // waves per workgroup (TG * KW)
constexpr int kLoadsPerLane = 16;        // 16-byte weight loads in flight per lane
constexpr int kLdsBudget = 64 * 1024;    // activation chunk + wave reduction
constexpr int kMaxKS = 64;               // cross-workgroup k-splits

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
  int ks;          // k-splits over workgroups (gridDim.y)
  int gpc;         // groups per workgroup k-chunk
  int gpw;         // groups per wave (gpc split over the KW waves of a tile)
  int kw;          // waves per tile
  int tg;          // tiles per workgroup
  int ldx;         // LDS row stride of the x chunk (halves)
  float* partial;  // [ks][MATS][part_rows][N] fp32 when ks > 1
  unsigned long long* counters;  // [E?][tiles] tagged counters (hn_arrive), left zero
  unsigned long long tag;        // this launch's counter tag (hn_next_tag)
  long part_rows;  // row capacity of one (split, mat) partial plane
  // grouped mode
  const ExpertW4* table;
  const int* active;
  const int* n_active;
  const int* offsets;
  int phase;       // 0 = gate/up (+SiLU), 1 = down
  int H, I;
  // unpack constants as registers (see hn_unpack8_regs)
  uint32_t m_lo, m_hi, magic;
};

template <int MATS, int EPI, bool PREMUL, int NCH, int XR>
__device__ __forceinline__ void skinny_unit(const SkinnyArgs& A, const h16* __restrict__ x,
                                            int Mc, const W4Mat* mats, h16* __restrict__ out,
                                            float* __restrict__ part,
                                            unsigned long long* __restrict__ ctr,
                                            unsigned char* smem) {
  constexpr int BATCH = kLoadsPerLane / MATS;  // loads per lane per matrix (even)
  static_assert(BATCH % 2 == 0, "groups are loaded in pairs");
  const int tid = threadIdx.x;
  const int nthr = blockDim.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave
  const int col = lane & 15;  // MFMA column (weight row in the tile) / token in a 16-chunk
  const int q = lane >> 4;    // 32-k sub-block of a 128-k group
  const int N = A.N, K = A.K, group = A.group;
  const int G = (K + 127) >> 7;
  const int ks = blockIdx.y;
  HnUnpackRegs ur;
  ur.m_lo = A.m_lo;
  ur.m_hi = A.m_hi;
  ur.magic = hn_vgpr(A.magic);
  ur.bias_lo = hn_vgpr(0xE408E408u);    // half2(-1032, -1032)
  ur.sixteenth = hn_vgpr(0x2C002C00u);  // half2(0.0625, 0.0625)
  ur.bias_hi = hn_vgpr(0xD480D480u);    // half2(-72, -72)
  const int g0 = ks * A.gpc;                 // first group of the workgroup chunk
  const int gn = min(A.gpc, G - g0);         // groups in the chunk (>= 1)
  const int gn2 = (gn + 1) & ~1;             // staged groups (pairs; the pad is zero)
  const int kwi = wave % A.kw;               // k-slice of this wave within the chunk
  const int tile = blockIdx.x * A.tg + wave / A.kw;
  const int gl0 = kwi * A.gpw;               // first chunk-local group of this wave (even)
  const int gw = max(0, min(A.gpw, gn - gl0));  // groups of this wave (uniform)
  const int tiles = (N + kTileN - 1) / kTileN;
  const bool tile_ok = tile < tiles;
  const int n0 = tile * kTileN;
  const int ldx = A.ldx;
  h16* xs = reinterpret_cast<h16*>(smem);

  // ---- 1. activation chunk -> registers -> LDS (permuted to the unpack order)
  const int blocks8 = gn2 * 16;
  const int nblk = Mc * blocks8;
  half8_t xr[XR];
#pragma unroll
  for (int j = 0; j < XR; ++j) {
    const int i = min(tid + j * nthr, nblk - 1);
    const int m = i / blocks8;
    const int b = i - m * blocks8;
    const int k = min(g0 * 128 + b * 8, K - 8);
    xr[j] = *reinterpret_cast<const half8_t*>(x + (long)m * A.ld_x + k);
  }
#pragma unroll
  for (int j = 0; j < XR; ++j) {
    const int i = tid + j * nthr;
    if (i < nblk) {
      const int m = i / blocks8;
      const int b = i - m * blocks8;
      const bool in_k = (b < gn * 16) && (g0 * 128 + b * 8 < K);
      half8_t p;
#pragma unroll
      for (int t = 0; t < 8; ++t) p[t] = in_k ? xr[j][hn_perm8(t)] : (h16)0.0f;
      *reinterpret_cast<half8_t*>(xs + m * ldx + b * 8) = p;
    }
  }
  __syncthreads();
  // weights are issued only now: the waits for them then complete in issue
  // order, so a wave unpacks group i while groups i+1.. are still in flight
  __builtin_amdgcn_sched_barrier(0);

  // ---- 2. weights: each load instruction reads 8 rows x 128 B (full cache
  //         lines, non-temporal).  Load "lo" covers tile rows 0-7, load "hi"
  //         rows 8-15, both over the group pair (g, g+1).  Lane mapping:
  //           lo: row col%8,     chunk (col<8 ? q : 4+q)
  //           hi: row 8 + col%8, chunk (col>=8 ? q : 4+q)
  //         so lane l finds (row col, chunk q) of group g in lo if col<8 else hi
  //         (the "even" MFMA operand), and (row col^8, chunk q) of group g+1 in
  //         hi if col<8 else lo (the "odd" operand, whose MFMA columns are the
  //         weight rows XOR 8).  Buffer loads: rows past N and groups past the
  //         wave's range use a voffset past the descriptor's range and return
  //         0 without a memory access.
  constexpr uint32_t kOOB = 0x7ffffff0u;
  constexpr int PAIRS = BATCH / 2;
  u32x4 wlo[MATS][PAIRS], whi[MATS][PAIRS];
  h16 se[MATS][PAIRS], so[MATS][PAIRS];  // scales: even group (row col), odd (row col^8)
  const int rlo = n0 + (col & 7), rhi = n0 + 8 + (col & 7);
  const int clo = (col < 8) ? q : 4 + q, chi = (col >= 8) ? q : 4 + q;
  const int re = n0 + col, ro = n0 + (col ^ 8);
  __amdgpu_buffer_rsrc_t rq[MATS], rs[MATS];
  uint32_t vlo[MATS], vhi[MATS], vse[MATS], vso[MATS];
#pragma unroll
  for (int mt = 0; mt < MATS; ++mt) {
    rq[mt] = __builtin_amdgcn_make_buffer_rsrc((void*)mats[mt].q, (short)0,
                                               (int)((long)N * mats[mt].ld_q), 0x00020000);
    rs[mt] = __builtin_amdgcn_make_buffer_rsrc((void*)mats[mt].s, (short)0,
                                               (int)((long)N * mats[mt].ld_s * 2), 0x00020000);
    vlo[mt] = (tile_ok && rlo < N) ? (uint32_t)(rlo * mats[mt].ld_q + 16 * clo) : kOOB;
    vhi[mt] = (tile_ok && rhi < N) ? (uint32_t)(rhi * mats[mt].ld_q + 16 * chi) : kOOB;
    vse[mt] = (tile_ok && re < N) ? (uint32_t)(re * mats[mt].ld_s * 2) : kOOB;
    vso[mt] = (tile_ok && ro < N) ? (uint32_t)(ro * mats[mt].ld_s * 2) : kOOB;
  }
  constexpr int kAuxNT = 2;  // non-temporal: streamed once
#pragma unroll
  for (int pi = 0; pi < PAIRS; ++pi) {
    const int g = g0 + gl0 + 2 * pi;   // even group of the pair
    const bool pv = 2 * pi < gw;       // uniform
    const bool ov = 2 * pi + 1 < gw;   // odd group valid (uniform)
    // the range check covers voffset (+ immediate) only, never soffset: every
    // offset, and the out-of-range marker, goes in voffset
#pragma unroll
    for (int mt = 0; mt < MATS; ++mt) {
      const uint32_t gq = (uint32_t)(g * 64);
      wlo[mt][pi] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
          rq[mt], pv ? vlo[mt] + gq : kOOB, 0, kAuxNT));
      whi[mt][pi] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
          rq[mt], pv ? vhi[mt] + gq : kOOB, 0, kAuxNT));
      if (PREMUL) {
        const uint32_t ie = (uint32_t)((g * 128 + 32 * q) / group);
        const uint32_t io = (uint32_t)(((g + 1) * 128 + 32 * q) / group);
        se[mt][pi] = __builtin_bit_cast(h16, __builtin_amdgcn_raw_buffer_load_b16(
            rs[mt], pv ? vse[mt] + 2 * ie : kOOB, 0, 0));
        so[mt][pi] = __builtin_bit_cast(h16, __builtin_amdgcn_raw_buffer_load_b16(
            rs[mt], ov ? vso[mt] + 2 * io : kOOB, 0, 0));
      } else {
        se[mt][pi] = __builtin_bit_cast(h16, __builtin_amdgcn_raw_buffer_load_b16(
            rs[mt], pv ? vse[mt] + (uint32_t)(2 * ((g * 128) / group)) : kOOB, 0, 0));
        so[mt][pi] = __builtin_bit_cast(h16, __builtin_amdgcn_raw_buffer_load_b16(
            rs[mt], ov ? vso[mt] + (uint32_t)(2 * (((g + 1) * 128) / group)) : kOOB, 0, 0));
      }
    }
  }

  // ---- 4. unpack + MFMA.  acc_e: columns = tile rows; acc_o: columns = rows ^ 8.
  float4_t acc[NCH][MATS], acco[NCH][MATS];
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int mt = 0; mt < MATS; ++mt) {
      acc[c][mt] = float4_t{0.f, 0.f, 0.f, 0.f};
      acco[c][mt] = float4_t{0.f, 0.f, 0.f, 0.f};
    }
  const bool low_col = col < 8;
#pragma unroll
  for (int pi = 0; pi < PAIRS; ++pi) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      if (2 * pi + half < gw) {  // uniform
        const int gl = gl0 + 2 * pi + half;  // chunk-local group
#pragma unroll
        for (int mt = 0; mt < MATS; ++mt) {
          const h16 s16 = half ? so[mt][pi] : se[mt][pi];
          // even operand: lo for col<8, hi otherwise; odd operand: the reverse
          const bool take_lo = half ? !low_col : low_col;
          u32x4 w;
#pragma unroll
          for (int d = 0; d < 4; ++d) w[d] = take_lo ? wlo[mt][pi][d] : whi[mt][pi][d];
          half8_t b[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            b[t] = hn_unpack8_regs(w[t], ur);
            if (PREMUL) {
              const half8_t s8 = {s16, s16, s16, s16, s16, s16, s16, s16};
              b[t] = b[t] * s8;
            }
          }
#pragma unroll
          for (int c = 0; c < NCH; ++c) {
            // rows of A past the valid tokens only feed rows of C that are never
            // stored, so those lanes read a clamped valid row instead of branching
            const int tok = min(c * 16 + col, Mc - 1);
            const h16* arow = xs + tok * ldx + gl * 128 + 32 * q;
            float4_t& dst = half ? acco[c][mt] : acc[c][mt];
            float4_t cc = {0.f, 0.f, 0.f, 0.f};
            if (PREMUL) cc = dst;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const half8_t a = *reinterpret_cast<const half8_t*>(arow + 8 * t);
              cc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[t], cc, 0, 0, 0);
            }
            if (PREMUL) {
              dst = cc;
            } else {
              const float sf = (float)s16;
#pragma unroll
              for (int r = 0; r < 4; ++r) dst[r] = __builtin_fmaf(sf, cc[r], dst[r]);
            }
          }
        }
      }
    }
  }
  // fold the odd accumulator back: column c of acco belongs to row c ^ 8
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int mt = 0; mt < MATS; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[c][mt][r] += __shfl_xor(acco[c][mt][r], 8, 16);
  const int row = n0 + col;
  const bool row_ok = tile_ok && row < N;

  // ---- 5. reduce the KW waves of each tile through LDS (fixed order)
  if (A.kw > 1) {
    // the reduction area reuses the activation chunk once every wave is done with it
    __syncthreads();
    float4_t* red = reinterpret_cast<float4_t*>(smem);
    if (kwi > 0) {
#pragma unroll
      for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int mt = 0; mt < MATS; ++mt) red[((wave * NCH + c) * MATS + mt) * 64 + lane] =
            acc[c][mt];
    }
    __syncthreads();
    if (kwi > 0) return;
    for (int j = 1; j < A.kw; ++j) {
      const int w2 = wave + j;
#pragma unroll
      for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int mt = 0; mt < MATS; ++mt) {
          const float4_t v = red[((w2 * NCH + c) * MATS + mt) * 64 + lane];
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[c][mt][r] += v[r];
        }
    }
  }

  // ---- 6. output: D lane layout is row (n0 + col), tokens 16c + 4q + r
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
  // split over workgroups: write partials, the last split of this tile reduces
  // in split order.  Partials are relaxed agent-scope atomics, published
  // before the count; the last split acquires before reading them
  // (hn_arrive).
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
  hn_publish_partials();
  int n = 0;
  if (lane == 0) n = hn_arrive(ctr + tile, A.tag);
  n = __shfl(n, 0, 64);
  if (n != A.ks - 1) return;
  hn_acquire_agent();
  if (lane == 0) hn_counter_reset(ctr + tile);
  // this wave now owns the tile's 16 rows x Mc tokens: lanes walk (token, row);
  // all partial loads of an element are issued together (one round trip)
  for (int e = lane; e < Mc * kTileN; e += 64) {
    const int m = e / kTileN;
    const int rr = n0 + (e % kTileN);
    if (rr >= N) continue;
    float v[MATS];
#pragma unroll
    for (int mt = 0; mt < MATS; ++mt) v[mt] = 0.f;
    for (int kb = 0; kb < A.ks; kb += 8) {
      float pv[MATS][8];
#pragma unroll
      for (int mt = 0; mt < MATS; ++mt)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int kc = min(kb + j, A.ks - 1);
          pv[mt][j] = __hip_atomic_load(part + (long)(kc * MATS + mt) * plane + (long)m * N + rr,
                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
      for (int mt = 0; mt < MATS; ++mt)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (kb + j < A.ks) v[mt] += pv[mt][j];
    }
    h16 o;
    if (EPI == 1) o = (h16)(hn_silu((float)(h16)v[0]) * (float)(h16)v[MATS - 1]);
    else o = (h16)v[0];
    out[(long)m * A.ld_o + rr] = o;
  }
}

template <int MATS, int EPI, bool PREMUL, int NCH, int XR>
__global__ __launch_bounds__(kMaxWaves * 64) void skinny_kernel(SkinnyArgs A) {
  extern __shared__ __align__(16) unsigned char smem[];
  const W4Mat mats[2] = {A.w[0], A.w[1]};
  skinny_unit<MATS, EPI, PREMUL, NCH, XR>(A, A.x, A.M, mats, A.out, A.partial, A.counters,
                                          smem);
}

// Grouped launch over the experts of one MoE layer; tokens are permuted so
// expert e owns rows [offsets[e], offsets[e+1]).  blockIdx.z walks the
// active-expert list (device), so no host sync is needed.
template <int PHASE, bool PREMUL, int NCH, int XR>
__global__ __launch_bounds__(kMaxWaves * 64) void grouped_kernel(SkinnyArgs A) {
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
  unsigned long long* ctr = A.counters + (long)e * tmax;
  float* part = A.partial + (long)t0 * A.N;  // row offset inside each plane
  if (PHASE == 0) {
    const W4Mat mats[2] = {{ew.gate_q, ew.gate_s, H / 2, H / g}, {ew.up_q, ew.up_s, H / 2, H / g}};
    skinny_unit<2, 1, PREMUL, NCH, XR>(A, A.x + (long)t0 * A.ld_x, Me, mats,
                                       A.out + (long)t0 * A.ld_o, part, ctr, smem);
  } else {
    const W4Mat mats[2] = {{ew.down_q, ew.down_s, I / 2, I / g},
                           {ew.down_q, ew.down_s, I / 2, I / g}};
    skinny_unit<1, 0, PREMUL, NCH, XR>(A, A.x + (long)t0 * A.ld_x, Me, mats,
                                       A.out + (long)t0 * A.ld_o, part, ctr, smem);
  }
}

// ROUND_SILU: the SiLU is rounded to fp16 before the product (two fp16
// operations, as F.silu(g) * u on fp16 tensors), else one rounding.
template <bool ROUND_SILU>
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
  const float sv = ROUND_SILU ? (float)(h16)hn_silu(gv) : hn_silu(gv);
  o[(long)m * ld_o + n] = (h16)(sv * uv);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Launch plan.  A tile's whole K is reduced inside one workgroup (ks = 1)
// whenever its activation chunk fits the LDS budget; otherwise K is chunked
// over workgroups and reduced through the partials.
struct Plan {
  int ks, gpc, gpw, kw, tg, ldx, nch, xr;
  size_t lds;
};

Plan make_plan(int rows, int K, int mats) {
  Plan p;
  const int G = (K + 127) / 128;
  const int gpw_max = kLoadsPerLane / mats;
  p.nch = rows <= 16 ? 1 : rows <= 32 ? 2 : 4;
  auto fits = [&](int gpc) {
    const int kw = (gpc + gpw_max - 1) / gpw_max;
    if (kw > kMaxWaves) return false;
    const int tg = kw >= 4 ? 1 : 4 / kw;
    const size_t xb = (size_t)rows * (((gpc + 1) & ~1) * 128 + 8) * 2;
    const size_t rb = (size_t)tg * kw * p.nch * mats * 1024;
    const int xr_need = (rows * ((gpc + 1) & ~1) * 16 + tg * kw * 64 - 1) / (tg * kw * 64);
    return (xb > rb ? xb : rb) <= (size_t)kLdsBudget && xr_need <= 8;
  };
  int gpc = G;
  if (!fits(gpc)) {
    // largest chunk that fits, then balanced over the splits
    gpc = 1;
    while (gpc < G && fits(gpc + 1)) ++gpc;
    const int ks = (G + gpc - 1) / gpc;
    gpc = (G + ks - 1) / ks;
  }
  p.gpc = gpc;
  p.ks = (G + gpc - 1) / gpc;
  p.kw = (gpc + gpw_max - 1) / gpw_max;
  p.gpw = (gpc + p.kw - 1) / p.kw;
  p.gpw += p.gpw & 1;  // groups are loaded in pairs: waves start on even groups
  p.tg = p.kw >= 4 ? 1 : 4 / p.kw;
  p.ldx = ((gpc + 1) & ~1) * 128 + 8;
  const int nthr = p.tg * p.kw * 64;
  const int need = (rows * ((gpc + 1) & ~1) * 16 + nthr - 1) / nthr;
  p.xr = need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : 8;
  const size_t xb = (size_t)rows * p.ldx * 2;
  const size_t rb = p.kw > 1 ? (size_t)p.tg * p.kw * p.nch * mats * 1024 : 0;
  p.lds = xb > rb ? xb : rb;
  return p;
}

#define HN_SKINNY_VARIANTS(KERNEL, ...)                                                    \
  do {                                                                                     \
    if (p.nch == 1 && p.xr == 1)                                                           \
      hipLaunchKernelGGL((KERNEL<__VA_ARGS__, 1, 1>), grid, block, p.lds, s, A);           \
    else if (p.nch == 1 && p.xr == 2)                                                      \
      hipLaunchKernelGGL((KERNEL<__VA_ARGS__, 1, 2>), grid, block, p.lds, s, A);           \
    else if (p.nch == 1 && p.xr == 4)                                                      \
      hipLaunchKernelGGL((KERNEL<__VA_ARGS__, 1, 4>), grid, block, p.lds, s, A);           \
    else if (p.nch == 1)                                                                   \
      hipLaunchKernelGGL((KERNEL<__VA_ARGS__, 1, 8>), grid, block, p.lds, s, A);           \
    else if (p.nch == 2)                                                                   \
      hipLaunchKernelGGL((KERNEL<__VA_ARGS__, 2, 8>), grid, block, p.lds, s, A);           \
    else                                                                                   \
      hipLaunchKernelGGL((KERNEL<__VA_ARGS__, 4, 8>), grid, block, p.lds, s, A);           \
  } while (0)

void apply_plan(SkinnyArgs& A, const Plan& p) {
  A.m_lo = 0x000F000Fu;
  A.m_hi = 0x00F000F0u;
  A.magic = 0x64006400u;
  A.ks = p.ks;
  A.gpc = p.gpc;
  A.gpw = p.gpw;
  A.kw = p.kw;
  A.tg = p.tg;
  A.ldx = p.ldx;
}

template <int MATS, int EPI, bool PREMUL>
int launch_single(SkinnyArgs& A, const Plan& p, hipStream_t s) {
  dim3 grid(hn_cdiv(hn_cdiv(A.N, kTileN), p.tg), p.ks, 1), block(p.tg * p.kw * 64);
  HN_SKINNY_VARIANTS(skinny_kernel, MATS, EPI, PREMUL);
  return 0;
}

template <int PHASE, bool PREMUL>
void launch_grouped(SkinnyArgs& A, const Plan& p, int E_max, hipStream_t s) {
  dim3 grid(hn_cdiv(hn_cdiv(A.N, kTileN), p.tg), p.ks, E_max), block(p.tg * p.kw * 64);
  HN_SKINNY_VARIANTS(grouped_kernel, PHASE, PREMUL);
}

constexpr int kMaxRows = 64;  // tokens per weight matrix handled per launch

// Workspace layout, the same for every call: [counters: a fixed 2 MiB region
// at the start][partials].  One buffer serves calls of every kind and size
// in turn; with the counter region fixed, no call's partials ever land on
// another call's counters (64-bit tagged words, hn_arrive: zero when the
// workspace is new; a launch leaves its counters at zero, and a counter left
// by a launch stopped part-way is reclaimed by the next launch's tag).
constexpr size_t kCtrRegion = 2u << 20;
constexpr long kMaxCounters = (long)(kCtrRegion / 8);
size_t ctr_bytes(long /*counters*/) { return kCtrRegion; }

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
  size_t m = a > b ? a : b;
  if (kind == 3) {  // hn_moe_experts_decode: fp32 K-slice partials of the down projection
    const size_t c = (size_t)kHnDownSplit * prow * H * 4;
    m = m > c ? m : c;
  }
  return (long)(ctr_bytes(ctr) + m);
}

// Persistent streaming kernels (hn_stream.hip): return HN_NOT_HANDLED when a
// shape is not theirs, 0 after a launch, a hipError_t if the launch failed.
extern "C" int hn_stream_linear_impl(int mats, const void* x, long ld_x, const void* q0,
                                     const void* s0, const void* q1, const void* s1, long ld_q,
                                     long ld_s, void* out, long ld_o, long M, long N, long K,
                                     long group, void* stream);
extern "C" int hn_stream_grouped_impl(int phase, const void* x, long ld_x, const void* table,
                                      const int* active, const int* n_active, const int* offsets,
                                      long E, long max_rows, long rows, long H, long I, long group,
                                      void* out, long ld_o, void* stream, int dry_run);
extern "C" int hn_stream_down_split_impl(const void* h, const void* table, const int* active,
                                         const int* n_active, const int* offsets, long E,
                                         long max_rows, long rows_cap, long H, long I,
                                         long group, float* part, void* stream, int dry_run);
extern "C" int hn_moe_unpermute(const void* y_perm, long ld_y, const int* inv, const int* idx,
                                const void* w, long T, long k, const void* shared, long ld_sh,
                                void* out, long ld_o, long H, void* stream);
// Unpermute (hn_route.hip) from the four fp32 slices of the split down projection.
extern "C" int hn_stream_route_gate_up_impl(const void* hx, long ld_hx, const void* gate,
                                            long ld_gate, const float* logits_in, long T, long E,
                                            long k, const void* table, long H, long I, long group,
                                            float eps, float scaling, float* logits_out,
                                            int* idx, void* w, int* offsets, int* perm,
                                            int* inv, int* active, int* n_active,
                                            long long* usage, void* h_ws, void* stream,
                                            int dry_run);
extern "C" int hn_stream_route_sel_gate_up_impl(const void* hx, long ld_hx,
                                                const float* logits_in, const float* bias, long T,
                                                long E, long k, int mode, float eps,
                                                float scaling, const void* table, long H, long I,
                                                long group, int* idx, void* w, int* offsets,
                                                int* perm, int* inv, int* active, int* n_active,
                                                long long* usage, void* h_ws, void* stream,
                                                int dry_run);
extern "C" int hn_moe_unpermute_split4_impl(const float* part, long ks_stride, const int* inv,
                                            const int* idx, const void* w, long T, long k,
                                            const void* shared, long ld_sh, void* out,
                                            long ld_o, long H, void* stream);

// Prefill GEMM kernels (hn_gemm.hip): same return convention.
extern "C" int hn_gemm_linear_impl(int mats, const void* x, long ld_x, const void* q0,
                                   const void* s0, const void* q1, const void* s1, long ld_q,
                                   long ld_s, void* out, long ld_o, long M, long N, long K,
                                   long group, void* work, long work_bytes, void* stream);
extern "C" int hn_gemm_grouped_impl(int phase, const void* x, long ld_x, const void* table,
                                    const int* active, const int* n_active, const int* offsets,
                                    long E, long rows, long H, long I, long group, void* out,
                                    long ld_o, void* work, long work_bytes, void* stream);
extern "C" long hn_gemm_workspace_bytes();

// Decode kernel family: 0 = automatic (streaming kernels where they apply),
// 1 = split-K kernels only.  Per calling thread (a switch in one thread never
// changes another thread's calls); for A/B measurement and tests.
static thread_local int g_decode_path = 0;
constexpr long kStreamMaxRows = 16;

// Whether the streaming kernels take a grouped decode launch.  They stage at
// most 8 tokens of an expert per pass over its weights, so an expert with more
// rows streams its weights once per 8; they are used up to 16 rows per expert,
// or up to 64 when the average over the experts is at most 8 (few rows per
// expert: GLM-4.5-Air's 128 experts x top-8; 64 tokens over 8 experts at top-1
// pass over each expert's weights about 1.4 times on average).
// The streaming kernels take a grouped launch when every expert's rows fit
// one pass (<= 16), or when the rows average at most 16 per expert (passes
// of 8 or 16 tokens; the decoder's 64-token batches at top-1 and top-2).
static bool stream_rows_ok(long max_rows, long rows, long E) {
  return max_rows <= kStreamMaxRows || (max_rows <= kMaxRows && rows <= 16 * E);
}

extern "C" int hn_set_decode_path(int path) {
  HN_ARG_CHECK(path == 0 || path == 1, "hn_set_decode_path: path must be 0 or 1 (got %d)", path);
  g_decode_path = path;
  return 0;
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
  // buffer descriptors span one matrix; the out-of-range offset marker
  // (0x7ffffff0) must lie past that extent
  HN_ARG_CHECK(N * w0.ld_q < 0x7ffffff0L && N * w0.ld_s * 2 < 0x7ffffff0L,
               "%s: one weight matrix must stay below 2 GiB - 16 B", who);
  if (M == 0 || N == 0) return 0;
  const bool premul = (group % 128) != 0;
  if (M > kMaxRows) {
    const int rc = hn_gemm_linear_impl(mats, x, ld_x, w0.q, w0.s, w1.q, w1.s, w0.ld_q, w0.ld_s,
                                       out, ld_o, M, N, K, group, ws, ws_size, s);
    if (rc != HN_NOT_HANDLED) return rc;
  }
  if (g_decode_path == 0 && !premul && M <= kStreamMaxRows) {
    const int rc = hn_stream_linear_impl(mats, x, ld_x, w0.q, w0.s, w1.q, w1.s, w0.ld_q, w0.ld_s,
                                         out, ld_o, M, N, K, group, s);
    if (rc != HN_NOT_HANDLED) return rc;
  }
  const int tiles = hn_cdiv(N, kTileN);
  for (long m0 = 0; m0 < M; m0 += kMaxRows) {
    const int rows = (int)((M - m0) > kMaxRows ? kMaxRows : (M - m0));
    const Plan p = make_plan(rows, (int)K, mats);
    HN_ARG_CHECK((n_counters < tiles ? tiles : n_counters) <= kMaxCounters,
                 "%s: N=%ld needs more split-K counters than the workspace holds", who, N);
    const size_t cb = ctr_bytes(n_counters < tiles ? tiles : n_counters);
    const size_t need = cb + part_bytes(p.ks, mats, rows, N);
    HN_ARG_CHECK(p.ks == 1 || (ws && (size_t)ws_size >= need),
                 "%s: workspace too small (%ld < %zu bytes)", who, ws_size, need);
    HN_ARG_CHECK(p.ks <= kHnMaxArrivals, "%s: K=%ld splits into too many chunks", who, K);
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
    apply_plan(A, p);
    A.counters = (unsigned long long*)ws;
    A.tag = hn_next_tag();
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
  hipLaunchKernelGGL(silu_mul_kernel<false>, dim3(hn_cdiv(M * N, 256)), dim3(256), 0,
                     (hipStream_t)stream, (const h16*)g, ld_g, (const h16*)u, ld_u, (h16*)out,
                     ld_o, (int)M, (int)N);
  HN_LAUNCH_CHECK("hn_silu_mul");
  return 0;
}

extern "C" int hn_silu_then_mul(const void* g, long ld_g, const void* u, long ld_u, void* out,
                                long ld_o, long M, long N, void* stream) {
  HN_ARG_CHECK(M >= 0 && N >= 0, "hn_silu_then_mul: negative dims");
  if (M == 0 || N == 0) return 0;
  hipLaunchKernelGGL(silu_mul_kernel<true>, dim3(hn_cdiv(M * N, 256)), dim3(256), 0,
                     (hipStream_t)stream, (const h16*)g, ld_g, (const h16*)u, ld_u, (h16*)out,
                     ld_o, (int)M, (int)N);
  HN_LAUNCH_CHECK("hn_silu_then_mul");
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
  HN_ARG_CHECK(H % 128 == 0 && I % 32 == 0, "%s: H=%ld must be a multiple of 128, I=%ld of 32",
               who, H, I);
  HN_ARG_CHECK(group >= 32 && group % 32 == 0 && H % group == 0 && I % group == 0,
               "%s: bad group=%ld", who, group);
  HN_ARG_CHECK(aligned16(x_perm) && aligned16(h_ws) && aligned16(y_perm), "%s: misaligned", who);
  HN_ARG_CHECK((I / 2) % 16 == 0, "%s: down rows (I/2=%ld bytes) must be 16-byte aligned", who,
               I / 2);
  HN_ARG_CHECK(I * (H / 2) < 0x7ffffff0L && I * (H / group) * 2 < 0x7ffffff0L,
               "%s: one weight matrix must stay below 2 GiB - 16 B", who);
  if (max_rows_per_expert == 0 || rows == 0) return 0;
  if (max_rows_per_expert > kMaxRows) {
    // prefill: the grouped MFMA GEMM (a workspace of hn_gemm_workspace_bytes
    // enables its stream-K split; without one whole tiles go round-robin)
    HN_ARG_CHECK(I % 128 == 0 && E <= 256,
                 "%s: more than %d rows per expert needs I %% 128 == 0 and E <= 256 "
                 "(I=%ld, E=%ld)", who, kMaxRows, I, E);
    hipStream_t s = (hipStream_t)stream;
    int rc = hn_gemm_grouped_impl(0, x_perm, H, table, active, n_active, offsets, E, rows, H, I,
                                  group, h_ws, I, work, work_bytes, s);
    if (rc == 0)
      rc = hn_gemm_grouped_impl(1, h_ws, I, table, active, n_active, offsets, E, rows, H, I,
                                group, y_perm, H, work, work_bytes, s);
    if (rc == HN_NOT_HANDLED) {
      hn_set_error("%s: shape not handled by the prefill GEMM (group=%ld)", who, group);
      return -22;
    }
    return rc;
  }
  const long need = hn_skinny_workspace_bytes(3, rows, H, I, E);
  HN_ARG_CHECK(work && work_bytes >= need, "%s: workspace too small (%ld < %ld)", who, work_bytes,
               need);
  hipStream_t s = (hipStream_t)stream;
  const bool premul = (group % 128) != 0;
  if (g_decode_path == 0 && !premul && stream_rows_ok(max_rows_per_expert, rows, E) &&
      hn_stream_grouped_impl(0, x_perm, H, table, active, n_active, offsets, E,
                             max_rows_per_expert, rows, H, I, group, h_ws, I, s, 1) == 0 &&
      hn_stream_grouped_impl(1, h_ws, I, table, active, n_active, offsets, E,
                             max_rows_per_expert, rows, H, I, group, y_perm, H, s, 1) == 0) {
    int rc = hn_stream_grouped_impl(0, x_perm, H, table, active, n_active, offsets, E,
                                    max_rows_per_expert, rows, H, I, group, h_ws, I, s, 0);
    if (rc) return rc;
    return hn_stream_grouped_impl(1, h_ws, I, table, active, n_active, offsets, E,
                                  max_rows_per_expert, rows, H, I, group, y_perm, H, s, 0);
  }
  const int rmax = (int)max_rows_per_expert;
  SkinnyArgs A = {};
  A.table = (const ExpertW4*)table;
  A.active = active;
  A.n_active = n_active;
  A.offsets = offsets;
  A.H = (int)H;
  A.I = (int)I;
  A.group = (int)group;
  A.counters = (unsigned long long*)work;
  A.tag = hn_next_tag();
  A.part_rows = rows;
  A.M = rmax;
  const long tmax = hn_cdiv(I, kTileN) > hn_cdiv(H, kTileN) ? hn_cdiv(I, kTileN)
                                                            : hn_cdiv(H, kTileN);
  HN_ARG_CHECK(E * tmax <= kMaxCounters, "%s: E=%ld x %ld tiles exceed the counter region", who,
               E, tmax);
  HN_ARG_CHECK(hn_cdiv(H, 128) <= kHnMaxArrivals && hn_cdiv(I, 128) <= kHnMaxArrivals,
               "%s: H=%ld or I=%ld splits into too many chunks", who, H, I);
  float* partial = (float*)((char*)work + ctr_bytes(E * tmax));
  {
    const Plan p = make_plan(rmax, (int)H, 2);
    A.x = (const h16*)x_perm; A.ld_x = H;
    A.out = (h16*)h_ws; A.ld_o = I;
    A.N = (int)I; A.K = (int)H;
    apply_plan(A, p);
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
    apply_plan(A, p);
    A.tag = hn_next_tag();
    A.partial = partial;
    A.phase = 1;
    if (premul) launch_grouped<1, true>(A, p, (int)E, s);
    else launch_grouped<1, false>(A, p, (int)E, s);
    HN_LAUNCH_CHECK("hn_grouped_expert_mlp_int4(down)");
  }
  return 0;
}

// One phase of the grouped SwiGLU at prefill sizes (the MFMA GEMM kernels):
// phase 0: h_ws[rows, I] = fp16(silu(x_perm Wg^T) * (x_perm Wu^T)) per expert;
// phase 1: y_perm[rows, H] = h_ws Wd^T per expert.  Same operands as
// hn_grouped_expert_mlp_int4; lets a caller time or schedule the phases apart.
extern "C" int hn_grouped_expert_phase_int4(int phase, const void* x_perm, const void* table,
                                            const int* active, const int* n_active,
                                            const int* offsets, long E, long rows, long H,
                                            long I, long group, void* h_ws, void* y_perm,
                                            void* work, long work_bytes, void* stream) {
  const char* who = "hn_grouped_expert_phase_int4";
  HN_ARG_CHECK(phase == 0 || phase == 1, "%s: phase must be 0 or 1", who);
  HN_ARG_CHECK(E > 0 && E <= 256 && rows >= 0, "%s: bad sizes (E=%ld, rows=%ld)", who, E, rows);
  HN_ARG_CHECK(H % 128 == 0 && I % 128 == 0, "%s: H=%ld and I=%ld must be multiples of 128",
               who, H, I);
  HN_ARG_CHECK(aligned16(x_perm) && aligned16(h_ws) && aligned16(y_perm), "%s: misaligned", who);
  if (rows == 0) return 0;
  const int rc = phase == 0
      ? hn_gemm_grouped_impl(0, x_perm, H, table, active, n_active, offsets, E, rows, H, I, group,
                             h_ws, I, work, work_bytes, stream)
      : hn_gemm_grouped_impl(1, h_ws, I, table, active, n_active, offsets, E, rows, H, I, group,
                             y_perm, H, work, work_bytes, stream);
  if (rc == HN_NOT_HANDLED) {
    hn_set_error("%s: shape not handled by the GEMM kernels (group=%ld)", who, group);
    return -22;
  }
  return rc;
}

// Whether hn_moe_experts_decode takes the streaming path with the K-split down
// projection for these sizes (the launches' own dry runs).
static bool experts_split_ok(long E, long max_rows, long rows, long H, long I, long group) {
  return rows > 0 && max_rows > 0 && stream_rows_ok(max_rows, rows, E) && g_decode_path == 0 &&
         group % 128 == 0 && H % 128 == 0 && I % 128 == 0 &&
         hn_stream_grouped_impl(0, nullptr, H, nullptr, nullptr, nullptr, nullptr, E, max_rows,
                                rows, H, I, group, nullptr, I, nullptr, 1) == 0 &&
         hn_stream_down_split_impl(nullptr, nullptr, nullptr, nullptr, nullptr, E, max_rows,
                                   rows, H, I, group, nullptr, nullptr, 1) == 0;
}

extern "C" int hn_moe_experts_decode_split_check(long E, long max_rows_per_expert, long rows,
                                                 long H, long I, long group) {
  return experts_split_ok(E, max_rows_per_expert, rows, H, I, group) ? 0 : 1;
}

// The experts half of a decode MoE layer: grouped SwiGLU over the routed rows
// and the ordered, weighted sum back per token.  Where the streaming kernels
// apply, the down projection runs in four K slices whose fp32 partials (in
// the workspace) the unpermute sums in slice order (out NULL: left there for
// the caller); otherwise this is hn_grouped_expert_mlp_int4 into y_ws
// followed by hn_moe_unpermute.
extern "C" int hn_moe_experts_decode(const void* x_perm, const void* table, const int* active,
                                     const int* n_active, const int* offsets, long E,
                                     long max_rows_per_expert, long rows, long H, long I,
                                     long group, void* h_ws, void* y_ws, const int* inv,
                                     const int* idx, const void* w, long T, long k,
                                     const void* shared, long ld_sh, void* out, long ld_o,
                                     void* work, long work_bytes, void* stream) {
  const char* who = "hn_moe_experts_decode";
  HN_ARG_CHECK(E > 0 && E <= 256 && max_rows_per_expert >= 0 && rows >= 0 && T >= 0 && k > 0,
               "%s: bad sizes", who);
  HN_ARG_CHECK(aligned16(out) && (!out || ld_o % 8 == 0) && H % 8 == 0,
               "%s: out rows must be 16-byte aligned", who);
  hipStream_t s = (hipStream_t)stream;
  if (!out && rows == 0) return 0;  // no rows: no partials to leave
  const bool split = experts_split_ok(E, max_rows_per_expert, rows, H, I, group) &&
                     aligned16(x_perm) && aligned16(h_ws);
  HN_ARG_CHECK(out || (split && !shared),
               "%s: out NULL (partials left for the caller) needs the streaming path with the "
               "K-split down projection (hn_moe_experts_decode_split_check) and no shared "
               "expert", who);
  if (split) {
    const long tmax = hn_cdiv(I, kTileN) > hn_cdiv(H, kTileN) ? hn_cdiv(I, kTileN)
                                                              : hn_cdiv(H, kTileN);
    const long need = hn_skinny_workspace_bytes(3, rows, H, I, E);
    HN_ARG_CHECK(work && work_bytes >= need, "%s: workspace too small (%ld < %ld)", who,
                 work_bytes, need);
    float* part = (float*)((char*)work + ctr_bytes(E * tmax));
    int rc = hn_stream_grouped_impl(0, x_perm, H, table, active, n_active, offsets, E,
                                    max_rows_per_expert, rows, H, I, group, h_ws, I, s, 0);
    if (rc == 0)
      rc = hn_stream_down_split_impl(h_ws, table, active, n_active, offsets, E,
                                     max_rows_per_expert, rows, H, I, group, part, s, 0);
    if (rc == 0 && out)
      rc = hn_moe_unpermute_split4_impl(part, rows * H, inv, idx, w, T, k, shared, ld_sh, out,
                                        ld_o, H, stream);
    return rc;
  }
  int rc = hn_grouped_expert_mlp_int4(x_perm, table, active, n_active, offsets, E,
                                      max_rows_per_expert, rows, H, I, group, h_ws, y_ws, work,
                                      work_bytes, stream);
  if (rc == 0)
    rc = hn_moe_unpermute(y_ws, H, inv, idx, w, T, k, shared, ld_sh, out, ld_o, H, stream);
  return rc;
}

// The first launch of hn_moe_decode_layer on its own: routing computed in the
// grouped gate/up streaming kernel, h_ws = SwiGLU gate/up of the routed rows.
extern "C" int hn_moe_route_gate_up(const void* h, long ld_h, const void* gate_w, long ld_w,
                                    const float* logits_in, long T, long E, long k,
                                    const void* table, long H, long I, long group, float eps,
                                    float scaling, void* logits_out, int* idx, void* w,
                                    int* offsets, int* perm, int* inv, int* active,
                                    int* n_active, long long* usage, void* h_ws, void* stream) {
  const char* who = "hn_moe_route_gate_up";
  HN_ARG_CHECK(aligned16(h) && (logits_in || aligned16(gate_w)) && aligned16(h_ws),
               "%s: h, gate and h_ws rows must be 16-byte aligned", who);
  HN_ARG_CHECK(g_decode_path == 0, "%s: needs the streaming kernels (decode path 0)", who);
  const int rc = hn_stream_route_gate_up_impl(h, ld_h, gate_w, ld_w, logits_in, T, E, k, table,
                                              H, I, group, eps, scaling, (float*)logits_out, idx,
                                              w, offsets, perm, inv, active, n_active, usage,
                                              h_ws, (hipStream_t)stream, 0);
  HN_ARG_CHECK(rc != HN_NOT_HANDLED, "%s: shape not covered (E <= 8, k 1 or 2, T k <= 64, T <= "
               "16 without logits_in, H %% 512 == 0, group 128; T=%ld E=%ld k=%ld H=%ld "
               "group=%ld)", who, T, E, k, H, group);
  return rc;
}

// 0 when hn_moe_decode_layer covers the shape (decode path 0 included),
// otherwise HN_NOT_HANDLED; sets no error.  has_logits: the caller passes
// logits_in.
extern "C" int hn_moe_decode_layer_check(long T, long E, long k, long H, long I, long group,
                                         int has_logits) {
  if (g_decode_path != 0) return HN_NOT_HANDLED;
  // dry runs: shapes only (no pointer is read; a non-null logits_in stands
  // for the caller's)
  static const float dummy = 0.f;
  const int a = hn_stream_route_gate_up_impl(nullptr, H, nullptr, H, has_logits ? &dummy : nullptr,
                                             T, E, k, nullptr, H, I, group, 0.f, 1.f, nullptr,
                                             nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                             nullptr, nullptr, nullptr, nullptr, 1);
  const int b = hn_stream_down_split_impl(nullptr, nullptr, nullptr, nullptr, nullptr, E, T,
                                          T * k, H, I, group, nullptr, nullptr, 1);
  return a == 0 && b == 0 ? 0 : HN_NOT_HANDLED;
}

// One Mixtral MoE layer at decode in three launches: the routing (logits
// unless given, softmax top-k, permutation) computed inside the gate/up
// streaming kernel, the down projection in four K slices, the ordered
// weighted unpermute.  Same results as hn_moe_route followed by
// hn_moe_experts_decode.
// Byte offset in hn_moe_decode_layer's workspace of the down projection's
// kHnDownSplit fp32 K-slice partials [kHnDownSplit][T k][H] (slice stride T k H
// floats).
extern "C" long hn_moe_decode_layer_partials(long T, long E, long k, long H, long I) {
  (void)T;
  (void)k;
  const long tmax = hn_cdiv(I, kTileN) > hn_cdiv(H, kTileN) ? hn_cdiv(I, kTileN)
                                                            : hn_cdiv(H, kTileN);
  return (long)ctr_bytes(E * tmax);
}

extern "C" int hn_moe_decode_layer(const void* h, long ld_h, const void* gate_w, long ld_w,
                                   const float* logits_in, long T, long E, long k,
                                   const void* table, long H, long I, long group, float eps,
                                   float scaling, void* logits_out, int* idx, void* w,
                                   int* offsets, int* perm, int* inv, int* active, int* n_active,
                                   long long* usage, void* h_ws, void* out, long ld_o, void* work,
                                   long work_bytes, void* stream) {
  const char* who = "hn_moe_decode_layer";
  HN_ARG_CHECK(aligned16(h) && (logits_in || aligned16(gate_w)) && aligned16(h_ws) &&
                   aligned16(out) && (!out || ld_o % 8 == 0),
               "%s: h, gate, h_ws and out rows must be 16-byte aligned", who);
  HN_ARG_CHECK(g_decode_path == 0, "%s: needs the streaming kernels (decode path 0)", who);
  hipStream_t s = (hipStream_t)stream;
  const long rows = T * k;
  const bool ok =
      hn_stream_route_gate_up_impl(h, ld_h, gate_w, ld_w, logits_in, T, E, k, table, H, I, group,
                                   eps, scaling, (float*)logits_out, idx, w, offsets, perm, inv,
                                   active, n_active, usage, h_ws, s, 1) == 0 &&
      hn_stream_down_split_impl(h_ws, table, active, n_active, offsets, E, T, rows, H, I, group,
                                nullptr, s, 1) == 0;
  HN_ARG_CHECK(ok, "%s: shape not covered (E <= 8, k 1 or 2, T k <= 64, T <= 16 without "
               "logits_in, H %% 512 == 0, I %% 512 == 0, group 128; T=%ld E=%ld k=%ld H=%ld "
               "I=%ld group=%ld)", who, T, E, k, H, I, group);
  const long tmax = hn_cdiv(I, kTileN) > hn_cdiv(H, kTileN) ? hn_cdiv(I, kTileN)
                                                            : hn_cdiv(H, kTileN);
  const long need = hn_skinny_workspace_bytes(3, rows, H, I, E);
  HN_ARG_CHECK(work && work_bytes >= need, "%s: workspace too small (%ld < %ld)", who,
               work_bytes, need);
  float* part = (float*)((char*)work + ctr_bytes(E * tmax));
  int rc = hn_stream_route_gate_up_impl(h, ld_h, gate_w, ld_w, logits_in, T, E, k, table, H, I,
                                        group, eps, scaling, (float*)logits_out, idx, w, offsets,
                                        perm, inv, active, n_active, usage, h_ws, s, 0);
  if (rc == 0)
    rc = hn_stream_down_split_impl(h_ws, table, active, n_active, offsets, E, T, rows, H, I,
                                   group, part, s, 0);
  // out NULL: the caller does the unpermute from the partials
  // (hn_moe_decode_layer_partials; e.g. hn_unpermute_add_rmsnorm)
  if (rc == 0 && out)
    rc = hn_moe_unpermute_split4_impl(part, rows * H, inv, idx, w, T, k, nullptr, H, out, ld_o,
                                      H, stream);
  if (rc == HN_NOT_HANDLED) {
    // the dry run passed but a launch declined (e.g. the device refused the
    // 160 KiB dynamic-LDS limit a plan needs): an argument-style error the
    // caller can fall back from
    hn_set_error("%s: the device cannot run this shape's plan (dynamic LDS limit); "
                 "T=%ld E=%ld k=%ld", who, T, E, k);
    return -22;
  }
  return rc;
}

// One phase of hn_moe_experts_decode's streaming path on its own: phase 0
// h_ws = fp16(silu(fp16(x Wg^T)) * fp16(x Wu^T)) per expert; phase 1 the
// down projection in four K slices into fp32 partials part[4][rows][H]
// (work after its counter region, as hn_moe_experts_decode keeps them).
// Returns an error when the streaming kernels do not cover the shape.
extern "C" int hn_grouped_decode_phase_int4(int phase, const void* x, const void* table,
                                            const int* active, const int* n_active,
                                            const int* offsets, long E,
                                            long max_rows_per_expert, long rows, long H, long I,
                                            long group, void* h_ws, void* work,
                                            long work_bytes, void* stream) {
  const char* who = "hn_grouped_decode_phase_int4";
  HN_ARG_CHECK(phase == 0 || phase == 1, "%s: phase must be 0 or 1", who);
  HN_ARG_CHECK(E > 0 && E <= 256 && rows >= 0 && max_rows_per_expert >= 0,
               "%s: bad sizes (E=%ld, rows=%ld)", who, E, rows);
  HN_ARG_CHECK(H % 128 == 0 && I % 128 == 0 && aligned16(x) && aligned16(h_ws),
               "%s: H, I multiples of 128 and 16-byte aligned buffers", who);
  HN_ARG_CHECK(stream_rows_ok(max_rows_per_expert, rows, E) && group == 128,
               "%s: the streaming kernels take <= %ld rows per expert (<= %ld when rows <= "
               "8 E) and group 128", who, kStreamMaxRows, kMaxRows);
  if (rows == 0 || max_rows_per_expert == 0) return 0;
  hipStream_t s = (hipStream_t)stream;
  int rc;
  if (phase == 0) {
    rc = hn_stream_grouped_impl(0, x, H, table, active, n_active, offsets, E,
                                max_rows_per_expert, rows, H, I, group, h_ws, I, s, 0);
  } else {
    const long tmax = hn_cdiv(I, kTileN) > hn_cdiv(H, kTileN) ? hn_cdiv(I, kTileN)
                                                              : hn_cdiv(H, kTileN);
    const long need = hn_skinny_workspace_bytes(3, rows, H, I, E);
    HN_ARG_CHECK(work && work_bytes >= need, "%s: workspace too small (%ld < %ld)", who,
                 work_bytes, need);
    rc = hn_stream_down_split_impl(x, table, active, n_active, offsets, E, max_rows_per_expert,
                                   rows, H, I, group, (float*)((char*)work + ctr_bytes(E * tmax)),
                                   s, 0);
  }
  if (rc == HN_NOT_HANDLED) {
    hn_set_error("%s: shape not handled by the streaming kernels", who);
    return -22;
  }
  return rc;
}

// 0 when hn_moe_route_experts_decode covers the shape, else HN_NOT_HANDLED
// (sets no error).
extern "C" int hn_moe_route_experts_decode_check(long T, long E, long k, int mode, long H,
                                                 long I, long group) {
  if (g_decode_path != 0) return HN_NOT_HANDLED;
  static const float dummy = 0.f;
  if (hn_stream_route_sel_gate_up_impl(nullptr, H, &dummy, nullptr, T, E, k, mode, 0.f, 1.f,
                                       nullptr, H, I, group, nullptr, nullptr, nullptr, nullptr,
                                       nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                       1) != 0)
    return HN_NOT_HANDLED;
  const long rows = T * k;
  const bool split = hn_stream_down_split_impl(nullptr, nullptr, nullptr, nullptr, nullptr, E, T,
                                               rows, H, I, group, nullptr, nullptr, 1) == 0;
  if (!split && hn_stream_grouped_impl(1, nullptr, I, nullptr, nullptr, nullptr, nullptr, E, T,
                                       rows, H, I, group, nullptr, H, nullptr, 1) != 0)
    return HN_NOT_HANDLED;
  return 0;
}

// A decode MoE layer from given router logits, in three launches: the
// routing (top-k in any mode, optional selection bias, E <= 256) computed in
// the grouped gate/up streaming kernel's prologue with the rows staged from
// h directly; the down projection (four K slices when I splits, else whole
// into y_ws); the ordered weighted unpermute with the optional fp16 shared
// addend.  shared_ready (a hipEvent_t, may be null): the stream waits for it
// right before the unpermute, so a shared expert computed on another stream
// overlaps the expert kernels.
extern "C" int hn_moe_route_experts_decode(const float* logits, const void* bias, long T, long E,
                                           long k, int mode, float eps, float scaling,
                                           const void* h, long ld_h, const void* table, long H,
                                           long I, long group, int* idx, void* w, int* offsets,
                                           int* perm, int* inv, int* active, int* n_active,
                                           long long* usage, void* h_ws, void* y_ws,
                                           void* shared_ready, const void* shared, long ld_sh,
                                           void* out, long ld_o, void* work, long work_bytes,
                                           void* stream) {
  const char* who = "hn_moe_route_experts_decode";
  HN_ARG_CHECK(logits && aligned16(logits) && aligned16(h) && aligned16(h_ws) && aligned16(y_ws) &&
                   aligned16(out) &&
                   ld_o % 8 == 0 && (!shared || (aligned16(shared) && ld_sh % 8 == 0)),
               "%s: logits needed; logits, h, h_ws, y_ws, shared and out rows 16-byte aligned",
               who);
  HN_ARG_CHECK(hn_moe_route_experts_decode_check(T, E, k, mode, H, I, group) == 0,
               "%s: shape not covered (decode path 0, E <= 256, k <= 16, T k <= the gate/up "
               "launch's threads, mode 0-2, H %% 512 == 0, group 128; T=%ld E=%ld k=%ld "
               "mode=%d H=%ld I=%ld group=%ld)", who, T, E, k, mode, H, I, group);
  hipStream_t s = (hipStream_t)stream;
  const long rows = T * k;
  const long tmax = hn_cdiv(I, kTileN) > hn_cdiv(H, kTileN) ? hn_cdiv(I, kTileN)
                                                            : hn_cdiv(H, kTileN);
  const long need = hn_skinny_workspace_bytes(3, rows, H, I, E);
  HN_ARG_CHECK(work && work_bytes >= need, "%s: workspace too small (%ld < %ld)", who,
               work_bytes, need);
  float* part = (float*)((char*)work + ctr_bytes(E * tmax));
  int rc = hn_stream_route_sel_gate_up_impl(h, ld_h, logits, (const float*)bias, T, E, k, mode,
                                            eps, scaling, table, H, I, group, idx, w, offsets,
                                            perm, inv, active, n_active, usage, h_ws, s, 0);
  const bool split = hn_stream_down_split_impl(nullptr, nullptr, nullptr, nullptr, nullptr, E, T,
                                               rows, H, I, group, nullptr, nullptr, 1) == 0;
  if (rc == 0)
    rc = split ? hn_stream_down_split_impl(h_ws, table, active, n_active, offsets, E, T, rows, H,
                                           I, group, part, s, 0)
               : hn_stream_grouped_impl(1, h_ws, I, table, active, n_active, offsets, E, T,
                                        rows, H, I, group, y_ws, H, s, 0);
  if (rc == 0 && shared_ready) {
    const hipError_t e = hipStreamWaitEvent(s, (hipEvent_t)shared_ready, 0);
    if (e != hipSuccess) {
      hn_set_error("%s: waiting for shared_ready failed: %s", who, hipGetErrorString(e));
      return (int)e;
    }
  }
  if (rc == 0)
    rc = split ? hn_moe_unpermute_split4_impl(part, rows * H, inv, idx, w, T, k, shared, ld_sh,
                                              out, ld_o, H, stream)
               : hn_moe_unpermute(y_ws, H, inv, idx, w, T, k, shared, ld_sh, out, ld_o, H,
                                  stream);
  if (rc == HN_NOT_HANDLED) {
    hn_set_error("%s: the device cannot run this shape's plan (dynamic LDS limit); T=%ld E=%ld "
                 "k=%ld", who, T, E, k);
    return -22;
  }
  return rc;
}
