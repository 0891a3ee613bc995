// W4A16 GEMM for prefill (many tokens per weight matrix), gfx950.
//
//   out[m, n] = sum_k x[m, k] * W[n, k],   W[n, k] = fp16((nibble - 8) * scale[n, k / group])
//
// Replaces, above 64 tokens per weight matrix, the Triton int4_matmul_kernel
// (kernels/int4_gemm.py:25-121, kernels/int4_expert_mlp.py:15-96) with its
// SwiGLU epilogue (kernels/int4_gemm.py:175-193), and in the grouped form the
// per-expert loop of MixtralMoELayer.forward / GLM4MoELayer.forward
// (model/mixtral.py:327-368, model/glm4.py:421-466) at prefill sizes.
//
// This is the one place the path is a real dense contraction, so it is built
// around the MFMA pipe (v_mfma_f32_16x16x32_f16):
//  * Tile = 128 tokens x (4 waves x NB x 16) weight rows of each matrix; a wave
//    owns NB 16-row blocks of every matrix (gate and up together for the SwiGLU
//    form, so its epilogue has both values of an output in the same lane) for
//    all 128 tokens.  Waves split N, never M, so each weight is dequantised by
//    exactly one wave of the workgroup and never goes through LDS.
//  * Weights: per 128-k group each lane issues one 16-byte buffer load per
//    16-row block: row (block + lane % 16), bytes [16 * (lane / 16), +16) of the
//    row's 64-byte group (one load instruction = 16 rows x 64 B).  Loads for
//    group g + 1 are in flight while group g computes.  In registers, each
//    packed dword becomes eight fp16 weights in k order: a byte broadcast
//    (v_perm_b32) and one v_and_or_b32 put two nibbles in the mantissas of
//    1024 (0x6400), one v_pk_fma_f16 gives the exact (n - 8) pair, and
//    v_pk_mul_f16 by the fp16 scale rounds the exact product once: the
//    reference's dequantised weight bit for bit.
//  * Activations: the 128 x 128 group slice goes HBM -> LDS directly
//    (global_load_lds_dwordx4, no registers), double-buffered with one barrier
//    per group.  Its 16-byte chunks are XOR-swizzled by row (chunk c of row r
//    sits at r * 16 + (c ^ (r & 15))), so the 16-byte A-fragment reads of the
//    16 rows of an MFMA block hit distinct banks.
//  * Row blocks of 16 tokens past the tile's valid rows skip their MFMAs, so a
//    ragged last tile of an expert costs what its rows need.
//  * Persistent grid (2 workgroups per CU).  Tiles are numbered per problem in
//    super-blocks of up to 8 M-tiles x n-tiles (n-tile slowest inside a
//    super-block), and workgroups on one XCD take consecutive tile numbers, so
//    the tiles running together on an XCD share activation and weight slices in
//    its L2.
#include "hn_common.h"

namespace {

constexpr int kBM = 128;          // tokens per tile
constexpr int kWaves = 4;         // waves per workgroup (split N)
constexpr int kMaxProb = 256;     // experts per grouped launch
constexpr int kSuperM = 8;        // M-tiles per super-block
constexpr uint32_t kOOB = 0x7ffffff0u;

struct GExpert {
  const uint8_t* gate_q; const h16* gate_s;
  const uint8_t* up_q;   const h16* up_s;
  const uint8_t* down_q; const h16* down_s;
};

struct GemmArgs {
  // single problem (grouped launches resolve these per expert)
  const h16* x; long ld_x; int M;
  const uint8_t* q[2];
  const h16* s[2];
  h16* out; long ld_o;
  int phase;        // grouped: 0 gate/up + SiLU (N = I, K = H); 1 down (N = H, K = I)
  int N, K, group;
  int ld_q;         // packed row stride (bytes)
  int ld_s;         // scale row stride (elements)
  uint32_t m_pair, magic;
};

template <int MATS, int NB>
struct BBuf {
  u32x4 w[MATS][NB];
  uint32_t s[MATS][NB];  // fp16 scale bits, zero-extended
};

struct Prob {
  const h16* x;
  h16* out;
  int rows;
  const uint8_t* q[2];
  const h16* s[2];
};

template <bool GROUPED>
__device__ __forceinline__ Prob resolve(const GemmArgs& A, const GExpert* __restrict__ table,
                                        const int* __restrict__ active,
                                        const int* __restrict__ offsets, int p) {
  Prob r;
  if (!GROUPED) {
    r.x = A.x; r.out = A.out; r.rows = A.M;
    r.q[0] = A.q[0]; r.s[0] = A.s[0];
    r.q[1] = A.q[1]; r.s[1] = A.s[1];
  } else {
    const int e = active[p];
    const int t0 = offsets[e];
    r.rows = offsets[e + 1] - t0;
    const GExpert ew = table[e];
    if (A.phase == 0) {
      r.q[0] = ew.gate_q; r.s[0] = ew.gate_s;
      r.q[1] = ew.up_q;   r.s[1] = ew.up_s;
    } else {
      r.q[0] = ew.down_q; r.s[0] = ew.down_s;
      r.q[1] = ew.down_q; r.s[1] = ew.down_s;
    }
    r.x = A.x + (long)t0 * A.ld_x;
    r.out = A.out + (long)t0 * A.ld_o;
  }
  return r;
}

typedef __attribute__((address_space(3))) void lds_void_t;

// Per-tile load state: buffer descriptors and the loop-invariant per-lane
// byte offsets; the group offset goes in soffset.  Rows past N get an offset
// past the descriptor's range (the load returns 0 and touches no memory): the
// range check covers voffset (+ immediate) only, so the per-row part must be
// in voffset.
// (Descriptors are rebuilt from these at each use: a few scalar moves that
// the compiler hoists; buffer-descriptor types cannot be struct members in
// the host pass.)
template <int MATS, int NB>
struct TileLoads {
  const void* px; int nx;             // activation rows of the tile, bytes
  const void* pq[MATS];               // packed weights
  const void* ps[MATS];               // scales
  int nq, ns;                         // bytes of one packed / scale matrix
  uint32_t va[8];                     // activation chunk offsets (8 DMA loads)
  uint32_t vq[NB], vs[NB];            // weight / scale offsets per 16-row block
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, bytes, 0x00020000);
}

// Activation slice of group g -> LDS: 128 rows x 128 k = 2048 16-byte chunks.
// Wave w issues 8 direct loads of 64 consecutive LDS chunks each; LDS chunk
// L = (row r, slot c') receives global chunk c' ^ (r & 15) of row r.  Rows
// past the valid ones repeat the last valid row (their results are never
// stored).
__device__ __forceinline__ uint32_t a_offset(int j, int wave, int lane, int rows, long ld_x) {
  const int L = (wave * 8 + j) * 64 + lane;
  const int r = L >> 4;
  const int c = (L & 15) ^ (r & 15);
  return (uint32_t)((min(r, rows - 1) * (int)ld_x + 8 * c) * 2);
}

// (Not a template: the host pass rejects this builtin in a dependent call.)
__device__ __forceinline__ void dma_a(const void* px, int nx, const uint32_t (&va)[8], int g,
                                      h16* xs, int wave) {
  const __amdgpu_buffer_rsrc_t r = rsrc(px, nx);
#pragma unroll
  for (int j = 0; j < 8; ++j)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)(xs + (wave * 8 + j) * 512), 16,
                                             va[j], 256 * g, 0, 0);
}

template <int MATS, int NB>
__device__ __forceinline__ void issue_b(BBuf<MATS, NB>& b, const TileLoads<MATS, NB>& tl, int g,
                                        int group) {
  const int soff_s = 2 * ((128 * g) / group);
#pragma unroll
  for (int bk = 0; bk < NB; ++bk)
#pragma unroll
    for (int mt = 0; mt < MATS; ++mt) {
      b.w[mt][bk] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  rsrc(tl.pq[mt], tl.nq), tl.vq[bk], 64 * g, 0));
      b.s[mt][bk] = (uint32_t)__builtin_bit_cast(unsigned short, __builtin_amdgcn_raw_buffer_load_b16(
                                                rsrc(tl.ps[mt], tl.ns), tl.vs[bk], soff_s, 0));
    }
}

// Unpack constants (gfx9 VOP3 takes no literals): mask in an SGPR, the rest
// in VGPRs.
struct DeqRegs {
  uint32_t m_pair;  // SGPR 0x00F0000F: low nibble of byte 0, high nibble of byte 2
  uint32_t magic;   // 0x64006400
  uint32_t mul;     // half2(1, 1/16)
  uint32_t add;     // half2(-1032, -72)
};

// Eight fp16 (n_k - 8) * s, k = 0..7 in order, from one packed dword.
__device__ __forceinline__ half8_t deq8(uint32_t w, const DeqRegs& c, half2_t s2) {
  u32x4 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t t = __builtin_amdgcn_perm(w, w, 0x01010101u * j);  // byte j, 4 times
    const half2_t v = hn_bits_h2(hn_and_or(t, c.m_pair, c.magic));    // (1024+n, 1024+16n')
    const half2_t d = __builtin_elementwise_fma(v, hn_bits_h2(c.mul), hn_bits_h2(c.add));
    r[j] = __builtin_bit_cast(uint32_t, d * s2);
  }
  return __builtin_bit_cast(half8_t, r);
}

// One group (4 MFMA k-steps of 32) for this wave.  FULL: all 8 row blocks
// valid (no per-block branches, so unpack and MFMA interleave freely).
template <int MATS, int NB, bool FULL>
__device__ __forceinline__ void compute(const BBuf<MATS, NB>& b, const h16* xs, int nrb, int col,
                                        int q, const DeqRegs& dr, float4_t (&acc)[8][MATS][NB]) {
  half2_t s2[MATS][NB];
#pragma unroll
  for (int mt = 0; mt < MATS; ++mt)
#pragma unroll
    for (int bk = 0; bk < NB; ++bk) s2[mt][bk] = hn_bits_h2(b.s[mt][bk] | (b.s[mt][bk] << 16));
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    half8_t bw[MATS][NB];
#pragma unroll
    for (int mt = 0; mt < MATS; ++mt)
#pragma unroll
      for (int bk = 0; bk < NB; ++bk) bw[mt][bk] = deq8(b.w[mt][bk][t], dr, s2[mt][bk]);
    const int slot = ((4 * q + t) ^ col) * 8;
#pragma unroll
    for (int rb = 0; rb < 8; ++rb) {
      if (FULL || rb < nrb) {  // uniform
        const half8_t a = *reinterpret_cast<const half8_t*>(xs + (rb * 16 + col) * 128 + slot);
#pragma unroll
        for (int mt = 0; mt < MATS; ++mt)
#pragma unroll
          for (int bk = 0; bk < NB; ++bk)
            acc[rb][mt][bk] =
                __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bw[mt][bk], acc[rb][mt][bk], 0, 0, 0);
      }
    }
  }
}

// s_waitcnt with only vmcnt = n (expcnt and lgkmcnt at their maxima; gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <int MATS, int NB, bool FULL>
__device__ __forceinline__ void main_loop(const TileLoads<MATS, NB>& tl, int group, int G,
                                          h16* xs0, h16* xs1, BBuf<MATS, NB>& b0,
                                          BBuf<MATS, NB>& b1, int nrb, int col, int q, int wave,
                                          const DeqRegs& dr, float4_t (&acc)[8][MATS][NB]) {
  constexpr int kBLoads = 2 * MATS * NB;  // weight + scale loads per group
  for (int g = 0; g < G; g += 2) {
    {
      const bool more = g + 1 < G;  // uniform
      if (more) {
        dma_a(tl.px, tl.nx, tl.va, g + 1, xs1, wave);
        __builtin_amdgcn_sched_barrier(0);
        issue_b(b1, tl, g + 1, group);
      }
      compute<MATS, NB, FULL>(b0, xs0, nrb, col, q, dr, acc);
      if (more) wait_vmcnt<kBLoads>();
      __syncthreads();
    }
    if (g + 1 < G) {
      const bool more = g + 2 < G;
      if (more) {
        dma_a(tl.px, tl.nx, tl.va, g + 2, xs0, wave);
        __builtin_amdgcn_sched_barrier(0);
        issue_b(b0, tl, g + 2, group);
      }
      compute<MATS, NB, FULL>(b1, xs1, nrb, col, q, dr, acc);
      if (more) wait_vmcnt<kBLoads>();
      __syncthreads();
    }
  }
}

template <bool GROUPED, int MATS>
__global__ __launch_bounds__(256, 2) void gemm_kernel(GemmArgs A,
                                                      const GExpert* __restrict__ table,
                                                      const int* __restrict__ active,
                                                      const int* __restrict__ n_active,
                                                      const int* __restrict__ offsets) {
  constexpr int NB = 4 / MATS;
  constexpr int WROWS = kWaves * NB * 16;  // weight rows per matrix per tile
  __shared__ __align__(16) h16 xs[2][kBM * 128];
  __shared__ int toff[kMaxProb + 1];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15;
  const int q = lane >> 4;
  const int N = A.N;
  const int G = A.K >> 7;
  const int NT = (N + WROWS - 1) / WROWS;
  DeqRegs dr;
  dr.m_pair = A.m_pair;
  dr.magic = hn_vgpr(A.magic);
  dr.mul = hn_vgpr(0x2C003C00u);  // half2(1, 0.0625)
  dr.add = hn_vgpr(0xD480E408u);  // half2(-1032, -72)

  // ---- M-tiles per problem -> prefix toff[]
  int nprob = 1;
  if (GROUPED) {
    nprob = min(*n_active, kMaxProb);
    for (int i = tid; i < nprob; i += blockDim.x) {
      const int e = active[i];
      toff[i + 1] = (offsets[e + 1] - offsets[e] + kBM - 1) / kBM;
    }
    __syncthreads();
    if (tid == 0) {
      toff[0] = 0;
      for (int i = 1; i <= nprob; ++i) toff[i] += toff[i - 1];
    }
  } else if (tid == 0) {
    toff[0] = 0;
    toff[1] = (A.M + kBM - 1) / kBM;
  }
  __syncthreads();
  if (nprob <= 0) return;
  const int total = __builtin_amdgcn_readfirstlane(toff[nprob]) * NT;
  const int nwg = gridDim.x;
  const int bid = blockIdx.x;
  // workgroups are dealt round-robin to the 8 XCDs: give each XCD a
  // contiguous run of tile numbers
  const int vid = (nwg % 8 == 0) ? (bid % 8) * (nwg / 8) + bid / 8 : bid;

  for (int tile = vid; tile < total; tile += nwg) {
    // ---- tile -> (problem, m-tile, n-tile)
    int p = 0;
    {
      const int mg = tile / NT;  // toff[p] <= mg < toff[p + 1]
      int lo = 0, hi = nprob - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (toff[mid] <= mg) lo = mid; else hi = mid - 1;
      }
      p = lo;
    }
    const int pt0 = toff[p], mtp = toff[p + 1] - pt0;
    const int local = tile - pt0 * NT;
    const int sb = local / (kSuperM * NT);           // super-block
    const int sm0 = sb * kSuperM;
    const int sbm = min(kSuperM, mtp - sm0);         // M-tiles in this super-block
    const int inb = local - sb * kSuperM * NT;
    const int mtile = sm0 + inb % sbm;
    const int ntile = inb / sbm;
    const Prob pr = resolve<GROUPED>(A, table, active, offsets, p);
    const int m0 = mtile * kBM;
    const int rows = min(kBM, pr.rows - m0);
    const int nrb = (rows + 15) >> 4;
    const int rbase = ntile * WROWS + wave * NB * 16 + col;

    TileLoads<MATS, NB> tl;
    tl.px = pr.x + (long)m0 * A.ld_x;
    tl.nx = (int)(rows * A.ld_x * 2);
#pragma unroll
    for (int j = 0; j < 8; ++j) tl.va[j] = a_offset(j, wave, lane, rows, A.ld_x);
#pragma unroll
    for (int mt = 0; mt < MATS; ++mt) {
      tl.pq[mt] = pr.q[mt];
      tl.ps[mt] = pr.s[mt];
    }
    tl.nq = N * A.ld_q;
    tl.ns = N * A.ld_s * 2;
#pragma unroll
    for (int bk = 0; bk < NB; ++bk) {
      const int row = rbase + 16 * bk;
      const bool ok = row < N;
      tl.vq[bk] = ok ? (uint32_t)(row * A.ld_q + 16 * q) : kOOB;
      tl.vs[bk] = ok ? (uint32_t)(2 * (row * A.ld_s + (32 * q) / A.group)) : kOOB;
    }
    float4_t acc[8][MATS][NB];
#pragma unroll
    for (int rb = 0; rb < 8; ++rb)
#pragma unroll
      for (int mt = 0; mt < MATS; ++mt)
#pragma unroll
        for (int bk = 0; bk < NB; ++bk) acc[rb][mt][bk] = float4_t{0.f, 0.f, 0.f, 0.f};

    BBuf<MATS, NB> b0, b1;
    constexpr int kBLoads = 2 * MATS * NB;
    // the previous tile's last reads of xs[0] end before anyone restages it
    __syncthreads();
    dma_a(tl.px, tl.nx, tl.va, 0, xs[0], wave);
    __builtin_amdgcn_sched_barrier(0);
    issue_b(b0, tl, 0, A.group);
    wait_vmcnt<kBLoads>();
    __syncthreads();

    // group g: restage g + 1 (activations first, then weights, so that the
    // wait for the activations leaves the weight loads in flight), compute g
    if (nrb == 8) main_loop<MATS, NB, true>(tl, A.group, G, xs[0], xs[1], b0, b1, nrb, col, q,
                                            wave, dr, acc);
    else main_loop<MATS, NB, false>(tl, A.group, G, xs[0], xs[1], b0, b1, nrb, col, q, wave,
                                    dr, acc);

    // ---- epilogue: lane (col, q) holds tokens rb*16 + 4q + i of row n
#pragma unroll
    for (int bk = 0; bk < NB; ++bk) {
      const int n = rbase + 16 * bk;
      if (n < N) {
#pragma unroll
        for (int rb = 0; rb < 8; ++rb) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int m = rb * 16 + 4 * q + i;
            if (m < rows) {
              h16 o;
              if (MATS == 2) {
                const float gv = (float)(h16)acc[rb][0][bk][i];
                const float uv = (float)(h16)acc[rb][MATS - 1][bk][i];
                o = (h16)(hn_silu(gv) * uv);
              } else {
                o = (h16)acc[rb][0][bk][i];
              }
              pr.out[(long)(m0 + m) * A.ld_o + n] = o;
            }
          }
        }
      }
    }
  }
}

int num_cus() {
  static int n = 0;
  if (n == 0) {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        v > 0)
      n = v;
    else
      n = 256;
  }
  return n;
}

void fill_consts(GemmArgs& A) {
  A.m_pair = 0x00F0000Fu;
  A.magic = 0x64006400u;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Workgroups: two per CU, fewer when there are fewer tiles.
int grid_for(long tiles_upper) {
  const long cap = 2L * num_cus();
  return (int)(tiles_upper < cap ? (tiles_upper < 1 ? 1 : tiles_upper) : cap);
}

}  // namespace

// Shape checks shared by the entry points below: 1 when the GEMM kernels
// handle the shape.
static int gemm_shape_ok(long N, long K, long group, long ld_q, long ld_s) {
  // the scale offset split (voffset: lane part, soffset: group part) needs
  // group in {32, 64} or a multiple of 128
  if (K <= 0 || K % 128 != 0 || K % group != 0) return 0;
  if (group != 32 && group != 64 && (group <= 0 || group % 128 != 0)) return 0;
  if (ld_q % 16 != 0) return 0;
  if (N * ld_q >= (long)kOOB || N * ld_s * 2 >= (long)kOOB) return 0;
  return 1;
}

// Single problem: out[M, N] = x @ deq(W)^T (mats 1) or the SwiGLU h (mats 2).
// Returns HN_NOT_HANDLED when the shape is not handled here, 0 after a launch,
// a HIP error code when the launch failed.
extern "C" int hn_gemm_linear_impl(int mats, const void* x, long ld_x, const void* q0,
                                   const void* s0, const void* q1, const void* s1, long ld_q,
                                   long ld_s, void* out, long ld_o, long M, long N, long K,
                                   long group, void* stream) {
  if (!gemm_shape_ok(N, K, group, ld_q, ld_s)) return HN_NOT_HANDLED;
  if (!aligned16(x) || ld_x % 8 != 0 || !aligned16(q0) || !aligned16(q1)) return HN_NOT_HANDLED;
  if (ld_x * 2 * kBM >= (long)kOOB) return HN_NOT_HANDLED;
  if (M <= 0 || N <= 0) return 0;
  GemmArgs A = {};
  A.x = (const h16*)x;
  A.ld_x = ld_x;
  A.M = (int)M;
  A.q[0] = (const uint8_t*)q0; A.s[0] = (const h16*)s0;
  A.q[1] = (const uint8_t*)q1; A.s[1] = (const h16*)s1;
  A.out = (h16*)out;
  A.ld_o = ld_o;
  A.N = (int)N;
  A.K = (int)K;
  A.group = (int)group;
  A.ld_q = (int)ld_q;
  A.ld_s = (int)ld_s;
  fill_consts(A);
  const long wrows = mats == 2 ? 128 : 256;
  const long tiles = ((M + kBM - 1) / kBM) * ((N + wrows - 1) / wrows);
  hipStream_t s = (hipStream_t)stream;
  if (mats == 2)
    hipLaunchKernelGGL((gemm_kernel<false, 2>), dim3(grid_for(tiles)), dim3(256), 0, s, A,
                       nullptr, nullptr, nullptr, nullptr);
  else
    hipLaunchKernelGGL((gemm_kernel<false, 1>), dim3(grid_for(tiles)), dim3(256), 0, s, A,
                       nullptr, nullptr, nullptr, nullptr);
  HN_LAUNCH_CHECK("hn_gemm_linear");
  return 0;
}

// Grouped over the active experts of one MoE layer; phase 0 = gate/up + SiLU
// into h [rows, I], phase 1 = down into y [rows, H].  rows = total permuted
// rows (bounds the tile count).  Same return convention.
extern "C" int hn_gemm_grouped_impl(int phase, const void* x, long ld_x, const void* table,
                                    const int* active, const int* n_active, const int* offsets,
                                    long E, long rows, long H, long I, long group, void* out,
                                    long ld_o, void* stream) {
  const long K = phase == 0 ? H : I, N = phase == 0 ? I : H;
  if (E > kMaxProb || !gemm_shape_ok(N, K, group, K / 2, K / group)) return HN_NOT_HANDLED;
  if (!aligned16(x) || ld_x % 8 != 0 || ld_x * 2 * kBM >= (long)kOOB) return HN_NOT_HANDLED;
  if (rows <= 0) return 0;
  GemmArgs A = {};
  A.x = (const h16*)x;
  A.ld_x = ld_x;
  A.out = (h16*)out;
  A.ld_o = ld_o;
  A.phase = phase;
  A.N = (int)N;
  A.K = (int)K;
  A.group = (int)group;
  A.ld_q = (int)(K / 2);
  A.ld_s = (int)(K / group);
  fill_consts(A);
  const long wrows = phase == 0 ? 128 : 256;
  const long mt_upper = (rows + kBM - 1) / kBM + (E < rows ? E : rows);
  const long tiles = mt_upper * ((N + wrows - 1) / wrows);
  hipStream_t s = (hipStream_t)stream;
  if (phase == 0)
    hipLaunchKernelGGL((gemm_kernel<true, 2>), dim3(grid_for(tiles)), dim3(256), 0, s, A,
                       (const GExpert*)table, active, n_active, offsets);
  else
    hipLaunchKernelGGL((gemm_kernel<true, 1>), dim3(grid_for(tiles)), dim3(256), 0, s, A,
                       (const GExpert*)table, active, n_active, offsets);
  HN_LAUNCH_CHECK("hn_gemm_grouped");
  return 0;
}
