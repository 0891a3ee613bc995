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
// around the MFMA pipe (v_mfma_f32_32x32x16_f16, which one wave per SIMD can
// keep busy back to back):
//  * Tile = up to 256 tokens (eight 32-token row blocks; an expert's last
//    M-tile runs the 2, 4 or 6 blocks that cover its rows) x 256 weight rows,
//    one workgroup of four waves per CU; a wave owns 64 weight rows -- one
//    32-row block of gate
//    and the same rows of up (so the SwiGLU epilogue has both values of an
//    output in one lane), or two 32-row blocks of one matrix -- for all the
//    tile's tokens.  Waves split N, never M, so each weight is dequantised by
//    exactly one wave per tile.
//  * Every load of the K loop goes HBM -> LDS directly (buffer_load ... lds,
//    with explicit waits), three LDS stages of 64 k:
//    activations (XOR-swizzled rows so A-fragment reads are conflict-free),
//    packed weights and the dwords holding the scales.
//  * Each k-step's A fragments and unpacked weights are double-buffered: step
//    s + 1's LDS reads and unpack are issued ahead of / under step s's MFMAs.
//    A packed dword becomes eight fp16 weights in k order: a byte broadcast
//    (v_perm_b32) and one bit-field insert put two nibbles in the mantissas of
//    1024 (0x6400), one v_pk_fma_f16 gives the exact (n - 8) pair, and
//    v_pk_mul_f16 by the fp16 scale rounds the exact product once: the
//    reference's dequantised weight bit for bit.
//  * Rows of a tile past the valid tokens read the last valid row (results
//    never stored).  Persistent grid: tiles are numbered per problem in
//    super-blocks of up to 8 M-tiles x n-tiles, and workgroups on one XCD
//    take consecutive numbers, so tiles running together on an XCD share
//    activation and weight slices in its L2.
//  * With a caller workspace, whole rounds of full tiles go round-robin and
//    the rest is split stream-K by cost-weighted (tile, chunk) iterations; a
//    tile whose chunks span several workgroups is summed by its last-arriving
//    wave from fp32 partials (tagged counters, agent-scope acquire,
//    hn_arrive).
#include "hn_common.h"

namespace {

constexpr int kRBMax = 8;         // 32-token row blocks of the largest tile
constexpr int kBMMax = 32 * kRBMax;  // tokens per tile, at most
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
  // stream-K (part != nullptr): the tiles short of a whole round are split by
  // cost-weighted (tile, chunk) iterations; a tile whose chunks span several
  // workgroups is summed from fp32 partial slots by the last of them to
  // arrive (per wave).
  float* part;      // [2 * grid][kWaves][kWaveSlot]
  unsigned long long* ctr;  // [items * kWaves] tagged counters (hn_arrive), left zero
  unsigned long long tag;   // this launch's counter tag (hn_next_tag)
  int sk_ch;        // stages per stream-K chunk (chunks start on whole scale groups)
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

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, bytes, 0x00020000);
}

// ---------------------------------------------------------------------------
// Loads.  Everything the K loop reads from memory goes HBM -> LDS directly
// (buffer_load ... lds: lane i's bytes land at m0 + size * i) through the
// compiler's LDS-DMA builtin, which sets M0 and places the wait states gfx9
// needs between a VALU or SALU write of an SGPR operand (M0, soffset, the
// descriptor) and the load that reads it.  The compiler does not wait on
// these loads before the K loop's LDS reads: every wait on them is explicit
// (s_waitcnt vmcnt below), and loads return in issue order.  Offsets: the
// per-lane part is in voffset (the buffer range check covers voffset only, so
// rows past N carry an offset past the descriptor's range and read as 0
// without touching memory); the per-group part is in soffset.
// ---------------------------------------------------------------------------
__device__ __forceinline__ lds_void_t* lds_ptr(uint32_t addr) {
  return (lds_void_t*)((__attribute__((address_space(3))) char*)nullptr + addr);
}

__device__ __forceinline__ void dma_b128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                         uint32_t lds) {
  // soffset and the LDS address are uniform by construction
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds_ptr(__builtin_amdgcn_readfirstlane(lds)), 16,
                                           voff, __builtin_amdgcn_readfirstlane(soff), 0, 0);
}

__device__ __forceinline__ void dma_b32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds_ptr(__builtin_amdgcn_readfirstlane(lds)), 4,
                                           voff, 0, 0, 0);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

// ---------------------------------------------------------------------------
// Work decomposition.  A tile is up to 256 tokens (NRB row blocks of 32) x 256
// weight rows; a workgroup of four waves computes it, each wave 64 rows: one
// 32-row block of gate and the same 32 rows of up (MATS 2, so the SwiGLU
// epilogue finds both values of an output in one lane) or two 32-row blocks
// of one matrix (MATS 1).  One workgroup per CU: its accumulators take all
// 256 AGPRs of each wave.  K advances in stages of 64: three LDS stages, the
// loads of stages t + 1 and t + 2 in flight while stage t computes.
// ---------------------------------------------------------------------------
#ifndef HN_GEMM_KSM
#define HN_GEMM_KSM 1         // k per stage = 64 * KSM
#endif
#ifndef HN_GEMM_OCC
#define HN_GEMM_OCC 1         // workgroups per CU (waves per SIMD)
#endif
constexpr int kKSM = HN_GEMM_KSM;
constexpr int kOccW = HN_GEMM_OCC;
constexpr int kBlk = 2;            // 32-row weight blocks per wave
constexpr int kKS = 64 * kKSM;     // k per stage
constexpr int kSteps = 4 * kKSM;   // MFMA k-steps (16 k) per stage
constexpr int kChunks = 8 * kKSM;  // 16-byte activation chunks per row per stage
constexpr int kNST = 3;            // LDS stages

// LDS stage (bytes): activations [256 rows][kChunks chunks of 16 B], chunk c of
// row r at slot c ^ key(r), so the 8 or 16 rows an A-fragment read serves per
// LDS cycle hit distinct banks; packed weights [wave][block][d][lane] 16 B;
// scale dwords [wave][block][lane] 4 B.
struct Stage {
  static constexpr int kA = 0;
  static constexpr int kB = kBMMax * kChunks * 16;
  static constexpr int kS = kB + kWaves * kBlk * kKSM * 1024;
  static constexpr int kSize = kS + kWaves * kBlk * 256;
};
// activation loads per lane for a tile of NRB row blocks; loads per stage
template <int NRB> constexpr int a_loads() { return kChunks * 32 * NRB / (kWaves * 64); }
template <int NRB> constexpr int loads_per_stage() { return a_loads<NRB>() + kBlk * kKSM + kBlk; }
constexpr int kALoadsMax = a_loads<kRBMax>();

__device__ __forceinline__ int akey(int r) {
  return kChunks == 16 ? (r & 15) : ((r & 7) ^ ((r >> 3) & 1));
}

// Per-tile load state.  (Buffer descriptors are rebuilt from the pointers at
// each use -- a few scalar moves the compiler hoists; descriptor types cannot
// be struct members in the host pass.)  Block b of the wave: matrix pq[b],
// rows row0[b] .. + 32.
struct TileLoads {
  const void* px; int nx;             // activation rows of the tile, bytes
  const void* pq[kBlk];               // packed weights of each block's matrix
  const void* ps[kBlk];               // scales
  int nq, ns;                         // bytes of one packed / scale matrix
  uint32_t va[kALoadsMax];            // activation chunk offsets (first a_loads<NRB>)
  uint32_t vq[kBlk];                  // weight byte offset of (lane's row, lane's 16 B)
  uint32_t vs[kBlk];                  // scale byte offset of (lane's row, lane's k)
  int group;
};

// Activation loads: wave w issues a_loads<NRB> loads of 64 consecutive LDS
// chunks (1 KiB each); LDS chunk L = (row r, slot c') holds global chunk
// c' ^ key(r) of row r.  Rows past the valid ones repeat the last valid row
// (their results are never stored).
template <int NRB>
__device__ __forceinline__ uint32_t a_offset(int j, int wave, int lane, int rows, long ld_x) {
  const int L = (wave * a_loads<NRB>() + j) * 64 + lane;
  const int r = L / kChunks;
  const int c = (L % kChunks) ^ akey(r);
  return (uint32_t)((min(r, rows - 1) * (int)ld_x + 8 * c) * 2);
}

// Issue stage t's loads into the LDS stage at byte address st.  Weights: per
// block kKSM loads; load d brings lane l's 16 bytes at 16 kKSM (l / 32) + 16 d
// of row (l % 32)'s 32 kKSM bytes of the stage.  Scales: the dword holding the
// lane's scale.  With real false the same loads go out against empty buffer
// ranges: they read nothing from memory (out of range), write zeros into a
// stage no one reads, and keep the count of loads per stage fixed, so the
// K loop's waits are the same at every stage (no branch in the loop).
template <int NRB>
__device__ __forceinline__ void issue_stage(const TileLoads& tl, int t, uint32_t st, int wave,
                                            bool real) {
  using L = Stage;
  constexpr int NA = a_loads<NRB>();
  {
    const __amdgpu_buffer_rsrc_t r = rsrc(tl.px, real ? tl.nx : 0);
#pragma unroll
    for (int j = 0; j < NA; ++j)
      dma_b128(r, tl.va[j], 2 * kKS * t, st + L::kA + (wave * NA + j) * 1024);
  }
#pragma unroll
  for (int b = 0; b < kBlk; ++b) {
    const __amdgpu_buffer_rsrc_t r = rsrc(tl.pq[b], real ? tl.nq : 0);
#pragma unroll
    for (int d = 0; d < kKSM; ++d)
      dma_b128(r, tl.vq[b] + 16 * d, kKS / 2 * t,
               st + L::kB + ((wave * kBlk + b) * kKSM + d) * 1024);
  }
  const uint32_t soff = 2 * ((kKS * t) / tl.group);
#pragma unroll
  for (int b = 0; b < kBlk; ++b)
    dma_b32(rsrc(tl.ps[b], real ? tl.ns : 0), (tl.vs[b] + soff) & ~3u,
            st + L::kS + (wave * kBlk + b) * 256);
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
    const half2_t v = hn_bits_h2((t & c.m_pair) | c.magic);           // (1024+n, 1024+16n')
    const half2_t d = __builtin_elementwise_fma(v, hn_bits_h2(c.mul), hn_bits_h2(c.add));
    r[j] = __builtin_bit_cast(uint32_t, d * s2);
  }
  return __builtin_bit_cast(half8_t, r);
}

template <typename T>
__device__ __forceinline__ T lds_read(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) T*>(
      (__attribute__((address_space(3))) char*)nullptr + addr);
}

// MFMA v_mfma_f32_32x32x16_f16: lane l supplies A[row l % 32][k 8 (l / 32) + 0..7],
// B[k 8 (l / 32) + 0..7][col l % 32] and holds D[8 (r / 4) + 4 (l / 32) + r % 4]
// [l % 32], r = 0..15.  In a stage, step s (0..3) gives lane half h the 8 k of
// chunk kSteps h + s: the 16 kKSM packed bytes a lane loaded are its steps.
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Operand registers of one wave.  A fragments and unpacked weights are
// double-buffered over steps: step s + 1's LDS reads and unpack are issued
// ahead of step s's MFMAs into the other buffer.
struct Ops {
  uint32_t pk[kBlk][kSteps];  // packed weights of the current stage, one dword per step
  uint32_t sv[kBlk];      // scales as read (fp16 bits in the low half)
  half2_t s2[kBlk];       // scales, both halves
  half8_t af[2][kRBMax];  // A fragments of the row blocks
  half8_t bw[2][kBlk];    // unpacked weights
};

__device__ __forceinline__ uint32_t a_addr(uint32_t st, int s, int row32, int h) {
  return st + row32 * (kChunks * 16) + (((h * kSteps + s) ^ akey(row32)) << 4);
}

template <int NRB>
__device__ __forceinline__ void read_a(Ops& o, int buf, uint32_t st, int s, int row32, int h) {
  const uint32_t base = a_addr(st, s, row32, h);
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb)
    o.af[buf][rb] = lds_read<half8_t>(base + rb * 32 * kChunks * 16);
}

// Weights + scales of the stage at st (stage number t); half-word of each
// scale dword from the byte offset the dword was loaded for.  LDS reads only:
// the scales are put in both halves by the first unpack of the stage.
__device__ __forceinline__ void read_b(Ops& o, const TileLoads& tl, uint32_t st, int t, int wave,
                                       int lane) {
  using L = Stage;
  const uint32_t soff = 2 * ((kKS * t) / tl.group);
#pragma unroll
  for (int b = 0; b < kBlk; ++b) {
#pragma unroll
    for (int d = 0; d < kKSM; ++d) {
      const u32x4 v =
          lds_read<u32x4>(st + L::kB + ((wave * kBlk + b) * kKSM + d) * 1024 + lane * 16);
#pragma unroll
      for (int i = 0; i < 4; ++i) o.pk[b][4 * d + i] = v[i];
    }
    const uint32_t hsel = (tl.vs[b] + soff) & 2u;
    o.sv[b] = lds_read<unsigned short>(st + L::kS + (wave * kBlk + b) * 256 + lane * 4 + hsel);
  }
}

__device__ __forceinline__ void deq_step(Ops& o, int buf, int s, const DeqRegs& dr) {
#pragma unroll
  for (int b = 0; b < kBlk; ++b) {
    if (s == 0) o.s2[b] = hn_bits_h2(o.sv[b] | (o.sv[b] << 16));
    o.bw[buf][b] = deq8(o.pk[b][s], dr, o.s2[b]);
  }
}

// MFMAs I0 .. I1 - 1 of a step, in the order (row block, weight block).
template <int I0, int I1>
__device__ __forceinline__ void mfma_range(const Ops& o, int buf, f32x16 (&acc)[kRBMax][kBlk]) {
#pragma unroll
  for (int i = I0; i < I1; ++i)
    acc[i / kBlk][i % kBlk] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
        o.af[buf][i / kBlk], o.bw[buf][i % kBlk], acc[i / kBlk][i % kBlk], 0, 0, 0);
}

// Interleave hint for one step: NRB kBlk x (1 MFMA, 16 / NRB VALU), with one
// of the next step's NRB A-fragment reads after every kBlk-th MFMA -- the
// next step's LDS reads and unpack under this step's MFMAs.  (Issued as a
// burst, the reads stall the wave's issue and the MFMA pipe with it:
// measured on MI355X, a stage of 64 MFMAs with its 32 reads in bursts took
// about 20 % longer than with them spread.)
template <int NRB>
__device__ __forceinline__ void sched_step() {
#pragma unroll
  for (int i = 0; i < NRB * kBlk; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);              // MFMA
    if (i % kBlk == 0) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
    __builtin_amdgcn_sched_group_barrier(0x002, 16 / NRB, 0);       // VALU
  }
}

// K loop of one tile over stages [tb, te) of kKS k each.  In a stage, step s's
// MFMAs overlap the unpack and A-fragment reads of step s + 1.  The last step
// is ordered by hand (scheduling fences; the compiler would otherwise hoist
// the barrier above the MFMAs and sink the unpack below it): the wave waits
// for its own loads of stage t + 1 (those of t + 2 stay in flight) and reads
// that stage's weights, issues a few MFMAs under the read, unpacks the next
// stage's first step under most of the rest, meets the other waves at the
// barrier (every wave's activation loads of t + 1 now visible, every read of
// stage t done) and reads the next stage's first A fragments under the last
// POST MFMAs.  Every stage issues the same loads (dummies past the end), so
// the waits take no branch; the loop ends waiting for all of them.
template <int NRB>
__device__ __forceinline__ void k_loop(const TileLoads& tl, int tb, int te, uint32_t lds0,
                                       int row32, int h, int wave, int lane, const DeqRegs& dr,
                                       f32x16 (&acc)[kRBMax][kBlk]) {
  using L = Stage;
  constexpr int LPS = loads_per_stage<NRB>();
  constexpr int NM = NRB * kBlk;                   // MFMAs per step
  constexpr int POST = NM / 2 < 6 ? NM / 2 : 6;    // MFMAs after the barrier
  constexpr int PRE = NM - POST;
  constexpr int COVER = PRE >= 8 ? 3 : (PRE >= 4 ? 2 : 1);  // MFMAs under the weight reads
  constexpr int VPM = PRE > COVER ? (40 + PRE - COVER - 1) / (PRE - COVER) : 40;
  Ops o;
  issue_stage<NRB>(tl, tb, lds0, wave, true);
  issue_stage<NRB>(tl, tb + 1 < te ? tb + 1 : tb, lds0 + L::kSize, wave, tb + 1 < te);
  wait_vmcnt<LPS>();
  __syncthreads();
  read_b(o, tl, lds0, tb, wave, lane);
  deq_step(o, 0, 0, dr);
  read_a<NRB>(o, 0, lds0, 0, row32, h);
  int sc = 0;  // LDS stage of stage t
  for (int t = tb; t < te; ++t) {
    const int s1 = sc + 1 == kNST ? 0 : sc + 1;
    const int s2 = s1 + 1 == kNST ? 0 : s1 + 1;
    const uint32_t cur = lds0 + sc * L::kSize;
    const uint32_t nxt = lds0 + s1 * L::kSize;
    const bool ahead = t + 2 < te;  // uniform
    issue_stage<NRB>(tl, ahead ? t + 2 : t, lds0 + s2 * L::kSize, wave, ahead);
#pragma unroll
    for (int s = 0; s < kSteps - 1; ++s) {
      // step s + 1's A fragments and unpack under step s's MFMAs
      read_a<NRB>(o, (s + 1) & 1, cur, s + 1, row32, h);
      deq_step(o, (s + 1) & 1, s + 1, dr);
      mfma_range<0, NM>(o, s & 1, acc);
      sched_step<NRB>();
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_vmcnt<LPS>();
    read_b(o, tl, nxt, t + 1, wave, lane);
    __builtin_amdgcn_sched_barrier(0);
    mfma_range<0, COVER>(o, 1, acc);
    __builtin_amdgcn_sched_barrier(0);
    deq_step(o, 0, 0, dr);
    mfma_range<COVER, PRE>(o, 1, acc);
#pragma unroll
    for (int i = COVER; i < PRE; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);  // VALU
    }
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    read_a<NRB>(o, 0, nxt, 0, row32, h);  // past the last stage: unused
    __builtin_amdgcn_sched_barrier(0);
    mfma_range<PRE, NM>(o, 1, acc);
    __builtin_amdgcn_sched_barrier(0);
    sc = s1;
  }
  // the last stages' dummy loads have landed before the K loop returns: the
  // next tile's loads (after a barrier) may write the same LDS bytes from
  // another wave when its row blocks differ, and loads of different waves
  // land in no fixed order
  wait_vmcnt<0>();
}

// Stream-K partial slots: one wave's accumulators (kRBMax x kBlk 32x32 fp32
// blocks), lane-interleaved so every store / load instruction is coalesced.
constexpr long kWaveSlot = (long)kRBMax * kBlk * 16 * 64;  // floats

// Work.  A problem's M-tiles are RBM row blocks each ("full"), except its
// last when that needs fewer: it runs the even number of blocks (2, 4, 6)
// that covers its rows ("tail"), so rows past a problem's end cost at most
// one block of MFMAs.  Tiles are numbered full ones first (problem by
// problem, super-blocks of kSuperM M-tiles x all n-tiles), then tails
// (problem by problem, n-tile by n-tile).
//
// Without a workspace every workgroup takes whole tiles round-robin.  With
// one, whole rounds of full tiles go round-robin (one tile per workgroup per
// round, all of equal cost: nothing to split), and the rest -- the full tiles
// short of a round, then the tails -- are dealt out stream-K: their (tile,
// chunk) iterations are numbered item by item and dealt by weight, a chunk of
// a tile running w row blocks counting w + kTailC units (the stage's cost:
// MFMAs per row block plus a part that does not shrink with the rows --
// weight loads and unpack, barrier); rank r takes the chunks that start in
// units [U r / nr, U (r + 1) / nr).  Every range holds at least as many units
// as the largest chunk (nr <= U / (RBM + kTailC)), so it holds a chunk start:
// no rank is idle, and the ranks holding a tile's chunks are consecutive.  A
// tile whose chunks belong to several ranks ("segments") is finished by the
// wave that arrives last: every segment stores its fp32 partial (relaxed
// agent-scope atomics), publishes them and counts itself in (hn_arrive); the
// last one acquires, sums the partials from the slots in segment order
// (deterministic) and resets the counter.
#ifndef HN_GEMM_TAILC
#define HN_GEMM_TAILC 4
#endif
constexpr int kTailC = HN_GEMM_TAILC;  // fixed stage cost, in row blocks' MFMA time

struct SkPlan {
  long U;            // units
  int nr;            // ranks
  int RF;            // full tiles dealt stream-K (items 0 .. RF - 1), before the tails
  int wF;            // their weight per chunk
  int NT, NCH, nprob;
  const int* thalf;  // tail M-tiles per problem, prefix (LDS)
  const int* wt;     // row blocks of each problem's tail M-tile (LDS)
  const long* upre;  // tail units per problem, prefix (LDS)

  __device__ long UF() const { return (long)RF * NCH * wF; }
  // first unit of chunk c of item i (a tail of problem p when i >= RF)
  __device__ long unit(int i, int c, int p) const {
    if (i < RF) return ((long)i * NCH + c) * wF;
    return UF() + upre[p] + ((long)(i - RF - thalf[p] * NT) * NCH + c) * (wt[p] + kTailC);
  }
  // number (item NCH + chunk) of the first chunk that starts at unit u or
  // later (the chunk count when none does)
  __device__ long chunk_at(long u) const {
    if (u < UF()) return (u + wF - 1) / wF;
    if (u >= U) return ((long)RF + (long)thalf[nprob] * NT) * NCH;
    const long ut = u - UF();
    int lo = 0, hi = nprob - 1;  // the largest p with upre[p] <= ut: it has a tail
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (upre[mid] <= ut) lo = mid; else hi = mid - 1;
    }
    const int w = wt[lo] + kTailC;
    return ((long)RF + (long)thalf[lo] * NT) * NCH + (ut - upre[lo] + w - 1) / w;
  }
  __device__ long bound(int r) const { return U * r / nr; }
  // rank whose range holds unit u: the largest r with U r / nr <= u
  __device__ int owner(long u) const { return (int)(((u + 1) * nr + U - 1) / U - 1); }
  // a rank's partial slot for an item: 2 r, + 1 unless the item is the rank's
  // first (a rank splits at most its first and its last item)
  __device__ long slot(int r, int item) const {
    return 2L * r + (chunk_at(bound(r)) / NCH == item ? 0 : 1);
  }
};

struct SkSeg {
  int wf, nseg;  // first rank of the tile's segments, their number
};

// Stores this wave's partial and counts it in.  True when it was the last
// segment of the tile (the caller then finishes the tile from the slots).
template <int RBM>
__device__ __forceinline__ bool streamk_arrive(const GemmArgs& A, const SkPlan& sp,
                                               const f32x16 (&acc)[kRBMax][kBlk], int nrb,
                                               int item, int p, int rank, int wave, int lane,
                                               SkSeg& sgi) {
  sgi.wf = sp.owner(sp.unit(item, 0, p));
  sgi.nseg = sp.owner(sp.unit(item, sp.NCH - 1, p)) - sgi.wf + 1;
  float* mine = A.part + (sp.slot(rank, item) * kWaves + wave) * kWaveSlot;
#pragma unroll
  for (int rb = 0; rb < RBM; ++rb)
    if (rb < nrb)  // uniform
#pragma unroll
      for (int b = 0; b < kBlk; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          __hip_atomic_store(mine + ((rb * kBlk + b) * 16 + r) * 64 + lane, acc[rb][b][r],
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  hn_publish_partials();
  unsigned long long* c = A.ctr + (long)item * kWaves + wave;
  int n = 0;
  if (lane == 0) n = hn_arrive(c, A.tag);
  n = __builtin_amdgcn_readfirstlane(n);
  if (n != sgi.nseg - 1) return false;
  hn_acquire_agent();
  if (lane == 0) hn_counter_reset(c);
  return true;
}

// Row block rb of the tile summed over its segments' partial slots, in
// segment order: v[b][r] for the wave's weight block b, accumulator register
// r.  Plain loads: the caller's agent-scope acquire (L2 invalidate) has made
// the other segments' stores, written through past their L2s, visible to
// them; two segments' loads are in flight together.
__device__ __forceinline__ void sk_sum_rb(const GemmArgs& A, const SkPlan& sp, const SkSeg& sgi,
                                          int item, int wave, int lane, int rb,
                                          float (&v)[kBlk][16]) {
  for (int s0 = 0; s0 < sgi.nseg; s0 += 2) {
    float t[2][kBlk][16];
#pragma unroll
    for (int q = 0; q < 2; ++q)
      if (s0 + q < sgi.nseg) {  // uniform
        const float* src = A.part + (sp.slot(sgi.wf + s0 + q, item) * kWaves + wave) * kWaveSlot +
                           (long)rb * kBlk * 16 * 64 + lane;
#pragma unroll
        for (int b = 0; b < kBlk; ++b)
#pragma unroll
          for (int r = 0; r < 16; ++r) t[q][b][r] = src[(b * 16 + r) * 64];
      }
#pragma unroll
    for (int q = 0; q < 2; ++q)
      if (s0 + q < sgi.nseg)
#pragma unroll
        for (int b = 0; b < kBlk; ++b)
#pragma unroll
          for (int r = 0; r < 16; ++r) v[b][r] = s0 + q == 0 ? t[q][b][r] : v[b][r] + t[q][b][r];
  }
}

// The K loop of a tile of NRB row blocks, with the activation offsets for it.
template <int NRB>
__device__ __forceinline__ void tile_k(TileLoads& tl, int rows, long ld_x, int nst, uint32_t lds0,
                                       int row32, int h, int wave, int lane, const DeqRegs& dr,
                                       f32x16 (&acc)[kRBMax][kBlk]) {
#pragma unroll
  for (int j = 0; j < a_loads<NRB>(); ++j) tl.va[j] = a_offset<NRB>(j, wave, lane, rows, ld_x);
  k_loop<NRB>(tl, 0, nst, lds0, row32, h, wave, lane, dr, acc);
}

// Stores row block rb of the tile's output: lane holds column n (+ 32 ob),
// tokens 32 rb + 8 (r / 4) + 4 h + r % 4.  MATS 2: silu(g) * u.
template <int MATS>
__device__ __forceinline__ void store_rb(const Prob& pr, const GemmArgs& A, int m0, int rows,
                                         int n0, int N, int h, int rb, const float (&v)[kBlk][16]) {
#pragma unroll
  for (int ob = 0; ob < kBlk / MATS; ++ob) {
    const int n = n0 + 32 * ob;
    if (n < N) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = 32 * rb + 8 * (r >> 2) + 4 * h + (r & 3);
        if (m < rows) {
          h16 o;
          if (MATS == 2) {
            // silu(g) * u in fp32 from the fp16-rounded projections; the
            // fast exp / reciprocal are well inside the fp16 rounding
            const float gv = (float)(h16)v[0][r];
            const float uv = (float)(h16)v[1][r];
            o = (h16)(gv * __builtin_amdgcn_rcpf(1.0f + __expf(-gv)) * uv);
          } else {
            o = (h16)v[ob][r];
          }
          pr.out[(long)(m0 + m) * A.ld_o + n] = o;
        }
      }
    }
  }
}

template <bool GROUPED, int MATS, int RBM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kOccW, kOccW))) void gemm_kernel(
    GemmArgs A, const GExpert* __restrict__ table, const int* __restrict__ active,
    const int* __restrict__ n_active, const int* __restrict__ offsets) {
  static_assert(RBM == 4 || RBM == 8, "M-tile of 128 or 256 tokens");
  constexpr int BM = 32 * RBM;
  constexpr int WN = kWaves * 32 * kBlk / MATS;  // output columns per tile
  using L = Stage;
  __shared__ __align__(16) unsigned char lds[kNST * L::kSize];
  __shared__ int toff[kMaxProb + 1];   // full M-tiles, prefix
  __shared__ int thalf[kMaxProb + 1];  // tail M-tiles (0 / 1 per problem), prefix
  __shared__ int twt[kMaxProb];        // row blocks of each problem's tail M-tile
  __shared__ long tunit[kMaxProb + 1]; // stream-K units of the tails, prefix
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int row32 = lane & 31;
  const int h = lane >> 5;
  const int N = A.N;
  const int T = A.K / kKS;
  const int NT = (N + WN - 1) / WN;
  const bool sk = A.part != nullptr;
  const int CH = sk ? A.sk_ch : T;
  const int NCH = T / CH;  // chunks per tile
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t*)lds;
  DeqRegs dr;
  dr.m_pair = A.m_pair;
  dr.magic = hn_vgpr(A.magic);
  dr.mul = hn_vgpr(0x2C003C00u);  // half2(1, 0.0625)
  dr.add = hn_vgpr(0xD480E408u);  // half2(-1032, -72)

  // ---- M-tiles per problem
  int nprob = 1;
  auto count = [&](int rows_p, int& nf, int& nh, int& w) {
    const int mt = (rows_p + BM - 1) / BM;
    const int rem = rows_p - (mt - 1) * BM;
    const int nrb = ((rem + 63) / 64) * 2;  // even row blocks covering the last M-tile
    const bool tail = mt > 0 && nrb < RBM;
    nh = tail ? 1 : 0;
    nf = mt - nh;
    w = tail ? nrb : 0;
  };
  if (GROUPED) {
    nprob = min(*n_active, kMaxProb);
    for (int i = tid; i < nprob; i += blockDim.x) {
      const int e = active[i];
      int nf, nh, w;
      count(offsets[e + 1] - offsets[e], nf, nh, w);
      toff[i + 1] = nf;
      thalf[i + 1] = nh;
      twt[i] = w;
    }
  } else if (tid == 0) {
    int nf, nh, w;
    count(A.M, nf, nh, w);
    toff[1] = nf;
    thalf[1] = nh;
    twt[0] = w;
  }
  __syncthreads();
  if (tid == 0) {
    toff[0] = 0;
    thalf[0] = 0;
    tunit[0] = 0;
    for (int i = 0; i < nprob; ++i) {
      toff[i + 1] += toff[i];
      thalf[i + 1] += thalf[i];
      tunit[i + 1] = tunit[i] + (twt[i] ? (long)NT * NCH * (twt[i] + kTailC) : 0);
    }
  }
  __syncthreads();
  if (nprob <= 0) return;
  const int tot_f = __builtin_amdgcn_readfirstlane(toff[nprob]) * NT;   // full tiles
  const int tot_h = __builtin_amdgcn_readfirstlane(thalf[nprob]) * NT;  // tail tiles
  const int nwg = gridDim.x;
  const int bid = blockIdx.x;
  // workgroups are dealt round-robin to the 8 XCDs: give each XCD a
  // contiguous run of tile numbers
  const int vid = (nwg % 8 == 0) ? (bid % 8) * (nwg / 8) + bid / 8 : bid;

  // full tiles taken whole, round-robin; the stream-K plan for the rest
  const int R = sk ? tot_f - tot_f % nwg : tot_f;
  SkPlan sp;
  sp.RF = tot_f - R;
  sp.wF = RBM + kTailC;
  sp.NT = NT;
  sp.NCH = NCH;
  sp.nprob = nprob;
  sp.thalf = thalf;
  sp.wt = twt;
  sp.upre = tunit;
  sp.U = sp.UF() + tunit[nprob];
  sp.nr = (int)max(1L, min((long)nwg, sp.U / (RBM + kTailC)));
  // A segment starts the K loop at stage 0 of tile pointers moved to its
  // first chunk (whole scale dwords), so the loop never starts at a
  // run-time stage.
  long it = 0, it_end = 0;  // stream-K: this rank's chunk range
  if (sk && vid < sp.nr) {
    it = sp.chunk_at(sp.bound(vid));
    it_end = sp.chunk_at(sp.bound(vid + 1));
  }
  int g_rr = vid;  // next whole tile (round-robin): full tiles < R, then (no workspace) tails
  const int tot_rr = sk ? R : tot_f + tot_h;
  while (true) {
    int g, c0, c1;   // tile number (full ones first, then tails), its chunks
    int item = -1;   // stream-K item (>= 0: counters and slots)
    if (g_rr < tot_rr) {
      g = g_rr;
      g_rr += nwg;
      c0 = 0;
      c1 = NCH;
    } else if (it < it_end) {
      item = (int)(it / NCH);
      c0 = (int)(it - (long)item * NCH);
      c1 = (int)min((long)NCH, (long)c0 + (it_end - it));
      it += c1 - c0;
      g = item < sp.RF ? R + item : tot_f + (item - sp.RF);
    } else {
      break;
    }
    g = __builtin_amdgcn_readfirstlane(g);
    c0 = __builtin_amdgcn_readfirstlane(c0);
    c1 = __builtin_amdgcn_readfirstlane(c1);
    const int k0 = c0 * CH * kKS;               // first k of this segment
    const int nst = (c1 - c0) * CH;              // its stages
    // ---- tile -> (problem, m-tile, n-tile, row blocks)
    const bool tail = g >= tot_f;
    const int tile = tail ? g - tot_f : g;
    const int* pref = tail ? thalf : toff;
    int p = 0;
    {
      const int mg = tile / NT;  // pref[p] <= mg < pref[p + 1]
      int lo = 0, hi = nprob - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (pref[mid] <= mg) lo = mid; else hi = mid - 1;
      }
      p = __builtin_amdgcn_readfirstlane(lo);  // uniform: keep the tile state in SGPRs
    }
    int mtile, ntile, nrb;
    if (!tail) {
      const int pt0 = __builtin_amdgcn_readfirstlane(toff[p]);
      const int mtp = __builtin_amdgcn_readfirstlane(toff[p + 1]) - pt0;
      const int local = tile - pt0 * NT;
      const int sb = local / (kSuperM * NT);           // super-block
      const int sm0 = sb * kSuperM;
      const int sbm = min(kSuperM, mtp - sm0);         // M-tiles in this super-block
      const int inb = local - sb * kSuperM * NT;
      mtile = sm0 + inb % sbm;
      ntile = inb / sbm;
      nrb = RBM;
    } else {
      // the problem's tail M-tile comes after its full ones
      mtile = __builtin_amdgcn_readfirstlane(toff[p + 1] - toff[p]);
      ntile = tile - __builtin_amdgcn_readfirstlane(thalf[p]) * NT;
      nrb = __builtin_amdgcn_readfirstlane(twt[p]);
    }
    const Prob pr = resolve<GROUPED>(A, table, active, offsets, p);
    const int m0 = mtile * BM;
    const int rows = min(BM, pr.rows - m0);
    // output column of this lane in block 0
    const int n0 = ntile * WN + wave * 32 * kBlk / MATS + row32;

    TileLoads tl;
    tl.px = pr.x + (long)m0 * A.ld_x + k0;
    tl.nx = (int)(rows * A.ld_x * 2 - 2 * k0);
    tl.nq = N * A.ld_q - k0 / 2;
    tl.ns = (N * A.ld_s - k0 / A.group) * 2;
    tl.group = A.group;
#pragma unroll
    for (int b = 0; b < kBlk; ++b) {
      const int mt = MATS == 2 ? b : 0;
      const int row = MATS == 2 ? n0 : n0 + 32 * b;
      tl.pq[b] = pr.q[mt] + k0 / 2;
      tl.ps[b] = pr.s[mt] + k0 / A.group;
      const bool ok = row < N;
      tl.vq[b] = ok ? (uint32_t)(row * A.ld_q + 16 * kKSM * h) : kOOB;
      tl.vs[b] = ok ? (uint32_t)(2 * (row * A.ld_s + (A.group == 32 * kKSM ? h : 0))) : kOOB;
    }
    f32x16 acc[kRBMax][kBlk];
#pragma unroll
    for (int rb = 0; rb < RBM; ++rb)
#pragma unroll
      for (int b = 0; b < kBlk; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[rb][b][r] = 0.f;

    // the previous tile's last reads of the stages end before anyone restages
    __syncthreads();
    if (RBM == 8 && nrb == 8)
      tile_k<RBM>(tl, rows, A.ld_x, nst, lds0, row32, h, wave, lane, dr, acc);
    else if (RBM == 8 && nrb == 6)
      tile_k<(RBM == 8 ? 6 : 2)>(tl, rows, A.ld_x, nst, lds0, row32, h, wave, lane, dr, acc);
    else if (nrb == 4)
      tile_k<4>(tl, rows, A.ld_x, nst, lds0, row32, h, wave, lane, dr, acc);
    else
      tile_k<2>(tl, rows, A.ld_x, nst, lds0, row32, h, wave, lane, dr, acc);
    if (c0 != 0 || c1 != NCH) {  // a segment of the tile (uniform)
      SkSeg sgi;
      if (!streamk_arrive<RBM>(A, sp, acc, nrb, item, p, vid, wave, lane, sgi))
        continue;  // another segment finishes this wave's part of the tile
      // last segment: the epilogue from the partial slots (acc no longer used)
#pragma unroll 1
      for (int rb = 0; rb < nrb; ++rb) {
        float v[kBlk][16];
        sk_sum_rb(A, sp, sgi, item, wave, lane, rb, v);
        store_rb<MATS>(pr, A, m0, rows, n0, N, h, rb, v);
      }
      continue;
    }

    // ---- epilogue from the accumulators
#pragma unroll
    for (int rb = 0; rb < RBM; ++rb) {
      float v[kBlk][16];
#pragma unroll
      for (int b = 0; b < kBlk; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) v[b][r] = acc[rb][b][r];
      store_rb<MATS>(pr, A, m0, rows, n0, N, h, rb, v);
    }
  }
}

int num_cus() { return hn_device_cus(); }

void fill_consts(GemmArgs& A) {
  A.m_pair = 0x00F0000Fu;
  A.magic = 0x64006400u;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

constexpr int kOcc = kOccW;  // workgroups per CU
#ifndef HN_GEMM_RB_GU
#define HN_GEMM_RB_GU 8
#endif
#ifndef HN_GEMM_RB_DN
#define HN_GEMM_RB_DN 8
#endif
constexpr int kRBGateUp = HN_GEMM_RB_GU;  // row blocks per M-tile, grouped gate/up
constexpr int kRBDown = HN_GEMM_RB_DN;    // and grouped down

// Workgroups: OCC per CU, fewer when there are fewer tiles.
int grid_for(long tiles_upper) {
  const long cap = (long)kOcc * num_cus();
  return (int)(tiles_upper < cap ? (tiles_upper < 1 ? 1 : tiles_upper) : cap);
}

// Stream-K workspace: per-(item, wave) counters, then two partial slots per
// workgroup of the full grid (its first and its last item).
constexpr long kSkCounters = 1L << 16;          // tiles * kWaves
constexpr long kSkCtrBytes = kSkCounters * 8;
constexpr int kSkMaxGrid = 256;   // workgroups (one per CU on MI355X)
static_assert(kSkMaxGrid <= kHnMaxArrivals, "segments per tile fit a counter");

long sk_bytes() { return kSkCtrBytes + 2L * kSkMaxGrid * kWaves * kWaveSlot * 4; }

// Stream-K over the full grid when the workspace holds its counters and slots
// (then every CU takes an equal share of the k-stages, tiles split at the
// shares' ends); else whole tiles round-robin.
bool sk_setup(GemmArgs& A, void* work, long work_bytes, long tiles_upper, dim3& grid) {
  const int g = kOcc * num_cus();
  if (!work || work_bytes < sk_bytes() || tiles_upper * kWaves > kSkCounters || g > kSkMaxGrid)
    return false;
  // chunk: the largest divisor of the stages per tile up to 16 whose k span
  // is an even number of scale groups (segment pointers then move by whole
  // scale dwords)
  const int T = A.K / kKS;
  int ch = 0;
  for (int c = T < 16 ? T : 16; c >= 1; --c)
    if (T % c == 0 && (c * kKS) % (2 * A.group) == 0) { ch = c; break; }
  if (ch == 0) return false;
  A.sk_ch = ch;
  A.ctr = (unsigned long long*)work;
  A.tag = hn_next_tag();
  A.part = (float*)((char*)work + kSkCtrBytes);
  grid = dim3(g);
  return true;
}



}  // namespace

// Shape checks shared by the entry points below: 1 when the GEMM kernels
// handle the shape.
static int gemm_shape_ok(long N, long K, long group, long ld_q, long ld_s) {
  // a lane's 32 kKSM k of a stage share one scale, and the scale offset split
  // (voffset: lane part, soffset: stage part) needs group 32 kKSM or a
  // multiple of the stage
  if (K <= 0 || K % kKS != 0 || group <= 0 || K % group != 0) return 0;
  if (group != 32 * kKSM && group % kKS != 0) return 0;
  if (ld_q % 16 != 0) return 0;
  if (N * ld_q >= (long)kOOB || N * ld_s * 2 >= (long)kOOB) return 0;
  return 1;
}

// Single problem: out[M, N] = x @ deq(W)^T (mats 1) or the SwiGLU h (mats 2).
// Returns HN_NOT_HANDLED when the shape is not handled here, 0 after a launch,
// a HIP error code when the launch failed.
// Bytes of workspace for the stream-K split (a caller's workspace of at least
// this size enables it; the counters must be zero at the first use and are
// left at zero).
extern "C" long hn_gemm_workspace_bytes() { return sk_bytes(); }

extern "C" int hn_gemm_linear_impl(int mats, const void* x, long ld_x, const void* q0,
                                   const void* s0, const void* q1, const void* s1, long ld_q,
                                   long ld_s, void* out, long ld_o, long M, long N, long K,
                                   long group, void* work, long work_bytes, void* stream) {
  if (!gemm_shape_ok(N, K, group, ld_q, ld_s)) return HN_NOT_HANDLED;
  if (!aligned16(x) || ld_x % 8 != 0 || !aligned16(q0) || !aligned16(q1)) return HN_NOT_HANDLED;
  if (ld_x * 2 * kBMMax >= (long)kOOB) return HN_NOT_HANDLED;
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
  const long wn = kWaves * 32 * kBlk / mats;
  const long bm = M > 128 ? 256 : 128;  // M-tile
  const long tiles = ((M + bm - 1) / bm) * ((N + wn - 1) / wn);
  hipStream_t s = (hipStream_t)stream;
  dim3 grid(grid_for(tiles));
  sk_setup(A, work, work_bytes, tiles, grid);
  if (mats == 2 && bm == 256)
    hipLaunchKernelGGL((gemm_kernel<false, 2, 8>), grid, dim3(256), 0, s, A, nullptr, nullptr,
                       nullptr, nullptr);
  else if (mats == 2)
    hipLaunchKernelGGL((gemm_kernel<false, 2, 4>), grid, dim3(256), 0, s, A, nullptr, nullptr,
                       nullptr, nullptr);
  else if (bm == 256)
    hipLaunchKernelGGL((gemm_kernel<false, 1, 8>), grid, dim3(256), 0, s, A, nullptr, nullptr,
                       nullptr, nullptr);
  else
    hipLaunchKernelGGL((gemm_kernel<false, 1, 4>), grid, dim3(256), 0, s, A, nullptr, nullptr,
                       nullptr, nullptr);
  HN_LAUNCH_CHECK("hn_gemm_linear");
  return 0;
}

// Grouped over the active experts of one MoE layer; phase 0 = gate/up + SiLU
// into h [rows, I], phase 1 = down into y [rows, H].  rows = total permuted
// rows (bounds the tile count).  Same return convention.
extern "C" int hn_gemm_grouped_impl(int phase, const void* x, long ld_x, const void* table,
                                    const int* active, const int* n_active, const int* offsets,
                                    long E, long rows, long H, long I, long group, void* out,
                                    long ld_o, void* work, long work_bytes, void* stream) {
  const long K = phase == 0 ? H : I, N = phase == 0 ? I : H;
  if (E > kMaxProb || !gemm_shape_ok(N, K, group, K / 2, K / group)) return HN_NOT_HANDLED;
  if (!aligned16(x) || ld_x % 8 != 0 || ld_x * 2 * kBMMax >= (long)kOOB) return HN_NOT_HANDLED;
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
  // 256-token M-tiles (128-token ones for the short remainders); with the
  // stream-K workspace the work spreads evenly whatever the tile count
  const long wn = kWaves * 32 * kBlk / (phase == 0 ? 2 : 1);
  const long bm = phase == 0 ? 32 * kRBGateUp : 32 * kRBDown;
  const long mt_upper = (rows + bm - 1) / bm + (E < rows ? E : rows);
  const long tiles = mt_upper * ((N + wn - 1) / wn);
  hipStream_t s = (hipStream_t)stream;
  dim3 grid(grid_for(tiles));
  sk_setup(A, work, work_bytes, tiles, grid);
  const GExpert* tb = (const GExpert*)table;
  if (phase == 0)
    hipLaunchKernelGGL((gemm_kernel<true, 2, kRBGateUp>), grid, dim3(256), 0, s, A, tb, active,
                       n_active, offsets);
  else
    hipLaunchKernelGGL((gemm_kernel<true, 1, kRBDown>), grid, dim3(256), 0, s, A, tb, active,
                       n_active, offsets);
  HN_LAUNCH_CHECK("hn_gemm_grouped");
  return 0;
}
