// Device-side pieces of the streaming decode kernels (hn_stream.hip): launch
// arguments, the weight-column loads, the biased-nibble unpack + MFMA chain,
// the activation staging with its bias corrections, and the column cursor.  The scheme
// (column decomposition, biased nibbles, corrections) is described at the
// top of hn_stream.hip.
#pragma once
#include "hn_common.h"

namespace {

constexpr int kTileN = 16;
constexpr uint32_t kOOB = 0x7ffffff0u;
constexpr int kMaxActive = 256;
constexpr int kMaxWaves = 8;  // per workgroup, one workgroup per CU: 2 per SIMD
constexpr int kMaxTc = 16;    // tokens per chunk (two MFMA rows each; 8 per MFMA)
constexpr int kCsw = 2 * kMaxTc;  // corrections per group pair: (token, parity)

struct SExpert {
  const uint8_t* gate_q; const h16* gate_s;
  const uint8_t* up_q;   const h16* up_s;
  const uint8_t* down_q; const h16* down_s;
};

struct StreamArgs {
  // single problem
  const h16* x; int ld_x; int M;
  const uint8_t* q[2];
  const h16* s[2];
  h16* out; int ld_o;
  int phase;  // grouped: 0 gate/up + SiLU (N = I, K = H); 1 down (N = H, K = I)
  int E;      // grouped: experts in the table
  // shape, shared by every problem of the launch
  int N, K;
  int ld_q;   // packed row stride (bytes)
  int ld_s;   // scale row stride (elements)
  int tc;     // tokens per chunk
  int ldx;    // LDS row stride of the staged activations (halves)
  int npair;  // group pairs per staged row (KW * LPW / 2)
  uint32_t m_lo, m_hi, magic;
  // K split (KS > 1, down phase only): K above is one slice; slice j of
  // row r goes to out32[j * ks_stride + r * N + n] in fp32
  float* out32;
  long ks_stride;
  // ROUTE (grouped gate/up only): the routing of hx computed in the kernel.
  // hx [T, H] fp16 hidden rows, gate [E, H] fp16 (or logits_in [T, E] fp32,
  // the router logits computed elsewhere); the permuted rows are staged from
  // hx directly; workgroup 0 writes the routing outputs.
  const h16* hx; int ld_hx;
  const h16* gate; int ld_gate;
  const float* logits_in;
  int T, topk;
  int mode;            // ROUTE 2: top-k mode (0 softmax, 1 sigmoid, 2 sigmoid unnormalised)
  const float* bias;   // ROUTE 2: optional selection bias [E]
  float eps, scaling;
  float* logits_out;
  int* idx_out; h16* w_out;
  int* offsets_out; int* perm_out; int* inv_out; int* active_out; int* n_active_out;
  long long* usage;  // optional [E]: += the routed rows per expert (workgroup 0)
};

// Weights and scales of one column for one wave.  Scales: with WIDE, dword
// pi holds the scales of groups (g0 + 2 pi, g0 + 2 pi + 1) of the lane's row
// (read as one vector per row); without, the lane's own scale per pair.
template <int MATS, int PAIRS, bool WIDE>
struct WBuf {
  u32x4 lo[MATS][PAIRS], hi[MATS][PAIRS];
  uint32_t slo[MATS][PAIRS], shi[MATS][PAIRS];
};

struct Problem {
  const h16* x;
  h16* out;
  int t0;    // first row of this problem in the launch
  int rows;  // tokens of this problem
  const uint8_t* q[2];
  const h16* s[2];
};

// Grouped-launch metadata: the active list, the row offsets and this
// phase's four weight pointers per expert, copied into LDS at the start in
// one round of independent loads (reading them on demand costs a chain of
// dependent memory round trips before the first weight load can go out).
struct Meta {
  const int* s_act;       // [E]
  const int* s_off;       // [E + 1]
  const uint64_t* s_ptr;  // [E][4]: q0, s0, q1, s1
};

__device__ __forceinline__ const void* rfl_ptr(uint64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const void*)(((uint64_t)hi << 32) | lo);
}

template <bool GROUPED>
__device__ __forceinline__ Problem resolve(const StreamArgs& A, const Meta& mt, int a) {
  Problem p;
  if (!GROUPED) {
    p.x = A.x;
    p.out = A.out;
    p.t0 = 0;
    p.rows = A.M;
    p.q[0] = A.q[0]; p.s[0] = A.s[0];
    p.q[1] = A.q[1]; p.s[1] = A.s[1];
  } else {
    const int e = __builtin_amdgcn_readfirstlane(mt.s_act[a]);
    const int t0 = __builtin_amdgcn_readfirstlane(mt.s_off[e]);
    p.t0 = t0;
    p.rows = __builtin_amdgcn_readfirstlane(mt.s_off[e + 1]) - t0;
    p.q[0] = (const uint8_t*)rfl_ptr(mt.s_ptr[4 * e + 0]);
    p.s[0] = (const h16*)rfl_ptr(mt.s_ptr[4 * e + 1]);
    p.q[1] = (const uint8_t*)rfl_ptr(mt.s_ptr[4 * e + 2]);
    p.s[1] = (const h16*)rfl_ptr(mt.s_ptr[4 * e + 3]);
    p.x = A.x + (long)t0 * A.ld_x;
    p.out = A.out + (long)t0 * A.ld_o;
  }
  return p;
}

// One column's loads for this wave: group pairs [g0, g0 + 2 * PAIRS) of tile
// `tile`.  Lane (col, q): lo = row n0 + col%8, hi = row n0 + 8 + col%8, 16
// bytes at chunk q of group g (col < 8) or g + 1 (col >= 8); the scale of
// that (row, group).  The whole offset is in voffset (+ the per-pair
// immediate): the buffer range check covers voffset + immediate only, not
// soffset, so soffset stays 0.  Rows past N and columns past the workgroup's
// range (valid == false) use an offset past the descriptor's range: those
// loads return 0 without touching memory.  Groups past K (the last wave of
// a K that is not a multiple of 2 * LPW * 128) read the next row or nothing;
// they meet zero activations and their products are skipped.
// WIDE scales: one load per (matrix, row) of the wave's LPW scales (LPW * 2
// bytes: b32 / b64 / b128 / 2 x b128), instead of one 2-byte load per lane
// and pair (which costs as much address work as a 1 KiB weight load).  The
// host selects it when the wave's groups lie inside the row (K / 128 = KW *
// LPW) and scale rows and pointers are 16-byte aligned.
template <int MATS, int PAIRS, bool WIDE>
__device__ __forceinline__ void issue(WBuf<MATS, PAIRS, WIDE>& b, const Problem& pr,
                                      const StreamArgs& A, int tile, int g0, bool valid,
                                      int col, int q) {
  const int N = A.N, ldq = A.ld_q, lds2 = 2 * A.ld_s;
  const int rlo = tile * kTileN + (col & 7), rhi = rlo + 8;
  const int odd = col >= 8 ? 1 : 0;
  const int ch = q + 4 * odd;
  const bool vl = valid && rlo < N, vh = valid && rhi < N;
  const uint32_t vlo = vl ? (uint32_t)(rlo * ldq + 64 * g0 + 16 * ch) : kOOB;
  const uint32_t vhi = vh ? (uint32_t)(rhi * ldq + 64 * g0 + 16 * ch) : kOOB;
  const int gs = WIDE ? g0 : g0 + odd;
  const uint32_t vslo = vl ? (uint32_t)(rlo * lds2 + 2 * gs) : kOOB;
  const uint32_t vshi = vh ? (uint32_t)(rhi * lds2 + 2 * gs) : kOOB;
  __amdgpu_buffer_rsrc_t rq[MATS], rs[MATS];
#pragma unroll
  for (int mt = 0; mt < MATS; ++mt) {
    rq[mt] = __builtin_amdgcn_make_buffer_rsrc((void*)pr.q[mt], (short)0, N * ldq, 0x00020000);
    rs[mt] = __builtin_amdgcn_make_buffer_rsrc((void*)pr.s[mt], (short)0, N * lds2, 0x00020000);
  }
  if constexpr (WIDE) {
#pragma unroll
    for (int mt = 0; mt < MATS; ++mt) {
      // lo rows' scales, then hi rows' (stored by name: no pointer into the
      // buffer, which keeps every element a plain register)
      if constexpr (PAIRS == 1) {
        b.slo[mt][0] = __builtin_amdgcn_raw_buffer_load_b32(rs[mt], vslo, 0, 0);
        b.shi[mt][0] = __builtin_amdgcn_raw_buffer_load_b32(rs[mt], vshi, 0, 0);
      } else if constexpr (PAIRS == 2) {
        const auto vl = __builtin_amdgcn_raw_buffer_load_b64(rs[mt], vslo, 0, 0);
        const auto vh = __builtin_amdgcn_raw_buffer_load_b64(rs[mt], vshi, 0, 0);
        b.slo[mt][0] = vl[0];
        b.slo[mt][1] = vl[1];
        b.shi[mt][0] = vh[0];
        b.shi[mt][1] = vh[1];
      } else {
#pragma unroll
        for (int j = 0; j < PAIRS / 4; ++j) {
          const u32x4 vl = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs[mt], vslo + 16 * j, 0, 0));
          const u32x4 vh = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs[mt], vshi + 16 * j, 0, 0));
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            b.slo[mt][4 * j + e] = vl[e];
            b.shi[mt][4 * j + e] = vh[e];
          }
        }
      }
    }
#pragma unroll
    for (int pi = 0; pi < PAIRS; ++pi) {
#pragma unroll
      for (int mt = 0; mt < MATS; ++mt) {
        b.lo[mt][pi] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq[mt], vlo + 128 * pi, 0, 2));
        b.hi[mt][pi] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq[mt], vhi + 128 * pi, 0, 2));
      }
    }
  } else {
    // issue order = use order (pair, matrix, lo/hi)
#pragma unroll
    for (int pi = 0; pi < PAIRS; ++pi) {
#pragma unroll
      for (int mt = 0; mt < MATS; ++mt) {
        b.lo[mt][pi] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq[mt], vlo + 128 * pi, 0, 2));
        b.slo[mt][pi] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs[mt], vslo + 4 * pi, 0, 0);
        b.hi[mt][pi] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq[mt], vhi + 128 * pi, 0, 2));
        b.shi[mt][pi] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs[mt], vshi + 4 * pi, 0, 0);
      }
    }
  }
}

// Biased unpack of one packed dword: (1024 + n) for even k, (1024 + 16 n)
// for odd k, in the order (k0,k4, k1,k5, k2,k6, k3,k7).
__device__ __forceinline__ half8_t unpack_biased(uint32_t w, const HnUnpackRegs& c) {
  const uint32_t w8 = w >> 8;
  const u32x4 r = {hn_and_or(w, c.m_lo, c.magic), hn_and_or(w, c.m_hi, c.magic),
                   hn_and_or(w8, c.m_lo, c.magic), hn_and_or(w8, c.m_hi, c.magic)};
  return __builtin_bit_cast(half8_t, r);
}

// Unpack + MFMA of one column for this wave.  acc_lo / acc_hi[h]: D rows
// 4q + r (token 8h + 2q + r/2, group parity r%2) of the lo / hi chains; TH
// token halves of 8 share each unpacked weight operand.
// FULL: every pair of the wave lies inside K (the common case): no per-pair
// guard, so the pairs' loads from LDS and MFMA chains form one basic block
// that the scheduler can interleave.  The arithmetic is the same either way.
template <int MATS, int PAIRS, bool WIDE, bool FULL, int TH>
__device__ __forceinline__ void compute_pairs(const WBuf<MATS, PAIRS, WIDE>& b, const h16* xs,
                                              const float* cs, int ldx, int pb0, int gw,
                                              const int (&arow_i)[TH], int q, int sshift,
                                              const HnUnpackRegs& ur, float4_t (&acc_lo)[TH][MATS],
                                              float4_t (&acc_hi)[TH][MATS]) {
#pragma unroll
  for (int h = 0; h < TH; ++h)
#pragma unroll
    for (int mt = 0; mt < MATS; ++mt) {
      acc_lo[h][mt] = float4_t{0.f, 0.f, 0.f, 0.f};
      acc_hi[h][mt] = float4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
  for (int pi = 0; pi < PAIRS; ++pi) {
    if (FULL || 2 * pi < gw) {  // uniform
      half8_t a[TH][4];
      float4_t negc[TH];
#pragma unroll
      for (int h = 0; h < TH; ++h) {
        const h16* arow = xs + arow_i[h] * ldx + (pb0 + pi) * 128 + 32 * q;
#pragma unroll
        for (int t = 0; t < 4; ++t) a[h][t] = *reinterpret_cast<const half8_t*>(arow + 8 * t);
        negc[h] = *reinterpret_cast<const float4_t*>(cs + (pb0 + pi) * kCsw + 16 * h + 4 * q);
      }
#pragma unroll
      for (int mt = 0; mt < MATS; ++mt) {
        // WIDE: the lane's group parity picks the half of the pair's dword
        const int sft = WIDE ? sshift : 0;
        if constexpr (TH == 1) {
          float4_t cl = negc[0], ch = negc[0];
#pragma unroll
          for (int t = 0; t < 4; ++t)
            cl = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[0][t], unpack_biased(b.lo[mt][pi][t], ur),
                                                        cl, 0, 0, 0);
#pragma unroll
          for (int t = 0; t < 4; ++t)
            ch = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[0][t], unpack_biased(b.hi[mt][pi][t], ur),
                                                        ch, 0, 0, 0);
          const float sl = (float)__builtin_bit_cast(h16, (uint16_t)(b.slo[mt][pi] >> sft));
          const float sh = (float)__builtin_bit_cast(h16, (uint16_t)(b.shi[mt][pi] >> sft));
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            acc_lo[0][mt][r] = __builtin_fmaf(sl, cl[r], acc_lo[0][mt][r]);
            acc_hi[0][mt][r] = __builtin_fmaf(sh, ch[r], acc_hi[0][mt][r]);
          }
        } else {
          const float sl = (float)__builtin_bit_cast(h16, (uint16_t)(b.slo[mt][pi] >> sft));
          const float sh = (float)__builtin_bit_cast(h16, (uint16_t)(b.shi[mt][pi] >> sft));
          half8_t wl[4], wh[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            wl[t] = unpack_biased(b.lo[mt][pi][t], ur);
            wh[t] = unpack_biased(b.hi[mt][pi][t], ur);
          }
#pragma unroll
          for (int h = 0; h < TH; ++h) {
            float4_t cl = negc[h], ch = negc[h];
#pragma unroll
            for (int t = 0; t < 4; ++t)
              cl = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[h][t], wl[t], cl, 0, 0, 0);
#pragma unroll
            for (int t = 0; t < 4; ++t)
              ch = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[h][t], wh[t], ch, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              acc_lo[h][mt][r] = __builtin_fmaf(sl, cl[r], acc_lo[h][mt][r]);
              acc_hi[h][mt][r] = __builtin_fmaf(sh, ch[r], acc_hi[h][mt][r]);
            }
          }
        }
      }
    }
  }
}

template <int MATS, int PAIRS, bool WIDE, int TH>
__device__ __forceinline__ void compute(const WBuf<MATS, PAIRS, WIDE>& b, const h16* xs,
                                        const float* cs, int ldx, int pb0, int gw,
                                        const int (&arow_i)[TH], int q, int sshift,
                                        const HnUnpackRegs& ur, float4_t (&acc_lo)[TH][MATS],
                                        float4_t (&acc_hi)[TH][MATS]) {
  if (gw >= 2 * PAIRS)  // uniform
    compute_pairs<MATS, PAIRS, WIDE, true, TH>(b, xs, cs, ldx, pb0, gw, arow_i, q, sshift, ur,
                                               acc_lo, acc_hi);
  else
    compute_pairs<MATS, PAIRS, WIDE, false, TH>(b, xs, cs, ldx, pb0, gw, arow_i, q, sshift, ur,
                                                acc_lo, acc_hi);
}

__device__ __forceinline__ float xor8(float v) {  // lane col ^ 8 of the same 16-lane row
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false));
}

// Activation staging.  Token t, group g goes to LDS row 2t + (g & 1), columns
// (g >> 1) * 128 + k % 128, in unpack order with odd k scaled by 1/16; groups
// past K are zero.  Out-of-range threads repeat the last block (same value to
// the same address), so loads and stores are branch-free.
struct StageGeom {
  int m0, Mc, blk_per_tok, nblk;
};

// ROUTE: rperm (LDS) maps a permuted row to its assignment (token * topk +
// slot), and the row is read from hx.  t0: the problem's first permuted row.
template <bool ROUTE = false>
__device__ __forceinline__ void stage_load(const StreamArgs& A, const h16* x,
                                           const StageGeom& sg, int base, half8_t v[4],
                                           const int* rperm = nullptr, int t0 = 0) {
  const int tid = threadIdx.x, nthr = blockDim.x, K = A.K;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = min(base + tid + j * nthr, sg.nblk - 1);
    const int t = i / sg.blk_per_tok;
    const int k = min((i - t * sg.blk_per_tok) * 8, K - 8);
    const h16* row = ROUTE ? A.hx + (long)(rperm[t0 + sg.m0 + t] / A.topk) * A.ld_hx
                           : x + (long)(sg.m0 + t) * A.ld_x;
    v[j] = *reinterpret_cast<const half8_t*>(row + k);
  }
}

// Also the bias corrections: the 16 blocks of one (token, group) sit in 16
// consecutive lanes (block index = base + tid + j * nthr, blk_per_tok a
// multiple of 16), so each lane's 8-term dot product is summed across its
// 16-lane DPP row and the row's first lane writes cs[pair * kCsw + 2 t +
// parity] = -C.  Lanes whose block is a repeat of the last one (past the chunk) skip
// the write; so does the whole row, as the chunk ends on a group boundary.
__device__ __forceinline__ void stage_store(const StreamArgs& A, const StageGeom& sg, int base,
                                            const half8_t v[4], h16* xs, float* cs) {
  const int tid = threadIdx.x, nthr = blockDim.x, K = A.K;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int ir = base + tid + j * nthr;
    const int i = min(ir, sg.nblk - 1);
    const int t = i / sg.blk_per_tok;
    const int b = i - t * sg.blk_per_tok;
    const int g = b >> 4;
    const bool in_k = b * 8 < K;
    half8_t p;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const h16 s = v[j][hn_perm8(e)];
      p[e] = in_k ? ((e & 2) ? s * (h16)0.0625f : s) : (h16)0.0f;
    }
    *reinterpret_cast<half8_t*>(xs + (2 * t + (g & 1)) * A.ldx + (g >> 1) * 128 + (b & 15) * 8) = p;
    // correction: sum over k of x * bias, bias 1032 (even k) / 1152 (odd k, x / 16 stored).
    // (fp32 fma per term: v_dot2c_f32_f16 with these operands was miscompiled here,
    // every dot product reading the first dword)
    float c = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) c = __builtin_fmaf((float)p[e], (e & 2) ? 1152.f : 1032.f, c);
    c += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, c), 0x128, 0xf, 0xf, false));
    c += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, c), 0x124, 0xf, 0xf, false));
    c += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, c), 0x122, 0xf, 0xf, false));
    c += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, c), 0x121, 0xf, 0xf, false));
    if ((tid & 15) == 0 && ir < sg.nblk) cs[(g >> 1) * kCsw + 2 * t + (g & 1)] = -c;
  }
}

// Corrections of MFMA rows past the chunk's tokens are zero (their outputs
// are never stored; the rows read a clamped token).
__device__ __forceinline__ void stage_zero_rows(const StreamArgs& A, int Mc, float* cs) {
  for (int i = threadIdx.x; i < A.npair * kCsw; i += blockDim.x)
    if (((i % kCsw) >> 1) >= Mc) cs[i] = 0.f;
}

// Whole staging of one chunk (used when the staged chunk changes mid-stream).
template <bool ROUTE = false>
__device__ __forceinline__ void stage(const StreamArgs& A, const h16* x, const StageGeom& sg,
                                      h16* xs, float* cs, const int* rperm = nullptr,
                                      int t0 = 0) {
  const int nthr = blockDim.x;
  __syncthreads();  // the previous chunk is no longer read
  stage_zero_rows(A, sg.Mc, cs);
  for (int base = 0; base < sg.nblk; base += 4 * nthr) {
    half8_t v[4];
    stage_load<ROUTE>(A, x, sg, base, v, rperm, t0);
    stage_store(A, sg, base, v, xs, cs);
  }
  __syncthreads();
}

// Column cursor: column -> (problem, chunk, tile).  Columns only move
// forward; the current problem's chunk range [lo, hi) sits in scalar registers.
struct Cursor {
  int a, lo, hi;
};

__device__ __forceinline__ void locate(Cursor& cu, const int* chunk_off, int nprob, int tiles,
                                       int c, int& prob, int& chunk, int& tile) {
  const int gc = c / tiles;
  tile = c - gc * tiles;
  while (gc >= cu.hi && cu.a + 1 < nprob) {
    ++cu.a;
    cu.lo = cu.hi;
    cu.hi = __builtin_amdgcn_readfirstlane(chunk_off[cu.a + 1]);
  }
  prob = cu.a;
  chunk = gc - cu.lo;
}

}  // namespace
