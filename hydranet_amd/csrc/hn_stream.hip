// Persistent streaming W4A16 kernels for decode, gfx950.
//
//   out[m, n] = sum_k x[m, k] * W[n, k],  W[n, k] = (nibble - 8) * scale[n, k / 128]
//
// Replaces, for up to 8 tokens per weight matrix and group size 128, the
// per-expert Triton int4_matmul_kernel launches (kernels/int4_gemm.py:25-121)
// and their SwiGLU epilogue (kernels/int4_gemm.py:175-193), one launch per
// projection over every active expert of a layer.
//
// Work decomposition
//  * A "column" is (problem, token chunk, 16-row tile).  A problem is one
//    weight matrix (or the gate/up pair) with its tokens: one expert in a
//    grouped MoE launch.  The grid is one workgroup per CU; each walks a
//    contiguous range of columns, so the active-expert count is read on the
//    device and the work is balanced over the CUs.
//  * The KW <= 8 waves of a workgroup split K (LPW groups of 128 k each).  A
//    wave keeps NBUF register buffers of weights and issues the loads of
//    column c + NBUF - 1 before it unpacks column c.
//  * Weight loads: 8 rows x 128 B per instruction (full cache lines,
//    non-temporal), "lo" = tile rows 0-7, "hi" = rows 8-15, each over a group
//    pair (g, g+1): lanes with MFMA column < 8 receive group g of row col % 8,
//    lanes >= 8 group g+1 of the same row.
//  * The MFMA A operand has two rows per token: row 2t + p holds token t's
//    activations of group g + p.  One MFMA chain over a lo (hi) load thus
//    yields group g of rows 0-7 (8-15) in its even D rows and group g + 1 in
//    its odd D rows; a single lane exchange per column (DPP row_ror:8) adds
//    the two.  Up to 8 tokens per chunk.
//
// Arithmetic (biased nibbles)
//  * A packed dword w holds k0..k7 (k0 in bits 0-3).  (w & 0x000F000F) |
//    0x64006400 is the fp16 pair (1024 + n_k0, 1024 + n_k4); with mask
//    0x00F000F0 it is (1024 + 16 n_k1, 1024 + 16 n_k5); w >> 8 gives k2,k6 and
//    k3,k7 the same way.  Five VALU operations per dword; the fp16 values are
//    exact.  Output order k = (0,4,1,5,2,6,3,7) (hn_perm8).
//  * The activations are staged in that order with the odd k (high nibbles)
//    multiplied by 1/16 (exact for normal fp16), so every product in the
//    MFMA is x * (n + bias): bias 1024 for even k, 64 for odd k.  The exact
//    correction C(t, g) = sum_even 1032 x + sum_odd 1152 x/16 over the group
//    is computed once per staged chunk in fp32; the MFMA chain starts from
//    -C, so after it the accumulator holds sum_k x (n - 8) for that group.
//  * The group scale multiplies that fp32 partial (v_fma_mix_f32, the scale
//    read as fp16).  Products in the chain are exact; the fp32 sums carry
//    magnitudes ~1024 |x|, i.e. a relative error ~1e-5 of the result, well
//    inside the fp16 output rounding.
#include "hn_stream_dev.h"

#include "hn_topk.h"

namespace {
// Decode routing in the gate/up kernel's prologue (ROUTE): Mixtral softmax
// top-k (k = 1 or 2) of E <= 8 experts over T tokens, T k <= 64.  The
// arithmetic is moe_route_kernel's (hn_route.hip): logits (T <= 16, fp16
// gate) by MFMA over 16 slices of H, the slice partials summed in slice order
// and rounded to fp16 (the fp16 Linear of TopKRouter, model/router.py:102),
// or read from logits_in; top-k and weights by topk_small; the stable order
// by expert from ballots (torch.where order, model/mixtral.py:333).  Every
// workgroup computes it into LDS (part: 16 KiB scratch, reused by the
// staging afterwards); workgroup 0 also writes the routing outputs.
// Returns the number of active experts (uniform).
__device__ int route_prologue(const StreamArgs& A, float* part, int* s_act, int* s_off,
                              int* rperm, int wave, int lane) {
  const int tid = threadIdx.x, KW = blockDim.x >> 6;
  const int T = A.T, E = A.E, H = A.K, k = A.topk, n = T * k;
  const bool lead = blockIdx.x == 0;
  float* s_lg = part + 16 * 16 * 16;           // [T * E] <= 512
  int* s_sel = reinterpret_cast<int*>(s_lg + 512);
  h16* s_w = reinterpret_cast<h16*>(s_sel + 64);
  int* s_na = reinterpret_cast<int*>(s_w + 64);
  // 1. logits: given, or slice sl of H/16 by wave sl % KW; lane (expert tl,
  //    tokens 4 (lane >> 4) + r)
  if (A.logits_in) {
    for (int i = tid; i < T * E; i += blockDim.x) s_lg[i] = A.logits_in[i];
  } else {
    const int ksl = H >> 4, steps = ksl >> 5;
    const int tl = lane & 15, kq = (lane >> 4) * 8;
    // lanes past the T tokens / E experts load nothing (their products are
    // never read): their MFMA operand is zero (C2 T = 16: a quarter of the
    // prologue's loads, the routed kernel 99 -> 96 us)
    const bool a_on = tl < T, b_on = tl < E;
    const h16* ap = A.hx + (long)min(tl, T - 1) * A.ld_hx + kq;
    const h16* bp = A.gate + (long)min(tl, E - 1) * A.ld_gate + kq;
    const half8_t z8 = {};
    // two slices per pass (sl0, sl0 + KW); each pass loads up to 8 steps of
    // both slices into registers before the MFMAs (steps past the slice
    // repeat the last one and are not multiplied), so the loads are in flight
    // together instead of one round trip per step
    constexpr int kSt = 8;
    for (int sl0 = wave; sl0 < 16; sl0 += 2 * KW) {
      const int sl1 = sl0 + KW;
      const bool has1 = sl1 < 16;  // uniform
      const int kb0 = sl0 * ksl, kb1 = (has1 ? sl1 : sl0) * ksl;
      float4_t acc0 = float4_t{0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
      for (int s0 = 0; s0 < steps; s0 += kSt) {
        half8_t a0[kSt], b0[kSt], a1[kSt], b1[kSt];
#pragma unroll
        for (int u = 0; u < kSt; ++u) {
          const int st = min(s0 + u, steps - 1);
          b0[u] = b_on ? *reinterpret_cast<const half8_t*>(bp + kb0 + 32 * st) : z8;
          a0[u] = a_on ? *reinterpret_cast<const half8_t*>(ap + kb0 + 32 * st) : z8;
          b1[u] = b_on ? *reinterpret_cast<const half8_t*>(bp + kb1 + 32 * st) : z8;
          a1[u] = a_on ? *reinterpret_cast<const half8_t*>(ap + kb1 + 32 * st) : z8;
        }
#pragma unroll
        for (int u = 0; u < kSt; ++u) {
          if (s0 + u < steps) {  // uniform
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0[u], b0[u], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1[u], b1[u], acc1, 0, 0, 0);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        part[(sl0 * 16 + 4 * (lane >> 4) + r) * 16 + tl] = acc0[r];
        if (has1) part[(sl1 * 16 + 4 * (lane >> 4) + r) * 16 + tl] = acc1[r];
      }
    }
    __syncthreads();
    for (int i = tid; i < T * E; i += blockDim.x) {
      const int t = i / E, e = i - t * E;
      float v = 0.f;
#pragma unroll
      for (int sl = 0; sl < 16; ++sl) v += part[(sl * 16 + t) * 16 + e];
      s_lg[i] = (float)(h16)v;
    }
  }
  __syncthreads();
  if (lead && A.logits_out)
    for (int i = tid; i < T * E; i += blockDim.x) A.logits_out[i] = s_lg[i];
  // 2. top-k and weights, one thread per token
  for (int t = tid; t < T; t += blockDim.x) {
    if (k == 2)
      topk_small<8, 2, 0>(s_lg + t * E, nullptr, E, 2, 0, A.eps, A.scaling, s_sel + t * 2,
                          s_w + t * 2);
    else
      topk_small<8, 1, 0>(s_lg + t * E, nullptr, E, 1, 0, A.eps, A.scaling, s_sel + t, s_w + t);
  }
  __syncthreads();
  // 3. stable order by expert (n <= 64: wave 0, one lane per assignment).
  //    Rank among equal experts from ballots over the bits of e (E <= 8:
  //    bits 0-2, and bit 3 set only for the -1 of no expert); the counts,
  //    offsets and the active list are wave-uniform scalar sums over the
  //    experts in order.
  if (wave == 0) {
    const int j = lane;
    int e = j < n ? s_sel[j] : -1;
    if (e < 0 || e >= E) e = -1;
    uint64_t same = ~0ull;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint64_t bal = __ballot((e >> b) & 1);
      same &= ((e >> b) & 1) ? bal : ~bal;
    }
    const int rank = __popcll(same & ((1ull << lane) - 1));
    int run = 0, nact = 0, off_e = 0;
    for (int x = 0; x < E; ++x) {  // uniform
      const int c = __popcll(__ballot(e == x));
      if (e == x) off_e = run;
      if (lane == 0) {
        s_off[x] = run;
        if (c > 0) s_act[nact] = x;
        if (lead) {
          A.offsets_out[x] = run;
          if (c > 0) A.active_out[nact] = x;
          if (A.usage && c > 0) A.usage[x] += c;
        }
      }
      nact += c > 0 ? 1 : 0;
      run += c;
    }
    if (lane == 0) {
      s_off[E] = run;
      *s_na = nact;
      if (lead) {
        A.offsets_out[E] = run;
        *A.n_active_out = nact;
      }
    }
    const int pos = off_e + rank;
    if (e >= 0) rperm[pos] = j;
    if (lead && j < n) {
      A.idx_out[j] = s_sel[j];
      A.w_out[j] = s_w[j];
      A.inv_out[j] = e >= 0 ? pos : -1;
      if (e >= 0) A.perm_out[pos] = j;
    }
  }
  __syncthreads();
  return __builtin_amdgcn_readfirstlane(*s_na);
}

// Decode routing from given logits in the gate/up kernel's prologue (ROUTE
// 2): any of the top-k modes (Mixtral softmax, GLM sigmoid with an optional
// selection bias, with or without the normalisation) over E <= 256 experts,
// T k <= the workgroup's threads.  The arithmetic is moe_route_kernel's
// (hn_route.hip) from given logits: the top-k of a token by one wave
// (topk_wave), the stable order by expert from nine ballots over the expert
// bits per wave and the per-wave counts, the offsets and the active list by
// wave scans.  Every workgroup computes it into LDS (scratch: the logits, the
// selection and the per-wave counts, in the staging area used afterwards);
// workgroup 0 also writes the routing outputs.  Returns the number of
// active experts (uniform).
__device__ int route_prologue_sel(const StreamArgs& A, unsigned char* scratch, int* s_act,
                                  int* s_off, int* rperm, int wave, int lane) {
  const int tid = threadIdx.x, KW = blockDim.x >> 6;
  const int T = A.T, E = A.E, k = A.topk, n = T * k;
  const bool lead = blockIdx.x == 0;
  float* s_lg = reinterpret_cast<float*>(scratch);          // [T * E]
  int* s_sel = reinterpret_cast<int*>(s_lg + T * E);        // [n]
  h16* s_w = reinterpret_cast<h16*>(s_sel + n);             // [n]
  int* s_wcnt = reinterpret_cast<int*>(s_w + ((n + 1) & ~1));  // [KW][E]
  int* s_na = s_wcnt + KW * E;
  // the selection bias goes out with the logits (once per wave)
  const TopkBias tb = topk_wave_bias(A.bias, E, lane);
  for (int i = tid; i < KW * E; i += blockDim.x) s_wcnt[i] = 0;
  copy_to_lds_f32(A.logits_in, s_lg, T * E);
  __syncthreads();
  // 1. top-k, one wave per token
  for (int t = wave; t < T; t += KW)
    topk_wave(s_lg + t * E, tb, E, k, A.mode, A.eps, A.scaling, lane, s_sel + t * k,
              s_w + t * k);
  __syncthreads();
  // 2. rank among equal experts within the wave (one thread per assignment)
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
  if (e >= 0 && rank == 0) s_wcnt[wave * E + e] = __popcll(same);
  __syncthreads();
  // 3. counts, offsets and the active list: 4 experts per lane, wave scans
  if (wave == 0) {
    int c[4], f[4], cs = 0, fs = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int ex = 4 * lane + q;
      c[q] = 0;
      if (ex < E)
        for (int w2 = 0; w2 < KW; ++w2) c[q] += s_wcnt[w2 * E + ex];
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
        if (f[q]) s_act[fo] = ex;
        if (lead) {
          A.offsets_out[ex] = co;
          if (f[q]) A.active_out[fo] = ex;
          if (A.usage && c[q]) A.usage[ex] += c[q];
        }
      }
      co += c[q];
      fo += f[q];
    }
    if (lane == 63) {
      s_off[E] = ci;
      *s_na = fi;
      if (lead) {
        A.offsets_out[E] = ci;
        *A.n_active_out = fi;
      }
    }
  }
  __syncthreads();
  // 4. the permutation
  if (j < n) {
    if (lead) {
      A.idx_out[j] = s_sel[j];
      A.w_out[j] = s_w[j];
    }
    if (e >= 0) {
      int pos = s_off[e] + rank;
      for (int w2 = 0; w2 < wave; ++w2) pos += s_wcnt[w2 * E + e];
      rperm[pos] = j;
      if (lead) {
        A.perm_out[pos] = j;
        A.inv_out[j] = pos;
      }
    } else if (lead) {
      A.inv_out[j] = -1;
    }
  }
  __syncthreads();
  return __builtin_amdgcn_readfirstlane(*s_na);
}

// At most 8 waves per workgroup and one workgroup per CU: 2 waves per SIMD,
// 256 VGPRs each.
// KS > 1: the columns of a chunk are (k slice, tile), the slices one after
// the other, so that a workgroup's contiguous range mostly stays on one
// slice (one staging); each column's wave-reduced partial is written in fp32
// and the caller sums the KS slices in order.  A slice keeps the workgroup's
// activations and the pipeline short where K is long (the down projection).
// Waves per SIMD the register budget must allow: single-matrix launches of
// 8-token chunks and four groups per wave run two 7- or 8-wave workgroups
// per CU (four waves per SIMD, so at most 128 VGPRs); the others one
// workgroup (their plans may still ask for two; launch_one then checks what
// the registers allow).
template <int MATS, int TH, int LPW>
constexpr int stream_waves_per_eu() { return MATS == 1 && TH == 1 && LPW <= 4 ? 4 : 1; }

template <bool GROUPED, int MATS, int EPI, int LPW, int NBUF, bool WIDE, int KS,
          int ROUTE = 0, int TH = 1>
__global__ __launch_bounds__(512)
__attribute__((amdgpu_waves_per_eu(stream_waves_per_eu<MATS, TH, LPW>()))) void stream_kernel(
    StreamArgs A,
                                                     const SExpert* __restrict__ table,
                                                     const int* __restrict__ active,
                                                     const int* __restrict__ n_active,
                                                     const int* __restrict__ offsets) {
  constexpr int PAIRS = LPW / 2;
  static_assert(NBUF == 2 || NBUF == 3, "two or three column buffers");
  static_assert(TH == 1 || TH == 2, "8 or 16 tokens per chunk");
  // reduction buffers: parity-double-buffered (one barrier per column) unless
  // that no longer fits beside 16 tokens of gate/up activations; then one
  // buffer and a second barrier per column
  constexpr int NRB = (TH == 2 && MATS == 2) ? 1 : 2;
  extern __shared__ __align__(16) unsigned char smem[];
  Meta meta = {nullptr, nullptr, nullptr};
  __shared__ int chunk_off[kMaxActive + 1];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int KW = blockDim.x >> 6;
  const int col = lane & 15;
  const int q = lane >> 4;
  const int N = A.N, TC = A.tc;
  const int G = A.K >> 7;
  const int tiles_n = (N + kTileN - 1) / kTileN;
  const int tiles = tiles_n * KS;              // columns per chunk
  const int g0 = wave * LPW;                   // this wave's first group
  const int gw = max(0, min(LPW, G - g0));     // its groups (uniform)
  const int pb0 = g0 >> 1;                     // its first group pair
  h16* xs = reinterpret_cast<h16*>(smem);
  float* cs = reinterpret_cast<float*>(smem + (size_t)TC * 2 * A.ldx * 2);
  float2* red = reinterpret_cast<float2*>(cs + A.npair * kCsw);
  // reduction slots per buffer: waves 1.. (TH 1: wave 0 reduces) or every
  // wave (TH 2: wave h reduces token half h)
  constexpr int kRedWaves = TH == 1 ? kMaxWaves - 1 : kMaxWaves;
  constexpr int kRedSlots = kRedWaves * TH * MATS * 64;
  HnUnpackRegs ur;
  ur.m_lo = A.m_lo;
  ur.m_hi = A.m_hi;
  ur.magic = hn_vgpr(A.magic);

  // ---- token chunks per problem -> prefix (chunk_off); columns = chunks * tiles
  int nprob = 1;
  int* rperm = nullptr;  // ROUTE: permuted row -> assignment
  if (GROUPED) {
    // one round of independent loads: active list, offsets, weight pointers
    // (ROUTE: the pointers only; the active list and offsets are computed)
    const int E = A.E;
    int* s_act = reinterpret_cast<int*>(red + NRB * kRedSlots);
    int* s_off = s_act + ((E + 1) & ~1);
    uint64_t* s_ptr = reinterpret_cast<uint64_t*>(s_off + ((E + 2) & ~1));
    const uint64_t* tw = reinterpret_cast<const uint64_t*>(table);
    int na;
    if constexpr (ROUTE == 1) {
      // pointers requested first, stored once the routing is done (4 E <= 32 threads)
      const uint64_t pv = tid < 4 * E ? tw[6 * (tid >> 2) + (tid & 3)] : 0;
      rperm = reinterpret_cast<int*>(s_ptr + 4 * E);
      na = route_prologue(A, reinterpret_cast<float*>(smem), s_act, s_off, rperm, wave, lane);
      if (tid < 4 * E) s_ptr[tid] = pv;
    } else if constexpr (ROUTE == 2) {
      // the weight pointers requested first, stored after the routing
      uint64_t pv[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int i = tid + u * (int)blockDim.x;
        pv[u] = i < 4 * E ? tw[6 * (i >> 2) + (i & 3)] : 0;
      }
      rperm = reinterpret_cast<int*>(s_ptr + 4 * E);
      na = route_prologue_sel(A, smem, s_act, s_off, rperm, wave, lane);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int i = tid + u * (int)blockDim.x;
        if (i < 4 * E) s_ptr[i] = pv[u];
      }
      for (int i = tid + 2 * (int)blockDim.x; i < 4 * E; i += blockDim.x)
        s_ptr[i] = tw[6 * (i >> 2) + (i & 3)];
    } else {
      na = *n_active;
      for (int i = tid; i < E; i += blockDim.x) s_act[i] = active[i];
      for (int i = tid; i <= E; i += blockDim.x) s_off[i] = offsets[i];
      for (int i = tid; i < 4 * E; i += blockDim.x) {
        const int e = i >> 2, j = i & 3;
        const int f = A.phase == 0 ? j : 4 + (j & 1);  // gate_q gate_s up_q up_s | down_q down_s
        s_ptr[i] = tw[6 * e + f];
      }
    }
    meta = {s_act, s_off, s_ptr};
    nprob = min(na, min(E, kMaxActive));
    __syncthreads();
    for (int i = tid; i < nprob; i += blockDim.x) {
      const int e = s_act[i];
      chunk_off[i + 1] = (s_off[e + 1] - s_off[e] + TC - 1) / TC;
    }
    __syncthreads();
    if (tid < 64) {  // prefix over <= 256 entries: 4 per lane, then a wave scan
      int v[4], sum = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = 4 * tid + j;
        v[j] = i < nprob ? chunk_off[i + 1] : 0;
        sum += v[j];
      }
      int incl = sum;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int o = __shfl_up(incl, off, 64);
        if (tid >= off) incl += o;
      }
      int run = incl - sum;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = 4 * tid + j;
        run += v[j];
        if (i < nprob) chunk_off[i + 1] = run;
      }
      if (tid == 0) chunk_off[0] = 0;
    }
  } else if (tid == 0) {
    chunk_off[0] = 0;
    chunk_off[1] = (A.M + TC - 1) / TC;
  }
  // reduction slots of waves this workgroup does not have stay zero
  for (int i = tid; i < NRB * kRedSlots; i += blockDim.x) {
    const int slot = (i / (TH * MATS * 64)) % kRedWaves;
    if (slot >= KW - (TH == 1 ? 1 : 0)) red[i] = float2{0.f, 0.f};
  }
  __syncthreads();
  if (nprob <= 0) return;
  const int C = __builtin_amdgcn_readfirstlane(chunk_off[nprob]) * tiles;
  const int cb = (int)((long)C * blockIdx.x / gridDim.x);
  const int ce = (int)((long)C * (blockIdx.x + 1) / gridDim.x);
  if (cb >= ce) return;  // uniform over the workgroup

  const int off1 = __builtin_amdgcn_readfirstlane(chunk_off[1]);
  Cursor cu_i = {0, 0, off1}, cu_c = {0, 0, off1};
  int pi_last;        // problem of the last issued column
  Problem pi_pr;      // its weights
  int st_p, st_ch;    // staged (problem, chunk)
  int st_kj = 0;      // and k slice
  Problem st_pr;      // its activations / output
  StageGeom sg;
  int ci = cb;        // next column to issue
  int parity = 0;
  const int blk_per_tok = A.npair * 2 * 16;

  auto issue_next = [&](WBuf<MATS, PAIRS, WIDE>& b) {
    const bool more = ci < ce;
    int p = 0, ch = 0, t = 0;
    if (more) {
      locate(cu_i, chunk_off, nprob, tiles, ci, p, ch, t);
      if (p != pi_last) {
        pi_pr = resolve<GROUPED>(A, meta, p);
        pi_last = p;
      }
    }
    const int kj = KS > 1 ? t / tiles_n : 0;
    issue<MATS, PAIRS, WIDE>(b, pi_pr, A, t - kj * tiles_n, g0 + kj * G, more, col, q);
    ++ci;
  };
  auto geom = [&](int ch) {
    StageGeom g;
    g.m0 = ch * TC;
    g.Mc = min(TC, st_pr.rows - g.m0);
    g.blk_per_tok = blk_per_tok;
    g.nblk = g.Mc * blk_per_tok;
    return g;
  };

  WBuf<MATS, PAIRS, WIDE> b0, b1, b2;
  // ---- prologue: the first chunk's activations (up to two rounds of loads)
  //      are requested before the first columns' weights and waited for
  //      alone (loads complete in issue order: a round issued after the
  //      weights would wait for them)
  {
    int p, ch, t;
    locate(cu_c, chunk_off, nprob, tiles, cb, p, ch, t);
    st_p = p;
    st_ch = ch;
    if constexpr (KS > 1) st_kj = t / tiles_n;
    st_pr = resolve<GROUPED>(A, meta, p);
    pi_pr = st_pr;
    pi_last = p;
    sg = geom(ch);
    const h16* xsl = st_pr.x + st_kj * A.K;
    const int round = 4 * (int)blockDim.x;
    const bool two = sg.nblk > round;  // uniform
    half8_t v[4], v2[4];
    stage_load<(ROUTE != 0)>(A, xsl, sg, 0, v, rperm, st_pr.t0);
    if (two) stage_load<(ROUTE != 0)>(A, xsl, sg, round, v2, rperm, st_pr.t0);
    issue_next(b0);
    if (NBUF == 3) issue_next(b1);
    stage_zero_rows(A, sg.Mc, cs);
    stage_store(A, sg, 0, v, xs, cs);
    if (two) stage_store(A, sg, round, v2, xs, cs);
    for (int base = 2 * round; base < sg.nblk; base += round) {
      stage_load<(ROUTE != 0)>(A, xsl, sg, base, v, rperm, st_pr.t0);
      stage_store(A, sg, base, v, xs, cs);
    }
    __syncthreads();
  }

  // One column: restage if its chunk changes (before the next column's loads
  // go out, so waiting for the activations never waits for those), issue
  // column c + NBUF - 1, unpack/MFMA column c, reduce over the waves.
  auto step = [&](int c, const WBuf<MATS, PAIRS, WIDE>& cur, WBuf<MATS, PAIRS, WIDE>& nxt) {
    int t = 0;
    if (c < ce) {  // uniform
      int p, ch;
      locate(cu_c, chunk_off, nprob, tiles, c, p, ch, t);
      const int kj = KS > 1 ? t / tiles_n : 0;
      if (p != st_p || ch != st_ch || kj != st_kj) {
        if (p != st_p) st_pr = resolve<GROUPED>(A, meta, p);
        st_p = p;
        st_ch = ch;
        st_kj = kj;
        sg = geom(ch);
        stage<(ROUTE != 0)>(A, st_pr.x + st_kj * A.K, sg, xs, cs, rperm, st_pr.t0);
      }
    }
    issue_next(nxt);
    if (c < ce) {
      const int Mc = sg.Mc;
      int arow_i[TH];
#pragma unroll
      for (int h = 0; h < TH; ++h) arow_i[h] = 2 * min(8 * h + (col >> 1), Mc - 1) + (col & 1);
      float4_t acc_lo[TH][MATS], acc_hi[TH][MATS];
      compute<MATS, PAIRS, WIDE, TH>(cur, xs, cs, A.ldx, pb0, gw, arow_i, q, col >= 8 ? 16 : 0,
                                     ur, acc_lo, acc_hi);
      // lane (col, q): row n0 + col, tokens 8h + 2q, 8h + 2q + 1 (both group parities)
      float2 v[TH][MATS];
      const bool low = col < 8;
#pragma unroll
      for (int h = 0; h < TH; ++h)
#pragma unroll
        for (int mt = 0; mt < MATS; ++mt) {
          const float e0 = low ? acc_lo[h][mt][0] : acc_hi[h][mt][1];
          const float u0 = low ? acc_hi[h][mt][0] : acc_lo[h][mt][1];
          const float e1 = low ? acc_lo[h][mt][2] : acc_hi[h][mt][3];
          const float u1 = low ? acc_hi[h][mt][2] : acc_lo[h][mt][3];
          v[h][mt] = float2{e0 + xor8(u0), e1 + xor8(u1)};
        }
      // the tile's outputs of token half h from the wave-summed partials
      auto emit = [&](int h, const float2 (&vv)[MATS]) {
        const int row = (t - st_kj * tiles_n) * kTileN + col;
        if (row >= N) return;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int m = 8 * h + 2 * q + j;
          if (m >= Mc) continue;
          const float g = j ? vv[0].y : vv[0].x;
          if (KS > 1) {
            A.out32[st_kj * A.ks_stride + (long)(st_pr.t0 + sg.m0 + m) * N + row] = g;
          } else {
            h16 o16;
            if (EPI == 1) {
              const float u = j ? vv[MATS - 1].y : vv[MATS - 1].x;
              o16 = (h16)(hn_silu((float)(h16)g) * (float)(h16)u);
            } else {
              o16 = (h16)g;
            }
            st_pr.out[(long)(sg.m0 + m) * A.ld_o + row] = o16;
          }
        }
      };
      // KW-wave reduction through LDS (parity-buffered: one barrier per
      // column; single-buffered: a second barrier first, after which the
      // previous column's partials have been read), summed in wave order
      float2* rb = red + (NRB == 2 ? parity * kRedSlots : 0);
      if (NRB == 1) __syncthreads();
      if constexpr (TH == 1) {
        // waves 1.. store; wave 0 adds them to its own and writes the tile
        if (wave > 0) {
#pragma unroll
          for (int mt = 0; mt < MATS; ++mt) rb[((wave - 1) * MATS + mt) * 64 + lane] = v[0][mt];
        }
        __syncthreads();
        if (wave == 0) {
          float2 o[kMaxWaves - 1][MATS];
#pragma unroll
          for (int w2 = 0; w2 < kMaxWaves - 1; ++w2)
#pragma unroll
            for (int mt = 0; mt < MATS; ++mt) o[w2][mt] = rb[(w2 * MATS + mt) * 64 + lane];
#pragma unroll
          for (int w2 = 0; w2 < kMaxWaves - 1; ++w2)
#pragma unroll
            for (int mt = 0; mt < MATS; ++mt) {
              v[0][mt].x += o[w2][mt].x;
              v[0][mt].y += o[w2][mt].y;
            }
          emit(0, v[0]);
        }
      } else {
        // every wave stores both halves; wave h sums half h over the waves in
        // wave order (slots of absent waves hold zeros) and writes its tokens
#pragma unroll
        for (int h = 0; h < TH; ++h)
#pragma unroll
          for (int mt = 0; mt < MATS; ++mt)
            rb[((wave * TH + h) * MATS + mt) * 64 + lane] = v[h][mt];
        __syncthreads();
        if (wave < TH) {
          const int h = wave;
          float2 o[kMaxWaves][MATS];
#pragma unroll
          for (int w2 = 0; w2 < kMaxWaves; ++w2)
#pragma unroll
            for (int mt = 0; mt < MATS; ++mt) o[w2][mt] = rb[((w2 * TH + h) * MATS + mt) * 64 + lane];
          float2 sum[MATS];
#pragma unroll
          for (int mt = 0; mt < MATS; ++mt) sum[mt] = o[0][mt];
#pragma unroll
          for (int w2 = 1; w2 < kMaxWaves; ++w2)
#pragma unroll
            for (int mt = 0; mt < MATS; ++mt) {
              sum[mt].x += o[w2][mt].x;
              sum[mt].y += o[w2][mt].y;
            }
          emit(h, sum);
        }
      }
      parity ^= 1;
    }
  };

  for (int c = cb; c < ce; c += NBUF) {
    if (NBUF == 2) {
      step(c, b0, b1);
      step(c + 1, b1, b0);
    } else {
      step(c, b0, b2);
      step(c + 1, b1, b0);
      step(c + 2, b2, b1);
    }
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
namespace {

constexpr int kLdsPerCu = 160 * 1024;
constexpr int kStaticLds = 1040;  // chunk_off[]

struct GroupedPtrs {
  const SExpert* table;
  const int* active;
  const int* n_active;
  const int* offsets;
};

struct StreamPlan {
  bool ok;
  bool wide;  // vector scale loads (set by the caller after its alignment checks)
  int lpw, nbuf, kw, tc, ldx, npair;
  int th;     // token halves of 8 per chunk (2: up to 16 tokens per pass)
  int lds;  // dynamic LDS bytes per workgroup
  int occ;  // workgroups per CU
};

// One workgroup per CU of KW <= 8 waves; LPW (2..16) groups of 128 k per wave
// per column, the smallest that covers K with 8 waves; three column buffers
// when they fit the register budget, else two.  tc tokens per chunk: up to 8,
// or up to 16 (two token halves per weight operand) when want16 and an
// instantiation exists, limited by the LDS left after the corrections and the
// reduction buffers.
// LDS scratch of the routing prologue (ROUTE), in front of the metadata:
// 16 slice partials of 16 x 16 logits, the logits (T E <= 512), the selection.
constexpr int kRouteScratch = 16 * 16 * 16 * 4 + 512 * 4 + 64 * 4 + 64 * 2 + 16;

// Shapes with a 16-token instantiation (launch_lpw): four groups per wave
// (grouped gate/up and the down K slices, one expert's gate/up).  Sixteen
// groups per wave (one expert's 14336-long down projection) would spill.
bool th2_instantiated(bool /*grouped*/, int /*mats*/, int lpw) { return lpw == 4; }

StreamPlan stream_plan(long K, int mats, long rows, long E = 0, bool route = false,
                       bool want16 = false, bool grouped = true, long route_rows = 64,
                       long route_scratch = kRouteScratch) {
  StreamPlan p{};
  const long G = K / 128;
  int lpw = 2;
  while (lpw < 16 && (G + lpw - 1) / lpw > kMaxWaves) lpw *= 2;
  // grouped single-matrix (down) launches: at least four groups per wave --
  // fewer waves per workgroup, more workgroups per CU (below); measured on
  // GLM's down projection (K = 1408): 2 groups x 6 waves, 2 workgroups per CU
  // 92 us, 4 groups x 3 waves, 4 workgroups per CU 79 us
  if (mats == 1 && grouped && !route && lpw < 4) lpw = 4;
  const long kw = (G + lpw - 1) / lpw;
  if (kw > kMaxWaves || rows < 1 || K % 128 != 0) return p;
  p.lpw = lpw;
  p.nbuf = mats * lpw * 3 <= 24 ? 3 : 2;
  p.kw = (int)kw;
  p.npair = (int)(kw * lpw / 2);
  p.ldx = p.npair * 128 + 8;  // row stride = 16 B mod 256 B: conflict-free A reads
  // grouped metadata copy: active [E], offsets [E + 1] (each padded to even), pointers [E][4]
  // (ROUTE: and the permuted-row map, route_rows entries)
  const int meta = (int)(((E + 1) & ~1L) * 4 + ((E + 2) & ~1L) * 4 + E * 32) +
                   (route ? (int)(4 * route_rows) : 0);
  const int cs = p.npair * kCsw * 4;
  const int per_tok = 2 * p.ldx * 2;
  for (int th = (want16 && rows > 8 && th2_instantiated(grouped, mats, lpw)) ? 2 : 1;
       th >= 1; --th) {
    const int nrb = (th == 2 && mats == 2) ? 1 : 2;  // the kernel's reduction buffers
    const int red = nrb * (th == 1 ? kMaxWaves - 1 : kMaxWaves) * th * mats * 64 * 8;
    const int want = (int)(rows < 8 * th ? rows : 8 * th);
    const int tcmax = (kLdsPerCu - kStaticLds - red - cs - meta) / per_tok;
    const int tc = tcmax < want ? tcmax : want;
    if (th == 2 && tc <= 8) continue;  // no room for a second token half
    p.th = th;
    p.tc = tc;
    if (p.tc < 1) return p;
    p.lds = p.tc * per_tok + cs + red + meta;
    if (route && p.tc * per_tok + cs + red < route_scratch) return p;
    // single-matrix (down) launches of 4 or more rows per matrix: as many
    // workgroups per CU (up to four) as their LDS and 16 waves allow, for more
    // loads in flight where a column has little work (measured: gate/up
    // launches and 1-row launches are faster with one); launch_one caps this
    // by what the registers allow
    p.occ = 1;
    if (mats == 1 && !route && rows >= 4)
      while (p.occ < 4 && (p.occ + 1) * (p.lds + kStaticLds) <= kLdsPerCu &&
             (p.occ + 1) * kw <= 16)
        ++p.occ;
    p.ok = true;
    return p;
  }
  return p;
}

int num_cus() { return hn_device_cus(); }

template <bool GROUPED, int MATS, int EPI, int LPW, int NBUF, bool WIDE, int KS = 1,
          int ROUTE = 0, int TH = 1>
int launch_one(const StreamArgs& A, const GroupedPtrs& g, const StreamPlan& p, hipStream_t s) {
  if (p.th != TH) return HN_NOT_HANDLED;  // the plan was sized for the other chunking
  auto kern = stream_kernel<GROUPED, MATS, EPI, LPW, NBUF, WIDE, KS, ROUTE, TH>;
  static HnPerDevice attr;  // per instantiation and device
  // workgroups per CU the registers allow, per block size (kw waves): one
  // instantiation serves several K (e.g. K = 1408 and 14336 down projections)
  static HnPerDevice fit[kMaxWaves + 1];
  const int dev = hn_current_device();
  std::atomic<int>& sa = attr.state[dev];
  int st = sa.load(std::memory_order_relaxed);
  if (st == 0) {
    st = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                             kLdsPerCu - kStaticLds) == hipSuccess ? 1 : 2;
    if (st == 2) (void)hipGetLastError();  // plans then stay within 64 KiB
    sa.store(st, std::memory_order_relaxed);
  }
  if (st != 1 && p.lds > 64 * 1024 - kStaticLds) return HN_NOT_HANDLED;
  int occ = p.occ;
  if (occ > 1) {
    // the plan checked LDS and waves; the registers decide too (a kernel
    // over 128 VGPRs holds three waves per SIMD: one 7-wave workgroup per CU)
    std::atomic<int>& sf = fit[p.kw].state[dev];
    int n = sf.load(std::memory_order_relaxed);
    if (n == 0) {
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, (const void*)kern, p.kw * 64, 0) !=
              hipSuccess || n < 1) {
        (void)hipGetLastError();
        n = 1;
      }
      sf.store(n, std::memory_order_relaxed);
    }
    occ = occ < n ? occ : n;
  }
  hipLaunchKernelGGL(kern, dim3(num_cus() * occ), dim3(p.kw * 64), (size_t)p.lds, s, A, g.table,
                     g.active, g.n_active, g.offsets);
  return 0;
}

template <bool GROUPED, int MATS, int EPI, bool WIDE>
int launch_lpw(const StreamArgs& A, const GroupedPtrs& g, const StreamPlan& p, hipStream_t s) {
  if (p.th == 2) {  // the shapes th2_instantiated() names
    // gate/up: two column buffers (a third spills); one matrix: three
    if (p.lpw == 4)
      return launch_one<GROUPED, MATS, EPI, 4, MATS == 2 ? 2 : 3, WIDE, 1, false, 2>(A, g, p, s);
    return HN_NOT_HANDLED;
  }
  if constexpr (MATS == 2) {
    if (p.lpw == 2) return launch_one<GROUPED, MATS, EPI, 2, 3, WIDE>(A, g, p, s);
    // one expert's gate/up (a few columns per workgroup): two columns in
    // flight stream faster than three (measured on MI355X: 16.4 vs 18.3 us at
    // Mixtral's shape, T = 1); the grouped launches keep three
    if (p.lpw == 4 && !GROUPED) return launch_one<GROUPED, MATS, EPI, 4, 2, WIDE>(A, g, p, s);
    if (p.lpw == 4) return launch_one<GROUPED, MATS, EPI, 4, 3, WIDE>(A, g, p, s);
    if (p.lpw == 8) return launch_one<GROUPED, MATS, EPI, 8, 2, WIDE>(A, g, p, s);
  } else {
    if (p.lpw == 2) return launch_one<GROUPED, MATS, EPI, 2, 3, WIDE>(A, g, p, s);
    if (p.lpw == 4) return launch_one<GROUPED, MATS, EPI, 4, 3, WIDE>(A, g, p, s);
    if (p.lpw == 8) return launch_one<GROUPED, MATS, EPI, 8, 3, WIDE>(A, g, p, s);
    if (p.lpw == 16) return launch_one<GROUPED, MATS, EPI, 16, 2, WIDE>(A, g, p, s);
  }
  return HN_NOT_HANDLED;
}

template <bool GROUPED, int MATS, int EPI>
int launch_stream(const StreamArgs& A, const GroupedPtrs& g, const StreamPlan& p,
                  hipStream_t s) {
  return p.wide ? launch_lpw<GROUPED, MATS, EPI, true>(A, g, p, s)
                : launch_lpw<GROUPED, MATS, EPI, false>(A, g, p, s);
}

// Down projection in kDownSplit K slices: one slice of I = 14336 is 28
// groups, 7 waves x 4 groups with three column buffers.
constexpr int kDownSplit = kHnDownSplit;

// 16-token chunks for a grouped launch when its rows average 5 or more per
// expert (e.g. 64 decode tokens at top-1 over 8 experts): an expert's rows
// then mostly exceed 8, and one pass over its weights replaces two.
bool want16_grouped(long rows, long E) { return E > 0 && rows >= 5 * E; }

// Vector scale loads need the wave's LPW groups inside the scale row and
// 16-byte aligned scale rows.
bool wide_scales_ok(const StreamPlan& p, long K, long ld_s) {
  return K / 128 == (long)p.kw * p.lpw && (ld_s * 2) % 16 == 0;
}

void fill_common(StreamArgs& A, const StreamPlan& p, long N, long K) {
  A.N = (int)N;
  A.K = (int)K;
  A.tc = p.tc;
  A.ldx = p.ldx;
  A.npair = p.npair;
  A.m_lo = 0x000F000Fu;
  A.m_hi = 0x00F000F0u;
  A.magic = 0x64006400u;
}

}  // namespace

// Streaming decode, single problem (the entry points of hn_gemv.hip call this
// first).  Returns HN_NOT_HANDLED when the shape is not handled here (the
// caller then uses the split-K kernels), 0 after a launch, a HIP error code if
// the launch failed.
extern "C" int hn_stream_linear_impl(int mats, const void* x, long ld_x, const void* q0,
                                     const void* s0, const void* q1, const void* s1, long ld_q,
                                     long ld_s, void* out, long ld_o, long M, long N, long K,
                                     long group, void* stream) {
  const StreamPlan p = stream_plan(K, mats, M, 0, false, true, false);
  if (!p.ok || group != 128 || M > p.tc) return HN_NOT_HANDLED;
  if (mats == 2 && p.lpw > 8) return HN_NOT_HANDLED;
  if (N * ld_q >= (long)kOOB || N * ld_s * 2 >= (long)kOOB || ld_x >= (1L << 31) ||
      ld_o >= (1L << 31))
    return HN_NOT_HANDLED;
  StreamPlan pw = p;
  pw.wide = wide_scales_ok(p, K, ld_s) && ((uintptr_t)s0 & 15) == 0 && ((uintptr_t)s1 & 15) == 0;
  StreamArgs A = {};
  A.x = (const h16*)x;
  A.ld_x = (int)ld_x;
  A.M = (int)M;
  A.q[0] = (const uint8_t*)q0; A.s[0] = (const h16*)s0;
  A.q[1] = (const uint8_t*)q1; A.s[1] = (const h16*)s1;
  A.ld_q = (int)ld_q;
  A.ld_s = (int)ld_s;
  A.out = (h16*)out;
  A.ld_o = (int)ld_o;
  fill_common(A, p, N, K);
  hipStream_t s = (hipStream_t)stream;
  const GroupedPtrs g = {};
  const int rc = mats == 2 ? launch_stream<false, 2, 1>(A, g, pw, s)
                           : launch_stream<false, 1, 0>(A, g, pw, s);
  if (rc) return rc;
  HN_LAUNCH_CHECK("hn_stream_linear");
  return 0;
}

// Streaming decode, grouped over the active experts of one MoE layer; phase 0
// is gate/up + SiLU into h, phase 1 the down projection.  dry_run: only say
// whether the shape is handled (0) or not (HN_NOT_HANDLED).
extern "C" int hn_stream_grouped_impl(int phase, const void* x, long ld_x, const void* table,
                                      const int* active, const int* n_active, const int* offsets,
                                      long E, long max_rows, long rows, long H, long I, long group,
                                      void* out, long ld_o, void* stream, int dry_run) {
  const int mats = phase == 0 ? 2 : 1;
  const long K = phase == 0 ? H : I, N = phase == 0 ? I : H;
  if (E > kMaxActive) return HN_NOT_HANDLED;
  const StreamPlan p = stream_plan(K, mats, max_rows, E, false, want16_grouped(rows, E));
  if (!p.ok || group != 128) return HN_NOT_HANDLED;
  if (mats == 2 && p.lpw > 8) return HN_NOT_HANDLED;
  if (N * (K / 2) >= (long)kOOB || N * (K / group) * 2 >= (long)kOOB) return HN_NOT_HANDLED;
  if (dry_run) return 0;
  // table pointers are 16-byte aligned (the grouped entry point's contract)
  StreamPlan pw = p;
  pw.wide = wide_scales_ok(p, K, K / group);
  StreamArgs A = {};
  A.x = (const h16*)x;
  A.ld_x = (int)ld_x;
  A.phase = phase;
  A.E = (int)E;
  A.ld_q = (int)(K / 2);
  A.ld_s = (int)(K / group);
  A.out = (h16*)out;
  A.ld_o = (int)ld_o;
  fill_common(A, p, N, K);
  const GroupedPtrs g = {(const SExpert*)table, active, n_active, offsets};
  hipStream_t s = (hipStream_t)stream;
  const int rc = mats == 2 ? launch_stream<true, 2, 1>(A, g, pw, s)
                           : launch_stream<true, 1, 0>(A, g, pw, s);
  if (rc) return rc;
  HN_LAUNCH_CHECK("hn_stream_grouped");
  return 0;
}

// Down projection of the grouped decode in kDownSplit K slices: fp32 partials
// part[j][row][H] (j < kDownSplit, ks_stride = rows_cap * H floats), summed
// in slice order by the caller.  Returns HN_NOT_HANDLED when the shape does
// not split (then the caller runs hn_stream_grouped_impl's phase 1).
extern "C" int hn_stream_down_split_impl(const void* h, const void* table, const int* active,
                                         const int* n_active, const int* offsets, long E,
                                         long max_rows, long rows_cap, long H, long I,
                                         long group, float* part, void* stream,
                                         int dry_run) {
  const long K = I / kDownSplit, N = H;
  if (I % (kDownSplit * 128) != 0 || group != 128 || E > kMaxActive) return HN_NOT_HANDLED;
  const StreamPlan p = stream_plan(K, 1, max_rows, E, false, want16_grouped(rows_cap, E));
  if (!p.ok || p.lpw != 4 || !wide_scales_ok(p, K, I / group)) return HN_NOT_HANDLED;
  if (N * (I / 2) >= (long)kOOB || N * (I / group) * 2 >= (long)kOOB) return HN_NOT_HANDLED;
  if (dry_run) return 0;
  StreamArgs A = {};
  A.x = (const h16*)h;
  A.ld_x = (int)I;
  A.phase = 1;
  A.E = (int)E;
  A.ld_q = (int)(I / 2);
  A.ld_s = (int)(I / group);
  A.out32 = part;
  A.ks_stride = rows_cap * H;
  fill_common(A, p, N, K);
  StreamPlan pw = p;
  pw.wide = true;
  const GroupedPtrs g = {(const SExpert*)table, active, n_active, offsets};
  const int rc = pw.th == 2
      ? launch_one<true, 1, 0, 4, 3, true, kDownSplit, false, 2>(A, g, pw, (hipStream_t)stream)
      : launch_one<true, 1, 0, 4, 3, true, kDownSplit>(A, g, pw, (hipStream_t)stream);
  if (rc) return rc;
  HN_LAUNCH_CHECK("hn_stream_down_split");
  return 0;
}

// Decode routing fused into the grouped gate/up launch: Mixtral softmax top-k
// (k = 1 or 2, T k <= 64) over E <= 8 experts, logits from the fp16 gate
// [E, H] (T <= 16; the arithmetic of hn_moe_route) or given in logits_in
// [T, E], then h_ws = SwiGLU gate/up of the routed rows, staged from hx
// directly (no x_perm).  Workgroup 0 writes logits_out (optional), idx, w,
// offsets, perm, inv, active and n_active for the down projection and the
// unpermute.  Returns HN_NOT_HANDLED when the shape is not covered.
extern "C" int hn_stream_route_gate_up_impl(const void* hx, long ld_hx, const void* gate,
                                            long ld_gate, const float* logits_in, long T, long E,
                                            long k, const void* table, long H, long I, long group,
                                            float eps, float scaling, float* logits_out,
                                            int* idx, void* w, int* offsets, int* perm,
                                            int* inv, int* active, int* n_active,
                                            long long* usage, void* h_ws, void* stream,
                                            int dry_run) {
  if (T < 1 || E < 1 || E > 8 || (k != 1 && k != 2) || T * k > 64 ||
      (!logits_in && T > 16) || H % 512 != 0 || group != 128 || I % 128 != 0 ||
      ld_hx % 8 != 0 || (!logits_in && ld_gate % 8 != 0) || ld_hx >= (1L << 31) ||
      ld_gate >= (1L << 31))
    return HN_NOT_HANDLED;
  const StreamPlan p = stream_plan(H, 2, T, E, true, want16_grouped(T * k, E));
  if (!p.ok || p.lpw > 8 || !wide_scales_ok(p, H, H / group)) return HN_NOT_HANDLED;
  if (I * (H / 2) >= (long)kOOB || I * (H / group) * 2 >= (long)kOOB) return HN_NOT_HANDLED;
  if (dry_run) return 0;
  StreamPlan pw = p;
  pw.wide = true;
  StreamArgs A = {};
  A.x = (const h16*)hx;  // unused: rows come from hx through the permutation
  A.ld_x = 0;
  A.phase = 0;
  A.E = (int)E;
  A.ld_q = (int)(H / 2);
  A.ld_s = (int)(H / group);
  A.out = (h16*)h_ws;
  A.ld_o = (int)I;
  fill_common(A, p, I, H);
  A.hx = (const h16*)hx;
  A.ld_hx = (int)ld_hx;
  A.gate = (const h16*)gate;
  A.ld_gate = (int)ld_gate;
  A.logits_in = logits_in;
  A.T = (int)T;
  A.topk = (int)k;
  A.eps = eps;
  A.scaling = scaling;
  A.logits_out = logits_out;
  A.idx_out = idx;
  A.w_out = (h16*)w;
  A.offsets_out = offsets;
  A.perm_out = perm;
  A.inv_out = inv;
  A.active_out = active;
  A.n_active_out = n_active;
  A.usage = usage;
  const GroupedPtrs g = {(const SExpert*)table, nullptr, nullptr, nullptr};
  hipStream_t s = (hipStream_t)stream;
  int rc = HN_NOT_HANDLED;
  if (p.th == 2) rc = launch_one<true, 2, 1, 4, 2, true, 1, 1, 2>(A, g, pw, s);
  else if (p.lpw == 2) rc = launch_one<true, 2, 1, 2, 3, true, 1, 1>(A, g, pw, s);
  else if (p.lpw == 4) rc = launch_one<true, 2, 1, 4, 3, true, 1, 1>(A, g, pw, s);
  else if (p.lpw == 8) rc = launch_one<true, 2, 1, 8, 2, true, 1, 1>(A, g, pw, s);
  if (rc) return rc;
  HN_LAUNCH_CHECK("hn_stream_route_gate_up");
  return 0;
}

// Decode routing from given logits fused into the grouped gate/up launch
// (ROUTE 2): top-k in mode 0 (softmax), 1 (sigmoid) or 2 (sigmoid,
// unnormalised) with an optional selection bias over E <= 256 experts, T k
// routed rows (at most the launch's threads), then h_ws = SwiGLU gate/up of
// the routed rows staged from hx.  Workgroup 0 writes idx, w, offsets, perm,
// inv, active and n_active (and adds the usage counts).  Returns
// HN_NOT_HANDLED when the shape is not covered.
extern "C" int hn_stream_route_sel_gate_up_impl(const void* hx, long ld_hx,
                                                const float* logits_in, const float* bias, long T,
                                                long E, long k, int mode, float eps,
                                                float scaling, const void* table, long H, long I,
                                                long group, int* idx, void* w, int* offsets,
                                                int* perm, int* inv, int* active, int* n_active,
                                                long long* usage, void* h_ws, void* stream,
                                                int dry_run) {
  if (T < 1 || E < 1 || E > kMaxActive || k < 1 || k > 16 || k > E || mode < 0 || mode > 2 ||
      H % 512 != 0 || group != 128 || I % 128 != 0 || ld_hx % 8 != 0 || ld_hx >= (1L << 31))
    return HN_NOT_HANDLED;
  const long n = T * k;
  const long G = H / 128;
  int lpw = 2;
  while (lpw < 16 && (G + lpw - 1) / lpw > kMaxWaves) lpw *= 2;
  const long kw = (G + lpw - 1) / lpw;
  if (n > kw * 64) return HN_NOT_HANDLED;  // one thread per routed row in the ranks
  const long scratch = T * E * 4 + n * 4 + ((n + 1) & ~1L) * 2 + kw * E * 4 + 16;
  const StreamPlan p = stream_plan(H, 2, T, E, true, false, true, n, scratch);
  if (!p.ok || p.lpw > 8 || p.th != 1 || !wide_scales_ok(p, H, H / group)) return HN_NOT_HANDLED;
  if (I * (H / 2) >= (long)kOOB || I * (H / group) * 2 >= (long)kOOB) return HN_NOT_HANDLED;
  if (dry_run) return 0;
  StreamPlan pw = p;
  pw.wide = true;
  StreamArgs A = {};
  A.x = (const h16*)hx;  // unused: rows come from hx through the permutation
  A.phase = 0;
  A.E = (int)E;
  A.ld_q = (int)(H / 2);
  A.ld_s = (int)(H / group);
  A.out = (h16*)h_ws;
  A.ld_o = (int)I;
  fill_common(A, p, I, H);
  A.hx = (const h16*)hx;
  A.ld_hx = (int)ld_hx;
  A.logits_in = logits_in;
  A.bias = bias;
  A.mode = mode;
  A.T = (int)T;
  A.topk = (int)k;
  A.eps = eps;
  A.scaling = scaling;
  A.idx_out = idx;
  A.w_out = (h16*)w;
  A.offsets_out = offsets;
  A.perm_out = perm;
  A.inv_out = inv;
  A.active_out = active;
  A.n_active_out = n_active;
  A.usage = usage;
  const GroupedPtrs g = {(const SExpert*)table, nullptr, nullptr, nullptr};
  hipStream_t s = (hipStream_t)stream;
  int rc = HN_NOT_HANDLED;
  if (p.lpw == 2) rc = launch_one<true, 2, 1, 2, 3, true, 1, 2>(A, g, pw, s);
  else if (p.lpw == 4) rc = launch_one<true, 2, 1, 4, 3, true, 1, 2>(A, g, pw, s);
  else if (p.lpw == 8) rc = launch_one<true, 2, 1, 8, 2, true, 1, 2>(A, g, pw, s);
  if (rc) return rc;
  HN_LAUNCH_CHECK("hn_stream_route_sel_gate_up");
  return 0;
}
