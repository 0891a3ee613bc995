// Shared device/host helpers for the gfx950 INT4 expert-MLP kernels.
//
// Packed INT4 format (HydraNet blob layout, preprocess/pack_weights.py:160-181):
//   packed[n, j] (uint8) holds W[n, 2j] in the low nibble and W[n, 2j+1] in the
//   high nibble, stored as (q + 8) with q in [-8, 7];
//   scales[n, k / group] (fp16);  W[n, k] = fp16((nibble - 8) * scale).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

typedef _Float16 h16;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define HN_WAVE 64

// ---------------------------------------------------------------------------
// Error plumbing for the C ABI (thread-local last error string).
// ---------------------------------------------------------------------------
#ifdef __cplusplus
extern "C" {
#endif
void hn_set_error(const char* fmt, ...);
// CU count of the current device (queried once per device, hn_abi.cpp).
int hn_device_cus(void);
// Current device index, clamped to the per-device caches' range (0..63).
int hn_current_device(void);
// A fresh launch tag for the last-arriver counters (see hn_arrive): process-
// wide, strictly increasing, in [1, 2^48).
unsigned long long hn_next_tag(void);
#ifdef __cplusplus
}
#endif

// One int per device index (0 = not yet known), for per-kernel facts that
// are set or queried once per device: whether its dynamic-LDS limit was
// raised to the CU's 160 KiB (1 raised, 2 refused), how many of its
// workgroups its registers let one CU hold.
struct HnPerDevice {
  std::atomic<int> state[64] = {};
};

#define HN_ARG_CHECK(cond, ...)              \
  do {                                       \
    if (!(cond)) {                           \
      hn_set_error(__VA_ARGS__);             \
      return -22; /* -EINVAL */              \
    }                                        \
  } while (0)

// Internal return code of the kernel-family dispatchers (hn_stream_*_impl,
// hn_gemm_*_impl): the shape is not handled by that family, try another.
// Never returned through the C ABI.
#define HN_NOT_HANDLED (-1000)

#define HN_LAUNCH_CHECK(what)                                              \
  do {                                                                     \
    hipError_t _e = hipGetLastError();                                     \
    if (_e != hipSuccess) {                                                \
      hn_set_error("%s: launch failed: %s", what, hipGetErrorString(_e));  \
      return (int)_e;                                                      \
    }                                                                      \
  } while (0)

// ---------------------------------------------------------------------------
// Nibble unpacking.
//
// A 32-bit word w of packed data holds 8 consecutive k (k0..k7); nibble k_i
// sits at bits [4i, 4i+4).  The fp16 "magic number" trick places a nibble in
// the mantissa of 1024.0 (0x6400): (w & 0x000F000F) | 0x64006400 is the pair
// (1024 + n0, 1024 + n4).  The high nibble of each byte is used in place as
// 1024 + 16 n, then rescaled with an exact fma.  Output order of the eight
// values is k = (0,4, 1,5, 2,6, 3,7): the activation operand of the matrix
// product is permuted the same way (see hn_perm8), so the reduction
// over k is unchanged.
//
// Every step is exact in fp16: (1024 + n) - 1032 = n - 8, and
// (1024 + 16 n) * 0.0625 - 72 = n - 8, both representable.
// ---------------------------------------------------------------------------
__device__ __forceinline__ half2_t hn_bits_h2(uint32_t v) {
  return __builtin_bit_cast(half2_t, v);
}

__device__ __forceinline__ void hn_unpack8_centered(uint32_t w, half2_t out[4]) {
  const uint32_t lo0 = (w & 0x000F000Fu) | 0x64006400u;
  const uint32_t hi0 = (w & 0x00F000F0u) | 0x64006400u;
  const uint32_t w8 = w >> 8;
  const uint32_t lo1 = (w8 & 0x000F000Fu) | 0x64006400u;
  const uint32_t hi1 = (w8 & 0x00F000F0u) | 0x64006400u;
  const half2_t bias_lo = {(h16)-1032.0f, (h16)-1032.0f};
  const half2_t sixteenth = {(h16)0.0625f, (h16)0.0625f};
  const half2_t bias_hi = {(h16)-72.0f, (h16)-72.0f};
  out[0] = hn_bits_h2(lo0) + bias_lo;                       // k0, k4
  out[1] = __builtin_elementwise_fma(hn_bits_h2(hi0), sixteenth, bias_hi);  // k1, k5
  out[2] = hn_bits_h2(lo1) + bias_lo;                       // k2, k6
  out[3] = __builtin_elementwise_fma(hn_bits_h2(hi1), sixteenth, bias_hi);  // k3, k7
}

// Same unpack, producing the MFMA operand directly.  gfx9 VOP3/VOP3P
// encodings take no literal constants and at most one SGPR, so the masks live
// in SGPRs and the magic number and the fp16 constants in VGPRs (put there
// once per kernel with hn_vgpr).  (w & m) | magic is written as the bit-field
// insert (w & m) | (magic & ~m) -- equal, since the magic has no bit under
// either mask -- which the compiler emits as one v_bfi_b32 (written as
// v_and + v_or, it is two).  It is plain C, not inline asm: the compiler's
// hazard checks between MFMAs and later VALU writes see through it.
struct HnUnpackRegs {
  uint32_t m_lo, m_hi;                       // SGPR: 0x000F000F, 0x00F000F0
  uint32_t magic;                            // VGPR: 0x64006400
  uint32_t bias_lo, sixteenth, bias_hi;      // VGPR: half2 (-1032), (1/16), (-72)
};

// A wave-uniform value in a VGPR (an identity DPP move: a real instruction,
// so the compiler neither folds it back into an SGPR operand nor loses track
// of it in its hazard checks).
__device__ __forceinline__ uint32_t hn_vgpr(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xE4, 0xF, 0xF, false);
}

__device__ __forceinline__ uint32_t hn_and_or(uint32_t w, uint32_t m, uint32_t o) {
  return (w & m) | (o & ~m);
}

__device__ __forceinline__ half8_t hn_unpack8_regs(uint32_t w, const HnUnpackRegs& c) {
  const half2_t bias_lo = hn_bits_h2(c.bias_lo);
  const half2_t sixteenth = hn_bits_h2(c.sixteenth);
  const half2_t bias_hi = hn_bits_h2(c.bias_hi);
  const uint32_t w8 = w >> 8;
  const half2_t p0 = hn_bits_h2(hn_and_or(w, c.m_lo, c.magic)) + bias_lo;
  const half2_t p1 = __builtin_elementwise_fma(hn_bits_h2(hn_and_or(w, c.m_hi, c.magic)),
                                               sixteenth, bias_hi);
  const half2_t p2 = hn_bits_h2(hn_and_or(w8, c.m_lo, c.magic)) + bias_lo;
  const half2_t p3 = __builtin_elementwise_fma(hn_bits_h2(hn_and_or(w8, c.m_hi, c.magic)),
                                               sixteenth, bias_hi);
  const u32x4 r = {__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1),
                   __builtin_bit_cast(uint32_t, p2), __builtin_bit_cast(uint32_t, p3)};
  return __builtin_bit_cast(half8_t, r);
}

// Position j of an 8-block in unpack order holds source index hn_perm8(j).
__host__ __device__ constexpr int hn_perm8(int j) { return (j >> 1) + ((j & 1) << 2); }

__device__ __forceinline__ half8_t hn_cat4(const half2_t p[4]) {
  half8_t r;
  r[0] = p[0][0]; r[1] = p[0][1];
  r[2] = p[1][0]; r[3] = p[1][1];
  r[4] = p[2][0]; r[5] = p[2][1];
  r[6] = p[3][0]; r[7] = p[3][1];
  return r;
}

__device__ __forceinline__ float hn_silu(float g) {
  return g / (1.0f + expf(-g));
}

// dst[0, n) = src[0, n) (global fp32 -> LDS) with every load of a round in
// flight before the first store: rounds of four 16-byte loads per thread
// (a plain loop waits out one memory round trip per element it copies).
// src and dst 16-byte aligned.
__device__ __forceinline__ void copy_to_lds_f32(const float* __restrict__ src, float* dst, int n) {
  const int nv = n >> 2, nthr = blockDim.x, tid = threadIdx.x;
  const float4_t* s4 = reinterpret_cast<const float4_t*>(src);
  float4_t* d4 = reinterpret_cast<float4_t*>(dst);
  for (int base = 0; base < nv; base += 4 * nthr) {
    float4_t v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = base + tid + u * nthr;
      v[u] = i < nv ? s4[i] : float4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = base + tid + u * nthr;
      if (i < nv) d4[i] = v[u];
    }
  }
  for (int i = 4 * nv + tid; i < n; i += nthr) dst[i] = src[i];
}

static inline int hn_cdiv(long a, long b) { return (int)((a + b - 1) / b); }

// ---------------------------------------------------------------------------
// Last-arriver counters of the split reductions (skinny split-K, GEMM
// stream-K).  A counter is a 64-bit word: bits [63:16] the tag of the launch
// that claimed it, bits [15:0] the arrivals counted under that tag.  Every
// launch takes a fresh tag (hn_next_tag).  An arriving wave first claims the
// word for its launch with an atomic max of tag << 16 — a word left by any
// earlier launch, finished or stopped part-way, holds a smaller tag and so
// becomes tag << 16, a count of zero — then adds 1.  The two atomics of one
// wave to one address stay in program order, so the claim precedes the
// count.  The last arrival resets the word to 0, which keeps replays of a
// captured graph (whose tag is fixed at capture) counting from zero.  Two
// cases are not healed by the next launch, because the word then holds a tag
// at or above the next launch's: a graph replay stopped part-way, and an
// eager launch (a later tag) stopped part-way before a replay of a graph
// captured earlier.  A caller recovering from a stopped launch re-zeroes the
// counter region (a fill kernel) before the next replay.
// Launches that share a workspace concurrently race (on the partials too).
//
// Ordering, with the wave's partial stores issued before the call:
//   hn_publish_partials();  n = hn_arrive(c, tag) on one lane;  broadcast n;
//   if last: hn_acquire_agent(), reset, read every split's partial.
// The partials are agent-scope atomic stores and loads (sc1: performed where
// every XCD sees them, past this XCD's L2).  Publishing waits until the
// wave's stores are acknowledged (vmcnt counts stores on gfx9) and is a
// compiler memory barrier, so "partials stored" precedes "counted in"; the
// last arrival's agent-scope acquire fence (L2/L1 invalidate) precedes its
// reads.  An agent-scope release fence in place of the wait would also write
// back this XCD's L2 for plain stores (buffer_wbl2), which the partials are
// not: measured on MI355X it made the split-K GEMV 2-4x and the stream-K GEMM
// 3-14 % slower, with identical results.  Returns the arrival's index,
// 0-based; the caller is last when it is n - 1 for n arrivals.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void hn_publish_partials() {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}
__device__ __forceinline__ void hn_acquire_agent() {
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}
__device__ __forceinline__ int hn_arrive(unsigned long long* c, unsigned long long tag) {
  __hip_atomic_fetch_max(c, tag << 16, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned long long old =
      __hip_atomic_fetch_add(c, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return (int)(old & 0xffffu);
}
__device__ __forceinline__ void hn_counter_reset(unsigned long long* c) {
  __hip_atomic_store(c, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Arrivals per counter are below 2^16.
constexpr long kHnMaxArrivals = 0xffff;

// K slices of the grouped decode's down projection.  Its fp32 partials are
// part[j][rows][H], j < kHnDownSplit, in the caller's workspace: the stream
// kernel's instantiation, the workspace size and both unpermutes that sum
// the slices take the count from here, so they cannot disagree (a kernel
// writing more slices than the workspace holds writes past its end).
constexpr int kHnDownSplit = 4;
