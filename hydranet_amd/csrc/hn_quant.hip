// INT4 dequantise and quantise kernels (gfx950).
//
// Dequantise follows the reference's dequantisers, which are bit-identical
// to one another: preprocess/pack_weights.py:230-268,
// cache/packed_expert_store.py:287-315, kernels/expert_mlp.py:305-330:
//   W[n, k] = fp16( (nibble(n, k) - 8) * scale[n, k / group] ).
// (nibble - 8) is exact in fp16 and the product is rounded once (RNE), which
// is what v_pk_mul_f16 does with fp16 denormals enabled (the gfx9 default).
//
// Quantise restates two reference quantisers in their own arithmetic:
//   mode 0  ExpertWeightPacker.quantize_tensor  (preprocess/pack_weights.py:133-181)
//   mode 1  Int4Linear.quantize_weight          (kernels/int4_linear.py:68-107)
#include "hn_common.h"

// One thread handles 32 consecutive k of one row: 16 packed bytes in,
// 32 fp16 (64 bytes) out.
__global__ __launch_bounds__(256) void hn_dequant_kernel(
    const uint8_t* __restrict__ packed, long ld_p,
    const h16* __restrict__ scales, long ld_s,
    h16* __restrict__ out, long ld_o,
    int N, int K, int group) {
  const int chunks = K >> 5;  // K % 32 == 0 checked on the host
  const long tid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (tid >= (long)N * chunks) return;
  const int n = (int)(tid / chunks);
  const int c = (int)(tid % chunks);
  const int k0 = c << 5;
  const u32x4 w = *reinterpret_cast<const u32x4*>(packed + n * ld_p + (k0 >> 1));
  const h16* srow = scales + n * ld_s;
  h16* orow = out + n * ld_o + k0;
  h16 res[32];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    half2_t p[4];
    hn_unpack8_centered(w[d], p);
    const int kb = k0 + 8 * d;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // p[i] = (k_i, k_{i+4}) relative to kb
      const h16 s_lo = srow[(kb + i) / group];
      const h16 s_hi = srow[(kb + i + 4) / group];
      const half2_t s2 = {s_lo, s_hi};
      const half2_t v = p[i] * s2;
      res[8 * d + i] = v[0];
      res[8 * d + i + 4] = v[1];
    }
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      half2_t h2 = {res[8 * q + 2 * j], res[8 * q + 2 * j + 1]};
      o[j] = __builtin_bit_cast(uint32_t, h2);
    }
    *reinterpret_cast<u32x4*>(orow + 8 * q) = o;
  }
}

// fp16 -> uint8 conversion of the shifted code, as torch's CPU cast does on
// x86 for the values that occur here: exact for 0..15, and NaN (an all-zero
// group gives scale 0 and 0/0) becomes 0 (observed with torch 2.10 on x86).
__device__ __forceinline__ uint32_t hn_code_u8(float q_plus8) {
  if (!(q_plus8 == q_plus8)) return 0u;
  return (uint32_t)(int)q_plus8 & 0xFFu;
}

template <typename T>
__device__ __forceinline__ float hn_load_f(const T* p);
template <>
__device__ __forceinline__ float hn_load_f<h16>(const h16* p) { return (float)*p; }
template <>
__device__ __forceinline__ float hn_load_f<float>(const float* p) { return *p; }

// Mode 0 (ExpertWeightPacker, fp16 input, arithmetic in fp16 with fp32 opmath):
//   absmax = max |w|                      (exact)
//   s      = fp16(float(absmax) / 7.0f)   (pack_weights.py:157, scalar divisor)
//   s      = clamp(s, min=fp16(1e-10)=0)  (:158, a no-op for s >= 0)
//   q      = rint(fp16(float(w) / float(s))), clamped to [-8, 7]   (:161)
//   code   = q + 8                        (:162)
// Mode 1 (Int4Linear.quantize_weight, arithmetic in the input dtype T):
//   absmax = max(max |w|, T(1e-8))        (int4_linear.py:92)
//   s      = fp16(absmax / 7)             (:94)
//   q      = rint(T(T(w / absmax) * 7)), clamped to [-8, 7]        (:97)
template <typename T, int MODE>
__global__ __launch_bounds__(256) void hn_quantize_kernel(
    const T* __restrict__ w, long ld_w,
    uint8_t* __restrict__ packed, long ld_p,
    h16* __restrict__ scales, long ld_s,
    int N, int K, int group) {
  const int groups = K / group;
  const long tid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (tid >= (long)N * groups) return;
  const int n = (int)(tid / groups);
  const int g = (int)(tid % groups);
  const T* row = w + n * ld_w + (long)g * group;
  float amax = 0.0f;
  bool nan_seen = false;
  for (int i = 0; i < group; ++i) {
    const float v = hn_load_f<T>(row + i);
    nan_seen |= !(v == v);
    amax = fmaxf(amax, fabsf(v));
  }
  if (nan_seen) amax = __builtin_nanf("");
  float absmax_t;  // absmax in the arithmetic dtype
  h16 s16;
  if (MODE == 0) {
    absmax_t = amax;  // fp16 value, exact in float
    s16 = (h16)(absmax_t / 7.0f);
  } else {
    if (sizeof(T) == 2) {
      // clamp(min=1e-8) with the scalar cast to fp16 first: fp16(1e-8) == 0
      absmax_t = fmaxf(amax, 0.0f);
      s16 = (h16)(float)(h16)(absmax_t / 7.0f);
    } else {
      absmax_t = fmaxf(amax, 1e-8f);
      s16 = (h16)(absmax_t / 7.0f);
    }
  }
  scales[n * ld_s + g] = s16;
  const float s = (float)s16;
  uint8_t* prow = packed + n * ld_p + ((long)g * group >> 1);
  for (int i = 0; i < group; i += 2) {
    uint32_t code[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float v = hn_load_f<T>(row + i + j);
      float q;
      if (MODE == 0) {
        q = (float)(h16)(v / s);           // fp16 tensor / fp16 tensor
      } else if (sizeof(T) == 2) {
        const float r = (float)(h16)(v / absmax_t);  // fp16 / fp16
        q = (float)(h16)(r * 7.0f);                  // fp16 * python scalar
      } else {
        q = (v / absmax_t) * 7.0f;                   // fp32 throughout
      }
      q = rintf(q);                                  // round half to even
      if (q == q) q = fminf(fmaxf(q, -8.0f), 7.0f);  // clamp keeps NaN
      if (MODE == 0) {
        code[j] = hn_code_u8(q + 8.0f);              // fp16 (q + 8) -> uint8
      } else {
        // q -> int8 first (NaN -> 0 on x86 torch), then int8 + 8 -> uint8
        code[j] = (uint32_t)(((q == q) ? (int)q : 0) + 8) & 0xFFu;
      }
    }
    prow[i >> 1] = (uint8_t)((code[1] << 4) | (code[0] & 0xFu));
  }
}

extern "C" int hn_int4_dequant(const void* packed, long ld_p, const void* scales, long ld_s,
                               void* out, long ld_o, long N, long K, long group,
                               void* stream) {
  HN_ARG_CHECK(N >= 0 && K >= 0, "hn_int4_dequant: negative dims");
  HN_ARG_CHECK(K % 32 == 0, "hn_int4_dequant: K=%ld must be a multiple of 32", K);
  HN_ARG_CHECK(group > 0 && K % group == 0, "hn_int4_dequant: group=%ld must divide K=%ld",
               group, K);
  HN_ARG_CHECK(((uintptr_t)packed % 16 == 0) && (ld_p % 16 == 0),
               "hn_int4_dequant: packed rows must be 16-byte aligned");
  HN_ARG_CHECK(((uintptr_t)out % 16 == 0) && (ld_o % 8 == 0),
               "hn_int4_dequant: output rows must be 16-byte aligned");
  if (N == 0 || K == 0) return 0;
  const long threads = N * (K / 32);
  hipLaunchKernelGGL(hn_dequant_kernel, dim3(hn_cdiv(threads, 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint8_t*)packed, ld_p, (const h16*)scales,
                     ld_s, (h16*)out, ld_o, (int)N, (int)K, (int)group);
  HN_LAUNCH_CHECK("hn_int4_dequant");
  return 0;
}

// dtype: 0 = fp16 input, 1 = fp32 input.  mode: 0 = expert packer, 1 = Int4Linear.
extern "C" int hn_int4_quantize(const void* w, long ld_w, int dtype, int mode, void* packed,
                                long ld_p, void* scales, long ld_s, long N, long K, long group,
                                void* stream) {
  HN_ARG_CHECK(N >= 0 && K >= 0, "hn_int4_quantize: negative dims");
  HN_ARG_CHECK(group > 0 && group % 2 == 0 && K % group == 0,
               "hn_int4_quantize: group=%ld must be even and divide K=%ld", group, K);
  HN_ARG_CHECK(dtype == 0 || dtype == 1, "hn_int4_quantize: dtype must be 0 (fp16) or 1 (fp32)");
  HN_ARG_CHECK(mode == 0 || mode == 1, "hn_int4_quantize: mode must be 0 or 1");
  HN_ARG_CHECK(!(mode == 0 && dtype == 1),
               "hn_int4_quantize: the expert packer takes fp16 weights (loaders cast to fp16)");
  if (N == 0 || K == 0) return 0;
  const long threads = N * (K / group);
  dim3 grid(hn_cdiv(threads, 256)), block(256);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == 0 && mode == 0)
    hipLaunchKernelGGL((hn_quantize_kernel<h16, 0>), grid, block, 0, s, (const h16*)w, ld_w,
                       (uint8_t*)packed, ld_p, (h16*)scales, ld_s, (int)N, (int)K, (int)group);
  else if (dtype == 0)
    hipLaunchKernelGGL((hn_quantize_kernel<h16, 1>), grid, block, 0, s, (const h16*)w, ld_w,
                       (uint8_t*)packed, ld_p, (h16*)scales, ld_s, (int)N, (int)K, (int)group);
  else
    hipLaunchKernelGGL((hn_quantize_kernel<float, 1>), grid, block, 0, s, (const float*)w,
                       ld_w, (uint8_t*)packed, ld_p, (h16*)scales, ld_s, (int)N, (int)K,
                       (int)group);
  HN_LAUNCH_CHECK("hn_int4_quantize");
  return 0;
}
