// Top-k selection and routing weights of one token's router logits
// (gfx950 device code shared by the routing kernels and the fused decode
// kernel).  Selection order: larger value first, equal values lower expert
// first.  mode 0 = Mixtral: fp32 softmax over the selected logits and
// renormalisation (model/router.py:109-120); mode 1 = GLM: sigmoid (exp in
// double, rounded once), optional per-expert selection bias, normalise with
// +eps and scale (model/glm4.py:282-309); mode 2 = GLM with
// norm_topk_prob=False: the selected sigmoids times the scale (:302-307).
#pragma once
#include "hn_common.h"

namespace {

constexpr int kMaxTopK = 16;

__device__ __forceinline__ float sigmoid_f32(float l) {
  return (float)(1.0 / (1.0 + exp(-(double)l)));
}

// fp32 product a * b, rounded to fp32 (the reference multiplies the fp32
// weights by the scale, then casts to fp16).  The identity DPP move keeps
// the compiler from converting the exact product to fp16 in one step
// (v_fma_mix), which rounds once instead of twice and can differ by an ulp.
__device__ __forceinline__ float f32_mul(float a, float b) {
  return __builtin_bit_cast(float, hn_vgpr(__builtin_bit_cast(uint32_t, a * b)));
}

// Selection order of top-k: larger value first, equal values lower expert
// first (a strict total order on (value, expert) for non-NaN values).
__device__ __forceinline__ bool topk_beats(float bv, int be, float av, int ae) {
  return bv > av || (bv == av && be < ae);
}

// Routing weights of the k selected experts sel[0..k) (already written) from
// the token's raw logits l: mode 0 fp32 softmax over the selected logits and
// renormalisation by the fp32 sum (model/router.py:114-117); mode 1 sigmoid
// (exp in double, rounded once: it also ranks the experts), / (sum + eps) * scaling
// (model/glm4.py:282-307); mode 2 sigmoid * scaling.  Compact loops: each element's value is recomputed
// where it is needed (same arithmetic each time) instead of kept in arrays.
__device__ __forceinline__ uint32_t order_key(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Unsigned max over the 64 lanes of a wave (every lane gets it): row_shr
// steps to lane 15 of each row of 16, row_bcast:15 and row_bcast:31 across
// the rows, then lane 63 read back (a zero fill is the identity of the max).
template <int CTL>
__device__ __forceinline__ uint32_t dpp_shr_zero(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTL, 0xf, 0xf, true);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_shr_zero<0x111>(v));  // row_shr:1
  v = max(v, dpp_shr_zero<0x112>(v));  // row_shr:2
  v = max(v, dpp_shr_zero<0x114>(v));  // row_shr:4
  v = max(v, dpp_shr_zero<0x118>(v));  // row_shr:8
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false));  // row_bcast:15
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false));  // row_bcast:31
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Top-k of one token's logits row by one wave: lanes hold experts lane +
// 64 j (E <= 256).  k rounds of a wave-wide maximum over the candidates'
// order keys (DPP), the winner being the lowest expert among equal keys
// (ballots, lowest register then lowest lane); the winner's key is cleared
// for the next round.  Rounds pick in selection order (value desc, expert
// asc), so the weights sum the selected in that order: the same selection
// and weight arithmetic as topk_small.
// The selection bias of the lane's four candidates (experts lane + 64 j),
// loaded once per wave and reused for every token: unconditional loads
// (index clamped to E - 1) that go out together.  Zero without a bias.
struct TopkBias {
  float v[4];
  bool on;
};
__device__ __forceinline__ TopkBias topk_wave_bias(const float* bias, int E, int lane) {
  TopkBias b;
  b.on = bias != nullptr;
  const float* src = b.on ? bias : nullptr;
#pragma unroll
  for (int j = 0; j < 4; ++j) b.v[j] = 0.f;
  if (b.on) {  // uniform
#pragma unroll
    for (int j = 0; j < 4; ++j) b.v[j] = src[min(lane + 64 * j, E - 1)];
  }
  return b;
}

__device__ __forceinline__ void topk_wave(const float* l, const TopkBias& bias, int E, int k,
                                          int mode, float eps, float scaling, int lane,
                                          int* idx_o, h16* w_o) {
  constexpr int NJ = 4;
  uint32_t key[NJ];
  float raw[NJ];  // sigmoid (mode >= 1) or logit (mode 0) of the candidate
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int e = lane + 64 * j;
    const bool ok = e < E;
    const float lv = ok ? l[e] : 0.f;
    float v = lv;
    if (mode >= 1 && ok) {
      v = sigmoid_f32(lv);
      raw[j] = v;
      if (bias.on) v = v + bias.v[j];
    } else {
      raw[j] = lv;
    }
    // every real key is above 0 (the key of -inf is 0x007fffff): absent
    // candidates (key 0) are never picked while k <= E
    key[j] = ok ? order_key(v) : 0u;
  }
  int my_e = -1;       // lane r < k: the r-th selected expert
  float my_raw = 0.f;  // and its raw value
  for (int r = 0; r < k; ++r) {  // uniform
    uint32_t m = key[0];
#pragma unroll
    for (int j = 1; j < NJ; ++j) m = max(m, key[j]);
    const uint32_t best = wave_max_u32(m);
    int we = 0x7fffffff;
    float wr = 0.f;
#pragma unroll
    for (int j = NJ - 1; j >= 0; --j) {  // the lowest register with a tie wins
      const uint64_t b = __ballot(key[j] == best);
      if (b) {  // uniform
        const int wl = __builtin_ctzll(b);
        we = wl + 64 * j;
        wr = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, raw[j]), wl));
      }
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      if (lane + 64 * j == we) key[j] = 0u;
    if (lane == r) {
      my_e = we;
      my_raw = wr;
    }
  }
  auto at = [&](int r) -> float {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_raw), r));
  };
  if (mode == 0) {
    // fp32 softmax over the selected logits, renormalised (as topk_small)
    const float mx = at(0);
    float z = 0.f;
    for (int r = 0; r < k; ++r) z += expf(at(r) - mx);
    float sum = 0.f;
    for (int r = 0; r < k; ++r) sum += expf(at(r) - mx) / z;
    if (lane < k) {
      idx_o[lane] = my_e;
      w_o[lane] = (h16)((expf(my_raw - mx) / z) / sum);
    }
  } else if (mode == 1) {
    float sum = 0.f;
    for (int r = 0; r < k; ++r) sum += at(r);
    const float d = sum + eps;
    if (lane < k) {
      idx_o[lane] = my_e;
      w_o[lane] = (h16)f32_mul(my_raw / d, scaling);
    }
  } else {
    if (lane < k) {
      idx_o[lane] = my_e;
      w_o[lane] = (h16)f32_mul(my_raw, scaling);
    }
  }
}

// Top-k of one token's row by one thread for E <= EB experts: every loop is
// unrolled over compile-time bounds, so the candidates, the selection and the
// selected logits stay in registers (the weights read no memory).  Same
// selection and weight arithmetic as topk_wave: mode 0, fp32 softmax over the
// selected logits (exp of x - max), renormalised, as
// F.softmax(topk_logits.float()); mode 1, sigmoid / (sum + eps) * scaling;
// mode 2, sigmoid * scaling; each sum in selection order.
template <int EB, int KB = kMaxTopK, int MODE = -1>
__device__ __forceinline__ void topk_small(const float* l, const float* bias, int E, int k,
                                           int mode_rt, float eps, float scaling, int* idx_o,
                                           h16* w_o) {
  const int mode = MODE >= 0 ? MODE : mode_rt;
  float lv[EB], cv[EB];
  bool ok[EB];
#pragma unroll
  for (int e = 0; e < EB; ++e) {
    ok[e] = e < E;
    lv[e] = ok[e] ? l[e] : 0.f;
    float v = lv[e];
    if (mode >= 1 && ok[e]) {
      v = sigmoid_f32(v);
      if (bias) v = v + bias[e];
    }
    cv[e] = v;
  }
  int sel[KB];
  float sr[KB];  // the selected experts' logits
#pragma unroll
  for (int i = 0; i < KB; ++i) {
    sel[i] = -1;
    sr[i] = 0.f;
    if (i < k) {
      float bv = -__builtin_inff(), br = 0.f;
      int be = 0x7fffffff;
#pragma unroll
      for (int e = 0; e < EB; ++e)
        if (ok[e] && topk_beats(cv[e], e, bv, be)) {
          bv = cv[e];
          be = e;
          br = lv[e];
        }
      sel[i] = be < E ? be : -1;
      sr[i] = br;
#pragma unroll
      for (int e = 0; e < EB; ++e)
        if (e == be) ok[e] = false;
    }
  }
#pragma unroll
  for (int i = 0; i < KB; ++i)
    if (i < k) idx_o[i] = sel[i];
  if (mode == 0) {
    const float mx = sr[0];
    float z = 0.f;
#pragma unroll
    for (int i = 0; i < KB; ++i)
      if (i < k) z += expf(sr[i] - mx);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < KB; ++i)
      if (i < k) s += expf(sr[i] - mx) / z;
#pragma unroll
    for (int i = 0; i < KB; ++i)
      if (i < k) w_o[i] = (h16)((expf(sr[i] - mx) / z) / s);
  } else if (mode == 1) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < KB; ++i)
      if (i < k) s += sigmoid_f32(sr[i]);
    const float d = s + eps;
#pragma unroll
    for (int i = 0; i < KB; ++i)
      if (i < k) w_o[i] = (h16)f32_mul(sigmoid_f32(sr[i]) / d, scaling);
  } else {
#pragma unroll
    for (int i = 0; i < KB; ++i)
      if (i < k) w_o[i] = (h16)f32_mul(sigmoid_f32(sr[i]), scaling);
  }
}

}  // namespace
