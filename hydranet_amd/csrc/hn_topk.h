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
__device__ __noinline__ void topk_weights(const float* l, const int* sel, int k, int mode,
                                          float eps, float scaling, h16* w_o) {
  if (mode == 0) {
    // fp32 softmax as F.softmax(topk_logits.float()) (exp of x - max)
    const float mx = l[sel[0]];
    float z = 0.f;
#pragma unroll 1
    for (int i = 0; i < k; ++i) z += expf(l[sel[i]] - mx);
    float s = 0.f;
#pragma unroll 1
    for (int i = 0; i < k; ++i) s += expf(l[sel[i]] - mx) / z;
#pragma unroll 1
    for (int i = 0; i < k; ++i) w_o[i] = (h16)((expf(l[sel[i]] - mx) / z) / s);
  } else if (mode == 1) {
    float s = 0.f;
#pragma unroll 1
    for (int i = 0; i < k; ++i) s += sigmoid_f32(l[sel[i]]);
    const float d = s + eps;
#pragma unroll 1
    for (int i = 0; i < k; ++i) w_o[i] = (h16)f32_mul(sigmoid_f32(l[sel[i]]) / d, scaling);
  } else {
#pragma unroll 1
    for (int i = 0; i < k; ++i) w_o[i] = (h16)f32_mul(sigmoid_f32(l[sel[i]]), scaling);
  }
}

// Unsigned key with the order of the float: larger value, larger key.
__device__ __forceinline__ uint32_t order_key(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Top-k of one token's logits row by one wave: lanes hold experts lane +
// 64 j (E <= 256).  The k-th largest candidate key is found by bisection over
// its 32 bits (one ballot per bit and candidate register: no lane exchanges),
// ties at that key go to the lower experts.  The selected candidates (at most
// k <= 16) are then moved to lanes 0..k-1 in expert order (ds_permute to
// their rank among the selected), each finds its place in the (value desc,
// expert asc) order against the others (readlane over the k lanes), and a
// second ds_permute puts them in selection order, so the weight sums read
// lane p for the p-th selected.  Same selection and weight arithmetic as
// topk_small / topk_weights: the sums over the selected experts run in
// selection order.
__device__ __forceinline__ void topk_wave(const float* l, const float* bias, int E, int k,
                                          int mode, float eps, float scaling, int lane,
                                          int* idx_o, h16* w_o) {
  constexpr int NJ = 4;
  const uint64_t lt = (1ull << lane) - 1;
  uint32_t key[NJ];
  float raw[NJ];  // sigmoid (mode 1) or logit (mode 0) of the candidate
  bool ok[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int e = lane + 64 * j;
    ok[j] = e < E;
    const float lv = ok[j] ? l[e] : 0.f;
    float v = lv;
    if (mode >= 1 && ok[j]) {
      v = sigmoid_f32(lv);
      raw[j] = v;
      if (bias) v = v + bias[e];
    } else {
      raw[j] = lv;
    }
    key[j] = ok[j] ? order_key(v) : 0u;
  }
  // Largest t with at least k candidates of key >= t.  Every real key is
  // above 0 (the key of -inf is 0x007fffff) and the thresholds tried are >= 1,
  // so the zero keys of absent candidates never count: no per-register
  // conditions, no branches in the 32 steps.
  uint32_t t = 0;
#pragma unroll
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t c = t | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < NJ; ++j) cnt += __popcll(__ballot(key[j] >= c));
    t = cnt >= k ? c : t;
  }
  bool sel[NJ];
  int above = 0;
#pragma unroll
  for (int j = 0; j < NJ; ++j) above += __popcll(__ballot(key[j] > t));
  int tie = 0;  // ties at t in expert order until k are selected
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const bool eq = key[j] == t;
    const uint64_t m = __ballot(eq);
    sel[j] = key[j] > t || (eq && above + tie + __popcll(m & lt) < k);
    tie += __popcll(m);
  }
  // 1. the selected to lanes 0..ns-1 in expert order: the candidate of rank
  //    r among the selected sends (key, expert, raw) to lane r; the others
  //    send to lane 63 (>= 16 > ns), whose values are never read
  int ns = 0;
  uint32_t ck = 0u;
  int ce = 0;
  float cr = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const uint64_t m = __ballot(sel[j]);
    const int cnt = __popcll(m);
    if (cnt) {  // uniform
      const int dst = 4 * (sel[j] ? ns + __popcll(m & lt) : 63);
      const uint32_t pk = (uint32_t)__builtin_amdgcn_ds_permute(dst, (int)key[j]);
      const int pe = __builtin_amdgcn_ds_permute(dst, lane + 64 * j);
      const float pr =
          __builtin_bit_cast(float, __builtin_amdgcn_ds_permute(dst, __builtin_bit_cast(int, raw[j])));
      if (lane >= ns && lane < ns + cnt) {
        ck = pk;
        ce = pe;
        cr = pr;
      }
      ns += cnt;
    }
  }
  // 2. place of lane r's candidate: selected candidates ahead of it (a larger
  //    key, or an equal key and a lower expert = a lower lane)
  int pos = 0;
#pragma unroll
  for (int s = 0; s < kMaxTopK; ++s) {
    if (s < ns) {  // uniform
      const uint32_t ks = (uint32_t)__builtin_amdgcn_readlane((int)ck, s);
      pos += (ks > ck || (ks == ck && s < lane)) ? 1 : 0;
    }
  }
  // 3. lane p holds the p-th selected (expert, raw)
  const int dst = 4 * (lane < ns ? pos : 63);
  const int oe = __builtin_amdgcn_ds_permute(dst, ce);
  const float orr = __builtin_bit_cast(float, __builtin_amdgcn_ds_permute(dst, __builtin_bit_cast(int, cr)));
  auto at = [&](int r) -> float {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, orr), r));
  };
  if (mode == 0) {
    // fp32 softmax over the selected logits, renormalised (topk_weights)
    const float mx = at(0);
    float z = 0.f;
    for (int r = 0; r < ns; ++r) z += expf(at(r) - mx);
    float sum = 0.f;
    for (int r = 0; r < ns; ++r) sum += expf(at(r) - mx) / z;
    if (lane < ns) {
      idx_o[lane] = oe;
      w_o[lane] = (h16)((expf(orr - mx) / z) / sum);
    }
  } else if (mode == 1) {
    float sum = 0.f;
    for (int r = 0; r < ns; ++r) sum += at(r);
    const float d = sum + eps;
    if (lane < ns) {
      idx_o[lane] = oe;
      w_o[lane] = (h16)f32_mul(orr / d, scaling);
    }
  } else {
    if (lane < ns) {
      idx_o[lane] = oe;
      w_o[lane] = (h16)f32_mul(orr, scaling);
    }
  }
}

// Top-k of one token's row by one thread for E <= EB experts: every loop is
// unrolled over compile-time bounds, so the candidates and the selection
// stay in registers.  Same selection and weight arithmetic as topk_wave.
template <int EB, int KB = kMaxTopK, int MODE = -1>
__device__ __forceinline__ void topk_small(const float* l, const float* bias, int E, int k,
                                           int mode_rt, float eps, float scaling, int* idx_o,
                                           h16* w_o) {
  const int mode = MODE >= 0 ? MODE : mode_rt;
  float cv[EB];
  bool ok[EB];
#pragma unroll
  for (int e = 0; e < EB; ++e) {
    ok[e] = e < E;
    float v = ok[e] ? l[e] : 0.f;
    if (mode >= 1 && ok[e]) {
      v = sigmoid_f32(v);
      if (bias) v = v + bias[e];
    }
    cv[e] = v;
  }
  int sel[KB];
#pragma unroll
  for (int i = 0; i < KB; ++i) {
    sel[i] = -1;
    if (i < k) {
      float bv = -__builtin_inff();
      int be = 0x7fffffff;
#pragma unroll
      for (int e = 0; e < EB; ++e)
        if (ok[e] && topk_beats(cv[e], e, bv, be)) { bv = cv[e]; be = e; }
      sel[i] = be < E ? be : -1;
#pragma unroll
      for (int e = 0; e < EB; ++e)
        if (e == be) ok[e] = false;
    }
  }
#pragma unroll
  for (int i = 0; i < KB; ++i)
    if (i < k) idx_o[i] = sel[i];
  topk_weights(l, idx_o, k, mode, eps, scaling, w_o);
}

}  // namespace
