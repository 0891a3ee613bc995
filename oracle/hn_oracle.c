/*
 * TEST INFRASTRUCTURE ONLY — the CPU oracle for the INT4 expert-MLP path.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this; the product never does.
 *
 * Plain-C restatement of the reference's arithmetic (file:line cited per
 * function).  Floating-point is IEEE binary32 via SSE (x86-64, no fast-math),
 * fp16 conversion is written out from the IEEE-754 definition below.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---------------- fp16 <-> fp32 (IEEE-754 binary16, round to nearest even) */
static float h2f(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1f;
  const uint32_t m = h & 0x3ff;
  uint32_t x;
  if (e == 0) {
    if (m == 0) {
      x = sign;
    } else { /* subnormal: m * 2^-24, exact in float */
      float v = (float)m * (1.0f / 16777216.0f);
      memcpy(&x, &v, 4);
      x |= sign;
    }
  } else if (e == 31) {
    x = sign | 0x7f800000u | (m << 13);
  } else {
    x = sign | ((e - 15 + 127) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &x, 4);
  return f;
}

static uint16_t f2h(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t a = x & 0x7fffffffu;
  if (a >= 0x7f800000u) return sign | 0x7c00 | (a > 0x7f800000u ? 0x200 : 0);
  if (a >= 0x477ff000u) return sign | 0x7c00; /* >= 65520 rounds to inf */
  if (a < 0x38800000u) {                        /* below 2^-14: subnormal or 0 */
    float v;
    memcpy(&v, &a, 4);
    const float r = nearbyintf(v * 16777216.0f); /* units of 2^-24, RNE */
    return sign | (uint16_t)r;
  }
  uint32_t hbits = ((((a >> 23) - 127 + 15)) << 10) | ((a & 0x7fffffu) >> 13);
  const uint32_t rem = a & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (hbits & 1u))) hbits += 1;
  return sign | (uint16_t)hbits;
}

static float r16(float f) { return h2f(f2h(f)); }

void oracle_f32_to_f16(const float* in, uint16_t* out, long n) {
  for (long i = 0; i < n; ++i) out[i] = f2h(in[i]);
}
void oracle_f16_to_f32(const uint16_t* in, float* out, long n) {
  for (long i = 0; i < n; ++i) out[i] = h2f(in[i]);
}

/* ---------------- quantisers
 * mode 0: ExpertWeightPacker.quantize_tensor, preprocess/pack_weights.py:147-181
 *   absmax (:156), s = absmax / 7.0 in fp32 opmath rounded to fp16 (:157),
 *   clamp(min=1e-10) with the bound cast to fp16 (== 0) (:158),
 *   q = round(fp16(w / s)).clamp(-8, 7) (:161), +8 -> uint8 (:162),
 *   packed = (odd << 4) | even (:177-179).  NaN -> uint8 is 0 (x86 torch).
 * mode 1: Int4Linear.quantize_weight, kernels/int4_linear.py:84-107
 *   absmax.clamp(min=1e-8) in the weight dtype (:92), s = fp16(absmax / 7) (:94),
 *   q = round(T(T(w / absmax) * 7)).clamp(-8, 7) -> int8 (NaN -> 0) (:97),
 *   +8 -> uint8 (:98), packed = (even & 0xF) | ((odd & 0xF) << 4) (:105).
 * dtype 0: w is uint16 fp16 bits; dtype 1: w is float32.
 */
static float wload(const void* w, int dtype, long i) {
  return dtype == 0 ? h2f(((const uint16_t*)w)[i]) : ((const float*)w)[i];
}

void oracle_quantize(const void* w, int dtype, int mode, long N, long K, long group,
                     uint8_t* packed, uint16_t* scales) {
  const long G = K / group;
  for (long n = 0; n < N; ++n) {
    for (long g = 0; g < G; ++g) {
      const long base = n * K + g * group;
      float amax = 0.0f;
      int nan_seen = 0;
      for (long i = 0; i < group; ++i) {
        const float v = wload(w, dtype, base + i);
        if (v != v) nan_seen = 1;
        const float av = fabsf(v);
        if (av > amax) amax = av;
      }
      if (nan_seen) amax = NAN;
      float absmax_t;
      uint16_t s16;
      if (mode == 0) {
        absmax_t = amax;
        s16 = f2h(absmax_t / 7.0f);
      } else if (dtype == 0) {
        absmax_t = amax; /* clamp(min=fp16(1e-8) = 0) */
        s16 = f2h(absmax_t / 7.0f);
      } else {
        absmax_t = (amax > 1e-8f || amax != amax) ? amax : 1e-8f;
        s16 = f2h(absmax_t / 7.0f);
      }
      scales[n * G + g] = s16;
      const float s = h2f(s16);
      for (long i = 0; i < group; i += 2) {
        uint32_t code[2];
        for (int j = 0; j < 2; ++j) {
          const float v = wload(w, dtype, base + i + j);
          float q;
          if (mode == 0) q = r16(v / s);
          else if (dtype == 0) q = r16(r16(v / absmax_t) * 7.0f);
          else q = (v / absmax_t) * 7.0f;
          q = nearbyintf(q);
          if (q == q) q = q < -8.0f ? -8.0f : (q > 7.0f ? 7.0f : q);
          if (mode == 0) code[j] = (q == q) ? (uint32_t)(int)(q + 8.0f) & 0xffu : 0u;
          else code[j] = (uint32_t)(((q == q) ? (int)q : 0) + 8) & 0xffu;
        }
        packed[(n * K + g * group + i) / 2] = (uint8_t)(((code[1] << 4) | (code[0] & 0xfu)) & 0xffu);
      }
    }
  }
}

/* ---------------- dequant: preprocess/pack_weights.py:248-268,
 * cache/packed_expert_store.py:295-315, kernels/expert_mlp.py:313-330
 *   W[n, k] = fp16((nibble - 8) * scale[n, k / group])  (one rounding) */
void oracle_dequant(const uint8_t* packed, const uint16_t* scales, long N, long K, long group,
                    uint16_t* out) {
  const long G = K / group;
  for (long n = 0; n < N; ++n)
    for (long k = 0; k < K; ++k) {
      const uint8_t b = packed[n * (K / 2) + k / 2];
      const int nib = (k & 1) ? (b >> 4) : (b & 0xf);
      out[n * K + k] = f2h((float)(nib - 8) * h2f(scales[n * G + k / group]));
    }
}

/* ---------------- out[M, N] = fp16(x @ deq(W)^T), fp32 accumulation in k order
 * (kernels/int4_gemm.py:124-172 semantics) */
void oracle_int4_linear(const uint16_t* x, const uint8_t* packed, const uint16_t* scales, long M,
                        long N, long K, long group, uint16_t* out) {
  const long G = K / group;
  float* wf = (float*)malloc(sizeof(float) * K);
  for (long n = 0; n < N; ++n) {
    for (long k = 0; k < K; ++k) {
      const uint8_t b = packed[n * (K / 2) + k / 2];
      const int nib = (k & 1) ? (b >> 4) : (b & 0xf);
      wf[k] = r16((float)(nib - 8) * h2f(scales[n * G + k / group]));
    }
    for (long m = 0; m < M; ++m) {
      float acc = 0.0f;
      for (long k = 0; k < K; ++k) acc += h2f(x[m * K + k]) * wf[k];
      out[m * N + n] = f2h(acc);
    }
  }
  free(wf);
}

/* ---------------- router logits: fp16 gate Linear then .float() (model/router.py:102)
 * or fp32 F.linear(h.float(), W.float()) (model/glm4.py:279). */
void oracle_router_logits(const uint16_t* h, const void* w, int w_dtype, long T, long E, long H,
                          float* logits) {
  for (long t = 0; t < T; ++t)
    for (long e = 0; e < E; ++e) {
      float acc = 0.0f;
      for (long k = 0; k < H; ++k) acc += h2f(h[t * H + k]) * wload(w, w_dtype == 0 ? 0 : 1, e * H + k);
      logits[t * E + e] = w_dtype == 0 ? r16(acc) : acc;
    }
}

static float sigmoid_cr(float l) { return (float)(1.0 / (1.0 + exp(-(double)l))); }

/* ---------------- group-limited selection (model/glm4.py:285-298): group score
 * = max sigmoid over the group's E / n_group consecutive experts; the
 * topk_group largest groups are kept (equal scores: the lower group first);
 * out = logits with -inf (sigmoid 0, the masked score) outside them. */
void oracle_router_group_limit(const float* logits, long T, long E, long n_group,
                               long topk_group, float* out) {
  const long gs = E / n_group;
  float gsc[256];
  for (long t = 0; t < T; ++t) {
    const float* l = logits + t * E;
    for (long g = 0; g < n_group; ++g) {
      float m = -INFINITY;
      for (long j = 0; j < gs; ++j) {
        const float v = sigmoid_cr(l[g * gs + j]);
        if (v > m) m = v;
      }
      gsc[g] = m;
    }
    for (long g = 0; g < n_group; ++g) {
      long rank = 0;
      for (long o = 0; o < n_group; ++o)
        if (gsc[o] > gsc[g] || (gsc[o] == gsc[g] && o < g)) ++rank;
      for (long j = 0; j < gs; ++j)
        out[t * E + g * gs + j] = rank < topk_group ? l[g * gs + j] : -INFINITY;
    }
  }
}

/* ---------------- top-k
 * mode 0 (model/router.py:109-120): topk over logits (ties: lower index first),
 *   p = softmax(selected) in fp32, w = p / sum(p), fp16.
 * mode 1 (model/glm4.py:282-309): s = sigmoid(l); select by s + bias (bias may be
 *   NULL; a selection-only bias), w = s_sel / (sum + eps) * scaling, fp16.
 * mode 2 (norm_topk_prob=False, model/glm4.py:302-307): as mode 1, w = s_sel * scaling. */
void oracle_router_topk(const float* logits, const float* bias, long T, long E, long k, int mode,
                        float eps, float scaling, int32_t* idx_out, uint16_t* w_out) {
  float key[64];
  int sel[64];
  for (long t = 0; t < T; ++t) {
    const float* l = logits + t * E;
    int n = 0;
    for (int e = 0; e < E; ++e) {
      float v = l[e];
      if (mode >= 1) {
        v = sigmoid_cr(v);
        if (bias) v = v + bias[e];
      }
      if (n < k || v > key[n - 1]) {
        int p = (n < k) ? n : (int)k - 1;
        while (p > 0 && v > key[p - 1]) {
          key[p] = key[p - 1];
          sel[p] = sel[p - 1];
          --p;
        }
        key[p] = v;
        sel[p] = e;
        if (n < k) ++n;
      }
    }
    float wt[64];
    if (mode == 0) {
      const double mx = (double)l[sel[0]];
      double z = 0.0;
      for (int i = 0; i < n; ++i) z += exp((double)l[sel[i]] - mx);
      float s = 0.0f;
      for (int i = 0; i < n; ++i) {
        wt[i] = (float)(exp((double)l[sel[i]] - mx) / z);
        s += wt[i];
      }
      for (int i = 0; i < n; ++i) wt[i] = wt[i] / s;
    } else if (mode == 1) {
      float s = 0.0f;
      for (int i = 0; i < n; ++i) {
        wt[i] = sigmoid_cr(l[sel[i]]);
        s += wt[i];
      }
      const float d = s + eps;
      for (int i = 0; i < n; ++i) wt[i] = (wt[i] / d) * scaling;
    } else {
      for (int i = 0; i < n; ++i) wt[i] = sigmoid_cr(l[sel[i]]) * scaling;
    }
    for (int i = 0; i < k; ++i) {
      idx_out[t * k + i] = i < n ? sel[i] : -1;
      w_out[t * k + i] = i < n ? f2h(wt[i]) : 0;
    }
  }
}

/* ---------------- permute: stable sort of flattened assignments by expert
 * (model/mixtral.py:296, :333 — unique() ascending, torch.where row-major). */
void oracle_moe_permute(const int32_t* idx, long n, long E, int32_t* offsets, int32_t* perm,
                        int32_t* inv, int32_t* active, int32_t* n_active) {
  long* cnt = (long*)calloc((size_t)E + 1, sizeof(long));
  for (long j = 0; j < n; ++j)
    if (idx[j] >= 0 && idx[j] < E) cnt[idx[j]]++;
  long acc = 0;
  int na = 0;
  for (long e = 0; e < E; ++e) {
    offsets[e] = (int32_t)acc;
    if (cnt[e] > 0) active[na++] = (int32_t)e;
    acc += cnt[e];
  }
  offsets[E] = (int32_t)acc;
  *n_active = na;
  long* fill = (long*)calloc((size_t)E + 1, sizeof(long));
  for (long j = 0; j < n; ++j) {
    const int e = idx[j];
    if (e < 0 || e >= E) {
      inv[j] = -1;
      continue;
    }
    const long p = offsets[e] + fill[e]++;
    perm[p] = (int32_t)j;
    inv[j] = (int32_t)p;
  }
  free(cnt);
  free(fill);
}

/* ---------------- unpermute: out = zeros fp16; for experts in ascending order:
 * out[t] += fp16(y * w) with fp16 rounding per add (model/mixtral.py:299, :365-368);
 * optional out = fp16(shared + out) (model/glm4.py:473). */
void oracle_moe_unpermute(const uint16_t* y_perm, const int32_t* inv, const int32_t* idx,
                          const uint16_t* w, long T, long k, const uint16_t* shared, long H,
                          uint16_t* out) {
  for (long t = 0; t < T; ++t) {
    int ord[64];
    int n = 0;
    for (int s = 0; s < k; ++s) {
      if (inv[t * k + s] < 0) continue;
      int q = n;
      while (q > 0 && idx[t * k + ord[q - 1]] > idx[t * k + s]) {
        ord[q] = ord[q - 1];
        --q;
      }
      ord[q] = s;
      ++n;
    }
    for (long c = 0; c < H; ++c) {
      float acc = 0.0f;
      for (int i = 0; i < n; ++i) {
        const long j = t * k + ord[i];
        const float prod = r16(h2f(y_perm[(long)inv[j] * H + c]) * h2f(w[j]));
        acc = r16(acc + prod);
      }
      if (shared) acc = r16(h2f(shared[t * H + c]) + acc);
      out[t * H + c] = f2h(acc);
    }
  }
}
