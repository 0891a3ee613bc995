// The ordered, weighted sum of one token's expert outputs (the MoE layer's
// unpermute), shared by moe_unpermute_kernel (hn_route.hip) and the fused
// unpermute + residual add + RMSNorm of the decoder (hn_decoder.hip), so both
// give the same bits.
//
// Reference arithmetic (model/mixtral.py:327-368): the experts a token was
// routed to are visited in ascending expert id (torch.unique order); each
// expert's output row y is scaled by its routing weight in fp16 and added
// into an fp16 accumulator: acc = fp16(acc + fp16(y * w)).
#pragma once
#include "hn_common.h"
#include "hn_topk.h"

// The token's assignments (position in the permuted rows, expert, weight)
// sorted by expert id; returns their number (assignments with inv < 0 are
// dropped).  Loads are unconditional (index clamped to k - 1): a load under
// `if (s < k)` ends its own block, and the compiler then waits for each in
// turn.
__device__ __forceinline__ int unp_select(int t, const int* __restrict__ inv,
                                          const int* __restrict__ idx,
                                          const h16* __restrict__ w, int k,
                                          int pos[kMaxTopK], float wt[kMaxTopK]) {
  int ex[kMaxTopK];
  int pv[kMaxTopK], ev[kMaxTopK];
  h16 wv[kMaxTopK];
#pragma unroll
  for (int s = 0; s < kMaxTopK; ++s) {
    const int j = t * k + (s < k ? s : k - 1);
    pv[s] = inv[j];
    ev[s] = idx[j];
    wv[s] = w[j];
  }
  int n = 0;
#pragma unroll
  for (int s = 0; s < kMaxTopK; ++s) {
    if (s >= k) break;
    const int p = pv[s];
    if (p < 0) continue;
    const int e = ev[s];
    // insertion by expert id (ascending)
    int q = n;
    while (q > 0 && ex[q - 1] > e) {
      ex[q] = ex[q - 1];
      pos[q] = pos[q - 1];
      wt[q] = wt[q - 1];
      --q;
    }
    ex[q] = e;
    pos[q] = p;
    wt[q] = (float)wv[s];
    ++n;
  }
  return n;
}

// Columns c .. c + 7 of the token's weighted sum over its n sorted
// assignments.  KS = 0: y is fp16 [rows, ld_y]; KS > 0: y is given as KS fp32
// partial sums part[j * ks_stride + row * ld_y] (a K-split down
// projection), added in slice order and rounded to fp16 once.  The rows of a
// batch of B assignments are loaded before any is used.
template <int KS>
__device__ __forceinline__ half8_t unp_cols(const h16* __restrict__ y,
                                            const float* __restrict__ part, long ks_stride,
                                            long ld_y, const int pos[kMaxTopK],
                                            const float wt[kMaxTopK], int n, int c) {
  constexpr int B = KS == 0 ? 8 : 2;
  half8_t acc = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int s0 = 0; s0 < n; s0 += B) {
    half8_t v[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int s = s0 + u < n ? s0 + u : n - 1;
      if constexpr (KS == 0) {
        v[u] = *reinterpret_cast<const half8_t*>(y + (long)pos[s] * ld_y + c);
      } else {
        float f[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) f[q] = 0.f;
#pragma unroll
        for (int j = 0; j < KS; ++j) {
          const float* pp = part + j * ks_stride + (long)pos[s] * ld_y + c;
          const float4_t a = *reinterpret_cast<const float4_t*>(pp);
          const float4_t b = *reinterpret_cast<const float4_t*>(pp + 4);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            f[q] += a[q];
            f[4 + q] += b[q];
          }
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) v[u][q] = (h16)f[q];
      }
    }
#pragma unroll
    for (int u = 0; u < B; ++u) {
      if (s0 + u >= n) break;
      const float ws = wt[s0 + u];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const h16 prod = (h16)((float)v[u][j] * ws);
        acc[j] = (h16)((float)acc[j] + (float)prod);
      }
    }
  }
  return acc;
}
