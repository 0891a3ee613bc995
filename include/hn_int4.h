/*
 * hn_int4.h — C ABI of libhn_int4.so, the gfx950 INT4 expert-MLP hot path.
 *
 * Conventions
 *  - Every pointer argument is a device pointer unless stated otherwise; the
 *    library never allocates, frees or retains them.  Workspaces are passed in.
 *  - fp16 data is IEEE binary16 ("half"); packed weights are uint8 with two
 *    nibbles per byte (low nibble = even k), stored as q + 8, q in [-8, 7];
 *    scales are fp16, one per (row, group of `group` consecutive k).
 *  - ld_* arguments are row strides: bytes for packed weights, elements for
 *    everything else.  Inner dimensions are contiguous.
 *  - `stream` is a hipStream_t (e.g. torch.cuda.current_stream().cuda_stream);
 *    every call only enqueues work on it.
 *  - Return value: 0 on success, a negative errno-style code for a rejected
 *    argument, or a positive hipError_t from the launch.  The message is in
 *    hn_last_error_string() (thread-local).
 */
#ifndef HN_INT4_H
#define HN_INT4_H

#ifdef __cplusplus
extern "C" {
#endif

const char* hn_last_error_string(void);
int hn_abi_version(void);

/* Dequantise packed[N, K/2] + scales[N, K/group] into out[N, K] fp16, bit-exact
 * with fp16((nibble - 8) * scale).  Replaces GpuExpertSlot._dequant_tensor
 * (cache/packed_expert_store.py:287-315), ExpertWeightPacker.dequantize_tensor
 * (preprocess/pack_weights.py:230-268), ExpertMLPTriton._dequant
 * (kernels/expert_mlp.py:305-330).  K % 32 == 0. */
int hn_int4_dequant(const void* packed, long ld_p, const void* scales, long ld_s, void* out,
                    long ld_o, long N, long K, long group, void* stream);

/* Quantise w[N, K] (dtype 0 = fp16, 1 = fp32) into packed/scales.
 * mode 0 = ExpertWeightPacker.quantize_tensor (preprocess/pack_weights.py:133-181),
 * mode 1 = Int4Linear.quantize_weight (kernels/int4_linear.py:68-107). */
int hn_int4_quantize(const void* w, long ld_w, int dtype, int mode, void* packed, long ld_p,
                     void* scales, long ld_s, long N, long K, long group, void* stream);

/* Workspace bytes for the skinny (decode) kernels below.  kind 0: hn_int4_linear
 * (M, N, K); 1: hn_int4_gate_up_silu (M, N=I, K=H); 2: hn_expert_mlp_int4
 * (M=T, N=H, K=I); 3: hn_grouped_expert_mlp_int4 (M=rows, N=H, K=I, E).  The
 * workspace must be zero-filled once when allocated; the kernels leave its
 * counters at zero.  Its layout (counters in the first 2 MiB, partials after)
 * is the same for every call, so one buffer may serve calls of every kind and
 * size in turn.  Calls that run concurrently need distinct workspaces.
 * No counterpart in the reference (Triton needs no split-K workspace). */
long hn_skinny_workspace_bytes(int kind, long M, long N, long K, long E);

/* Workspace bytes of the prefill (MFMA GEMM) kernels' stream-K split: fp32
 * partial slots for two tile segments per workgroup plus per-(tile, wave)
 * counters.  Passed (zero-filled once; the kernels leave the counters at zero)
 * as the work argument of the entry points below at prefill sizes, it lets
 * the tiles short of a whole round over the CUs (and the experts' last,
 * shorter M-tiles) be split over every CU by cost-weighted (tile, k-chunk)
 * iterations, tiles split at the shares' ends being summed in a fixed order
 * by the last segment to finish.  No counterpart in the reference (Triton's
 * GEMM takes no workspace). */
long hn_gemm_workspace_bytes(void);

/* out[M, N] = fp16(x[M, K] @ deq(W)^T), fp32 accumulation.  Replaces the
 * int4_matmul_kernel launch in int4_gemm.int4_linear (kernels/int4_gemm.py:124-172)
 * and int4_expert_mlp.int4_linear (kernels/int4_expert_mlp.py:99-156).
 * K % 32 == 0, group a multiple of 32 dividing K, 16-byte aligned rows. */
int hn_int4_linear(const void* x, long ld_x, const void* wq, long ld_q, const void* ws, long ld_s,
                   void* out, long ld_o, long M, long N, long K, long group, void* work,
                   long work_bytes, void* stream);

/* h[M, N] = fp16(silu(fp16(x @ deq(Wg)^T)) * fp16(x @ deq(Wu)^T)): the gate and up
 * projections of expert_mlp_int4_fused plus fused_silu_mul
 * (kernels/int4_gemm.py:175-208, 241-247) in one launch. */
int hn_int4_gate_up_silu(const void* x, long ld_x, const void* gq, const void* gs, const void* uq,
                         const void* us, long ld_q, long ld_s, void* h, long ld_h, long M, long N,
                         long K, long group, void* work, long work_bytes, void* stream);

/* out[T, H] = down(silu(gate(x)) * up(x)) for one expert; h_ws is a [T, I] fp16
 * workspace.  Replaces int4_gemm.expert_mlp_int4_fused (kernels/int4_gemm.py:211-254)
 * and int4_expert_mlp.expert_mlp_int4 (kernels/int4_expert_mlp.py:213-252). */
int hn_expert_mlp_int4(const void* x, const void* gq, const void* gs, const void* uq,
                       const void* us, const void* dq, const void* ds, void* out, long T, long H,
                       long I, long group, void* h_ws, void* work, long work_bytes,
                       void* stream);

/* out = fp16(silu(float(g)) * float(u)).  Replaces fused_silu_mul / silu_mul
 * (kernels/int4_gemm.py:196-208, kernels/int4_expert_mlp.py:189-210). */
int hn_silu_mul(const void* g, long ld_g, const void* u, long ld_u, void* out, long ld_o, long M,
                long N, void* stream);

/* out = fp16(float(fp16(silu(float(g)))) * float(u)): the two fp16 operations
 * of act_fn(gate_proj(x)) * up_proj(x) in one launch.  Replaces the SiLU and
 * the product of GLM4DenseMLP.forward (model/glm4.py:232-233). */
int hn_silu_then_mul(const void* g, long ld_g, const void* u, long ld_u, void* out, long ld_o,
                     long M, long N, void* stream);

/* logits[T, E] fp32 = h[T, H] @ W^T.  w_dtype 0: fp16 gate, logits rounded to fp16
 * (TopKRouter.gate(...).float(), model/router.py:102); w_dtype 1: fp32 weight
 * (GLM4SigmoidRouter, model/glm4.py:279). */
int hn_router_logits(const void* h, long ld_h, const void* w, long ld_w, int w_dtype,
                     void* logits, long T, long E, long H, void* stream);

/* Top-k routing from fp32 logits.  mode 0: softmax over the selected logits and
 * renormalise (model/router.py:109-120); mode 1: sigmoid, optional selection-only
 * bias[E] (may be NULL), weights / (sum + eps) * scaling (model/glm4.py:282-309);
 * mode 2: as mode 1 without the normalisation, weights = sigmoid * scaling
 * (norm_topk_prob=False, model/glm4.py:302-307).
 * Ties go to the lower expert index.  idx_out int32 [T, k], w_out fp16 [T, k]. */
int hn_router_topk(const void* logits, const void* bias, long T, long E, long k, int mode,
                   float eps, float scaling, int* idx_out, void* w_out, void* stream);

/* Group-limited selection of GLM4SigmoidRouter.forward (model/glm4.py:285-298):
 * out[T, E] fp32 = logits, with -inf for every expert outside the token's
 * topk_group groups of largest max-sigmoid (groups = n_group runs of E/n_group
 * consecutive experts; equal group scores: the lower group).  A -inf logit has
 * sigmoid 0, the reference's masked score; hn_router_topk mode 1/2 then
 * selects from out.  n_group | E, n_group <= 64, E <= 256; out may equal logits. */
int hn_router_group_limit(const void* logits, long T, long E, long n_group, long topk_group,
                          void* out, void* stream);

/* Stable counting sort of the [T*k] assignments by expert (the per-expert
 * torch.where loop of MixtralMoELayer.forward, model/mixtral.py:296-338).
 * offsets[E+1], perm[T*k] (sorted position -> assignment), inv[T*k]
 * (assignment -> sorted position), active[E] (experts with tokens, ascending),
 * n_active[1].  E <= 256. */
int hn_moe_permute(const int* idx, long T, long k, long E, int* offsets, int* perm, int* inv,
                   int* active, int* n_active, void* stream);

/* x_perm[p] = x[perm[p] / k] for p < offsets[E] (flat_hidden[token_indices],
 * model/mixtral.py:338).  rows = grid bound (T*k). */
int hn_moe_gather(const void* x, long ld_x, const int* perm, long k, const int* offsets, long E,
                  void* x_perm, long ld_p, long rows, long H, void* stream);

/* Decode routing in one launch: logits (w_dtype as hn_router_logits; skipped
 * when logits_in [T, E] fp32 is given), top-k (mode, bias, eps, scaling as
 * hn_router_topk), the stable permutation (as hn_moe_permute) and the gather
 * x_perm [T*k, H] (as hn_moe_gather); logits_out may be NULL.  Every
 * workgroup repeats the routing of all T tokens and copies a share of the
 * rows, so the outputs equal those of the four separate kernels.
 * T*E <= 8192, T*k <= 1024, E <= 256.  usage (may be NULL): int64 [E]
 * counters to which the call adds each expert's routed rows (TopKRouter's
 * usage counts, model/router.py:123-124).  Replaces TopKRouter.forward
 * (model/router.py:96-120) or GLM4SigmoidRouter.forward (model/glm4.py:275-309)
 * plus the unique()/where()/gather steps of MixtralMoELayer.forward
 * (model/mixtral.py:296-338) at decode sizes. */
int hn_moe_route(const void* h, long ld_h, const void* w, long ld_w, int w_dtype,
                 const void* logits_in, const void* bias, long T, long E, long H, long k,
                 int mode, float eps, float scaling, void* logits_out, int* idx_out,
                 void* w_out, int* offsets, int* perm, int* inv, int* active, int* n_active,
                 long long* usage, void* x_perm, long ld_p, void* stream);

/* out[T, H] = (shared +) sum over the token's experts (ascending id) of
 * fp16(y_perm[inv[t*k+s]] * w[t, s]) with fp16 accumulation: output.index_add_
 * (model/mixtral.py:365-368) and shared + routed (model/glm4.py:473). */
int hn_moe_unpermute(const void* y_perm, long ld_y, const int* inv, const int* idx, const void* w,
                     long T, long k, const void* shared, long ld_sh, void* out, long ld_o, long H,
                     void* stream);

/* Grouped SwiGLU over every active expert of one MoE layer in two launches:
 * the decode kernels up to 64 rows per expert, the MFMA GEMM kernels above
 * (which take no workspace: it may then be NULL / 0 bytes).  x_perm [rows, H] sorted by expert; table: E x
 * {gate_q, gate_s, up_q, up_s, down_q, down_s} device pointers (u64), each
 * 16-byte aligned (GpuExpertSlot slabs are); active /
 * n_active / offsets from hn_moe_permute; h_ws [rows, I] fp16 buffer;
 * y_perm [rows, H] fp16 out; work: hn_skinny_workspace_bytes(3, rows, H, I, E),
 * zero-filled once.  Above 64 rows per expert (the MFMA GEMM kernels) work
 * may instead hold hn_gemm_workspace_bytes() bytes, which enables their
 * stream-K split of the remainder tiles over the CUs, or be NULL (whole
 * tiles go round-robin).
 * Replaces the per-expert loop calling expert_mlp_int4_fused
 * (model/mixtral.py:327-354, model/glm4.py:421-455). */
int hn_grouped_expert_mlp_int4(const void* x_perm, const void* table, const int* active,
                               const int* n_active, const int* offsets, long E,
                               long max_rows_per_expert, long rows, long H, long I, long group,
                               void* h_ws, void* y_perm, void* work, long work_bytes,
                               void* stream);

/* The experts half of a MoE layer at decode: hn_grouped_expert_mlp_int4 plus
 * hn_moe_unpermute (same arguments; inv / idx / w / shared as for
 * hn_moe_unpermute, out [T, H]).  Where the streaming kernels apply, the down
 * projection runs in four K slices whose fp32 partials (kept in work) the
 * unpermute adds in slice order before the fp16 rounding; y_ws [rows, H] fp16
 * is then unused.  work: hn_skinny_workspace_bytes(3, rows, H, I, E).  out
 * NULL (only on that streaming path, hn_moe_experts_decode_split_check, and
 * without a shared expert): no unpermute; the partials stay in work at byte
 * hn_moe_decode_layer_partials(T, E, k, H, I) for the caller (e.g.
 * hn_unpermute_add_rmsnorm).
 * Replaces the per-expert loop and index_add_ of MixtralMoELayer.forward
 * (model/mixtral.py:327-368) / GLM4MoELayer.forward (model/glm4.py:421-473). */
int hn_moe_experts_decode(const void* x_perm, const void* table, const int* active,
                          const int* n_active, const int* offsets, long E,
                          long max_rows_per_expert, long rows, long H, long I, long group,
                          void* h_ws, void* y_ws, const int* inv, const int* idx, const void* w,
                          long T, long k, const void* shared, long ld_sh, void* out, long ld_o,
                          void* work, long work_bytes, void* stream);

/* 0 when hn_moe_experts_decode takes its streaming path with the K-split down
 * projection for (E, max_rows_per_expert, rows, H, I, group) under the current
 * decode kernel family (then out may be NULL), else a nonzero code (no
 * message set). */
int hn_moe_experts_decode_split_check(long E, long max_rows_per_expert, long rows, long H,
                                      long I, long group);

/* The first launch of hn_moe_decode_layer alone: the routing computed in the
 * grouped gate/up streaming kernel and h_ws [T k, I] = fp16(silu(fp16(x Wg^T))
 * * fp16(x Wu^T)) for the routed rows (same arguments; for per-kernel timing
 * and counter runs).  Replaces TopKRouter.forward and the gate/up half of the
 * per-expert loop (model/router.py:96-120, model/mixtral.py:327-354). */
int hn_moe_route_gate_up(const void* h, long ld_h, const void* gate_w, long ld_w,
                         const float* logits_in, long T, long E, long k, const void* table,
                         long H, long I, long group, float eps, float scaling, void* logits_out,
                         int* idx, void* w, int* offsets, int* perm, int* inv, int* active,
                         int* n_active, long long* usage, void* h_ws, void* stream);

/* 0 when hn_moe_decode_layer covers (T, E, k, H, I, group) with the current
 * decode kernel family, else a nonzero code (no error message is set).
 * has_logits: whether the call will pass logits_in. */
int hn_moe_decode_layer_check(long T, long E, long k, long H, long I, long group,
                              int has_logits);

/* One Mixtral MoE layer at decode (E <= 8 experts, softmax top-k with k 1 or
 * 2 and T k <= 64, group 128, H and I multiples of 512) in three launches:
 * the routing (top-k, stable permutation) computed inside the gate/up
 * streaming kernel from h [T, H] directly (no x_perm), the down projection in
 * four K slices, the ordered weighted unpermute into out [T, H].  The router
 * logits are either computed there from the fp16 gate [E, H] (T <= 16) or
 * given in logits_in [T, E] fp32 (fp16 values, e.g. from
 * hn_add_rmsnorm_router; gate_w may then be NULL).  Results equal
 * hn_moe_route + hn_moe_experts_decode; the routing outputs (logits_out may be
 * NULL, idx, w, offsets [E + 1], perm, inv, active, n_active, usage) are
 * written as hn_moe_route writes them.  h_ws [T k, I] fp16; work:
 * hn_skinny_workspace_bytes(3, T k, H, I, E).  out NULL: no unpermute; the
 * down projection's four fp32 K-slice partials stay in work at byte
 * hn_moe_decode_layer_partials(T, E, k, H, I) for the caller (e.g.
 * hn_unpermute_add_rmsnorm).  Replaces MixtralMoELayer.forward's router
 * call, per-expert loop and index_add_ (model/mixtral.py:283-368) at decode
 * sizes. */
int hn_moe_decode_layer(const void* h, long ld_h, const void* gate_w, long ld_w,
                        const float* logits_in, long T, long E, long k, const void* table,
                        long H, long I, long group, float eps, float scaling, void* logits_out,
                        int* idx, void* w, int* offsets, int* perm, int* inv, int* active,
                        int* n_active, long long* usage, void* h_ws, void* out, long ld_o,
                        void* work, long work_bytes, void* stream);

/* Byte offset in the workspace of hn_moe_decode_layer (and of
 * hn_moe_experts_decode with rows = T k on its split path) of the down
 * projection's four fp32 K-slice partials [4][T k][H] (slice stride T k H
 * floats). */
long hn_moe_decode_layer_partials(long T, long E, long k, long H, long I);

/* 0 when hn_moe_route_experts_decode covers (T, E, k, mode, H, I, group) with
 * the current decode kernel family, else a nonzero code (no message set). */
int hn_moe_route_experts_decode_check(long T, long E, long k, int mode, long H, long I,
                                      long group);

/* A decode MoE layer from given router logits [T, E] fp32 (e.g. hn_router_logits,
 * after hn_router_group_limit) in three launches: the top-k (mode 0 softmax,
 * 1 sigmoid / (sum + eps) * scaling, 2 sigmoid * scaling; optional selection
 * bias [E]) and the stable permutation computed inside the grouped gate/up
 * streaming kernel, whose rows are staged from h [T, H] directly (no x_perm);
 * the down projection (into y_ws [T k, H], or four fp32 K slices in work when
 * I splits); the ordered weighted unpermute into out [T, H], plus the fp16
 * shared addend [T, H] when given (GLM's shared expert).  shared_ready: a
 * hipEvent_t (may be NULL) the stream waits for just before the unpermute,
 * so a shared expert computed on another stream overlaps the expert kernels.
 * E <= 256, k <= 16, T k <= 64 x the gate/up launch's waves (512 at H = 4096),
 * H % 512 == 0, group 128.  Routing outputs as hn_moe_route writes them
 * (usage may be NULL); h_ws [T k, I]; work: hn_skinny_workspace_bytes(3, T k,
 * H, I, E).  Replaces GLM4MoELayer.forward's router call, per-expert loop and
 * shared + routed sum (model/glm4.py:275-309, 421-473) at decode sizes. */
int hn_moe_route_experts_decode(const float* logits, const void* bias, long T, long E, long k,
                                int mode, float eps, float scaling, const void* h, long ld_h,
                                const void* table, long H, long I, long group, int* idx, void* w,
                                int* offsets, int* perm, int* inv, int* active, int* n_active,
                                long long* usage, void* h_ws, void* y_ws, void* shared_ready,
                                const void* shared, long ld_sh, void* out, long ld_o, void* work,
                                long work_bytes, void* stream);

/* One phase of hn_moe_experts_decode's streaming path on its own (<= 16 rows per
 * expert, group 128): phase 0 reads x [rows, H] (sorted by expert) and writes
 * h_ws [rows, I]; phase 1 reads h_ws-shaped x [rows, I] and writes the four
 * fp32 K-slice partials of the down projection into work (after its counter
 * region, part[j][row][H]).  No separate counterpart in the reference; lets a
 * caller time the two decode phases apart (the benchmark's roofline). */
int hn_grouped_decode_phase_int4(int phase, const void* x, const void* table, const int* active,
                                 const int* n_active, const int* offsets, long E,
                                 long max_rows_per_expert, long rows, long H, long I, long group,
                                 void* h_ws, void* work, long work_bytes, void* stream);

/* One phase of hn_grouped_expert_mlp_int4's prefill path (the grouped MFMA GEMM):
 * phase 0 writes h_ws [rows, I] = fp16(silu(fp16(x Wg^T)) * fp16(x Wu^T)) per expert,
 * phase 1 writes y_perm [rows, H] = fp16(h_ws Wd^T) per expert.  Any rows per
 * expert; E <= 256; H, I multiples of 128; group 32 or a multiple of 64.
 * work (may be NULL / 0): with hn_gemm_workspace_bytes() bytes, zero-filled
 * once, the k-stages are split evenly over
 * the CUs (stream-K; tiles split at the shares' ends are summed in a fixed
 * order); without, whole tiles go round-robin.  Calls that run concurrently
 * need distinct workspaces.
 * No separate counterpart in the reference (its loop calls
 * expert_mlp_int4_fused per expert, model/mixtral.py:342-354); lets a caller
 * time or schedule the two phases apart. */
int hn_grouped_expert_phase_int4(int phase, const void* x_perm, const void* table,
                                 const int* active, const int* n_active, const int* offsets,
                                 long E, long rows, long H, long I, long group, void* h_ws,
                                 void* y_perm, void* work, long work_bytes, void* stream);

/* hn_expert_mlp_int4 without allocation: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments as
 * hn_expert_mlp_int4 minus the buffers: h [T, I] and the split-K workspace live
 * in a library-owned static device array of 17 MiB per GPU (held until the
 * process ends; set up on the first call on each device).  Limits: T <= 16,
 * T * I * 2 <= 1 MiB and hn_skinny_workspace_bytes(2, T, H, I, 0) <= 16 MiB
 * (Mixtral 4096/14336 at T = 16 needs 9 MiB); beyond them it returns -EINVAL
 * with a message.  Same kernels, so the same results as hn_expert_mlp_int4.
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (concurrent streams) race; calls in one stream's order do not. */
int hn_expert_mlp_int4_noalloc(const void* x, const void* gq, const void* gs, const void* uq,
                               const void* us, const void* dq, const void* ds, void* out, long T,
                               long H, long I, long group, void* stream);

/* Decoder-step helpers around the MoE layer (the whole-model decode harness).
 *
 * hn_add_rmsnorm: for rows t < T of H fp16 (H % 8 == 0, H <= 8192):
 *   x' = fp16(x[t] + res[t]) when res is given (written to x_out, which may
 *   alias x), else x' = x[t];  out[t] = fp16(w * (x' * rsqrt(mean(x'^2) + eps)))
 *   in fp32.  Replaces the residual add and RMSNorm of the reference's decoder
 *   block (model/mixtral.py:23-37, 407-427); the mean's fp32 summation order
 *   is its own (outputs within an fp16 ulp of the torch formulation).
 *
 * hn_rope_append: q [B*S, nh*hd], k / v [B*S, nkv*hd] (row b*S + s, fp16), the
 *   fp32 RoPE tables cos_t / sin_t [max_pos, hd], positions pos [S] (int64, on
 *   the device).  Writes the rotated queries to q_out [B, nkv, nh/nkv, S, hd]
 *   (the query heads sharing a KV head stacked), the rotated keys to
 *   kt [B, nkv, hd, max_len] at column pos[s] and the values to
 *   vc [B, nkv, max_len, hd] at row pos[s].  RoPE in the reference's fp16 steps
 *   (apply_rotary_pos_emb, model/mixtral.py:82-101; cache update,
 *   cache/kv_cache.py:26-284), bit for bit. */
int hn_add_rmsnorm(const void* x, long ld_x, const void* res, long ld_r, void* x_out,
                   long ld_xo, const void* w, void* out, long ld_o, long T, long H, float eps,
                   void* stream);
/* hn_add_rmsnorm_router: hn_add_rmsnorm, then the router logits of each
 *   normalised row against an fp16 gate [E, H] (row stride ld_g, E <= 16):
 *   logits[t, e] = fp16(sum_k out[t, k] * gate[e, k]) with fp32 sums, stored as
 *   fp32 [T, E].  The post-attention RMSNorm (model/mixtral.py:423-425) fused
 *   with TopKRouter's fp16 gate Linear (model/router.py:102); the logits feed
 *   hn_moe_route's logits_in.  The sum's order is its own: a logit may differ
 *   from a GEMM's by an fp16 ulp. */
int hn_add_rmsnorm_router(const void* x, long ld_x, const void* res, long ld_r, void* x_out,
                          long ld_xo, const void* w, void* out, long ld_o, long T, long H,
                          float eps, const void* gate, long ld_g, long E, float* logits,
                          void* stream);
/* hn_unpermute_add_rmsnorm: the MoE block's ordered weighted unpermute and
 *   the next block's residual add + RMSNorm in one launch, per token row t:
 *   m = the unpermute of hn_moe_unpermute from four fp32 K-slice partials
 *   part[j * ks_stride + p * ld_y] (fp32 sum in slice order, one fp16
 *   rounding; routing inv / idx / w [T k] as hn_moe_route writes them);
 *   x_out[t] = fp16(x[t] + m); out[t] = RMSNorm(x_out[t]) * w as
 *   hn_add_rmsnorm.  Bit-identical to hn_moe_unpermute's KS = 4 form followed
 *   by hn_add_rmsnorm (model/mixtral.py:365-368 then 407-427). */
int hn_unpermute_add_rmsnorm(const float* part, long ks_stride, long ld_y, const int* inv,
                             const int* idx, const void* rw, long T, long k, const void* x,
                             long ld_x, void* x_out, long ld_xo, const void* w, void* out,
                             long ld_o, long H, float eps, void* stream);
/* hn_attn_softmax: attention probabilities from fp16 scores [rows, L] (row
 *   stride ld_s, 1 <= L <= 1024): a = fp16(s * inv_scale), a = fp16(a +
 *   mask[row % mask_rows]) when mask [mask_rows, L] fp16 (0 / -inf) is given,
 *   out[row] = fp16(softmax_fp32(a)).  The scale, mask add, F.softmax(dtype=
 *   float32) and .to(fp16) of the reference's attention (model/mixtral.py:
 *   193-203) in one launch; inv_scale is the fp32 reciprocal torch multiplies
 *   by for a division by the Python scalar sqrt(head_dim); the softmax keeps
 *   the element-to-lane layout and reduction order of torch's warp softmax
 *   for rows of up to 1024. */
int hn_attn_softmax(const void* scores, long ld_s, const void* mask, long ld_m, long mask_rows,
                    long rows, long L, float inv_scale, void* out, long ld_o, void* stream);
/* hn_attn_decode: grouped-query attention of one query token per sequence
 *   over the KV cache, one launch per layer (the decode step of the
 *   reference's Attention, model/mixtral.py:150-207, in place of its two
 *   products and the softmax between them).  q [B][nkv][rep][hd] fp16 (the
 *   rotated queries of hn_rope_append), kt [B][nkv][hd][max_len] (keys
 *   transposed), v [B][nkv][max_len][hd]; attends over positions [0, L):
 *   s = fp16(q . k) (fp32 sums), a = fp16(s * inv_scale), a = fp16(a +
 *   mask[l]) with mask [L] fp16 (0 / -inf) when given, p = fp16(
 *   softmax_fp32(a)), out[b][(g * rep + r) * hd + d] = fp16(sum_l p v) (fp32
 *   sums).  hd 128, rep 1, 2 or 4, 1 <= L <= 1024, max_len a multiple of 8
 *   holding L rounded up to 8; 16-byte aligned operands. */
int hn_attn_decode(const void* q, const void* kt, const void* v, long max_len, long B, long nkv,
                   long rep, long hd, long L, const void* mask, float inv_scale, void* out,
                   long ld_o, void* stream);

/* hn_attn_decode_rope: hn_rope_append and hn_attn_decode of a one-token step
 *   in one launch: qkv [B][ld_qkv] fp16 holds the step's unrotated query heads
 *   (nkv * rep * hd), keys (nkv * hd) and values (nkv * hd) — the fused q/k/v
 *   projection — and pos [1] int64 (device) its position p; the keys and
 *   queries are rotated with cos_t / sin_t [positions][hd] fp32 exactly as
 *   hn_rope_append rotates them, the key and value written to kt[b][g][:][p]
 *   and v[b][g][p][:], and attention computed over [0, L) with the new key
 *   and value for position p.  A p outside [0, max_len) writes nothing.
 *   Same limits as hn_attn_decode; qkv rows 4-byte aligned. */
int hn_attn_decode_rope(const void* qkv, long ld_qkv, const float* cos_t, const float* sin_t,
                        const long* pos, void* kt, void* v, long max_len, long B, long nkv,
                        long rep, long hd, long L, const void* mask, float inv_scale, void* out,
                        long ld_o, void* stream);
int hn_rope_append(const void* q, long ld_q, const void* k, long ld_k, const void* v, long ld_v,
                   const float* cos_t, const float* sin_t, const long* pos, long B, long S,
                   long nh, long nkv, long hd, void* q_out, void* kt, void* vc, long max_len,
                   void* stream);

/* Decode kernel family for hn_int4_linear, hn_int4_gate_up_silu,
 * hn_expert_mlp_int4 and hn_grouped_expert_mlp_int4, for the calling thread
 * only (each thread starts at 0; a switch never affects another thread):
 *   0  automatic: the persistent streaming kernels for group 128 and at most
 *      16 rows per weight matrix, the split-K kernels otherwise (default);
 *   1  split-K kernels only.
 * Both give the same results to within fp32 summation order.  No counterpart
 * in the reference; for A/B measurement and tests. */
int hn_set_decode_path(int path);

/* A plain streaming read of bytes of buf (nwg workgroups, each one slice of
 * bytes / nwg; bytes a multiple of nwg x 16, under 2^31 bytes per
 * workgroup): the rate a launch that only reads its bytes reaches, the
 * yardstick for the expert kernels' HBM rates.  sink [nwg] fp32 is written
 * only if the folded data hits one fixed word (normally never).  No
 * counterpart in the reference; for measurement (bench.py --workload copy). */
int hn_hbm_read_probe(const void* buf, long bytes, long nwg, float* sink, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* HN_INT4_H */
