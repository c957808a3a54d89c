/*
 * mnemo_kernels.h -- C ABI of the MI355X (gfx950) quantized-matmul library.
 *
 * Drop-in for MnemoCUDA's kernel entry points: the functions named cuda_* keep the
 * reference's names, argument lists and semantics (forward.c declares them extern at
 * forward.c:23-152; they are defined in kernels.cu / gemm_q4k.cu at the lines cited per
 * declaration), with cudaStream_t replaced by hipStream_t.  The mnemo_* functions are
 * additions the reference lacks.
 *
 * Conventions shared by every entry point:
 *  - All pointers are device pointers owned by the caller; nothing here allocates.
 *  - Weights are raw GGUF bytes, row-major, ceil(n_cols/256) super-blocks per row:
 *    Q4_K 144 B (type id 12), Q6_K 210 B (type id 14), F32 router (type id 0).
 *  - Every call is asynchronous on `stream` and capture-safe (no sync, no malloc,
 *    no attribute changes at launch), so calls can be recorded into a hipGraph.
 *  - Errors: like the reference (KERNEL_LAUNCH_CHECK, kernels.cu:1062-1067) failures
 *    are printed to stderr and the call returns without launching; in addition the
 *    code is kept for mnemo_last_error().  Argument checks that the reference does not
 *    make (null pointers, non-positive sizes, K not a multiple of 256 for GEMMs) are
 *    reported the same way.
 */
#ifndef MNEMO_KERNELS_H
#define MNEMO_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifndef __HIP_PLATFORM_AMD__
#define __HIP_PLATFORM_AMD__ 1
#endif
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- errors */
#define MNEMO_OK 0
#define MNEMO_ERR_BAD_ARG 1
#define MNEMO_ERR_LAUNCH 2
#define MNEMO_ERR_UNSUPPORTED_TYPE 3
#define MNEMO_ERR_IO 4
#define MNEMO_ERR_ALLOC 5

/* Last error recorded by any entry point on this host thread (MNEMO_OK if none);
 * reading it clears it. */
int mnemo_last_error(void);
const char *mnemo_last_error_string(void);

/* Library version string, e.g. "mnemo-mi355x 0.1 gfx950". */
const char *mnemo_version(void);

/* Replaces cuda_kernels_init (kernels.cu:2217-2240, called once at load,
 * engine.c:1203-1207).  Nothing needs raising on gfx950 (every kernel stays within the
 * default LDS limit); the call checks that the current device is gfx950. */
void cuda_kernels_init(void);

/* ---------------------------------------------------------------- decode GEMVs */
/* y = W x, W Q4_K [n_rows][n_cols]                       (kernels.cu:66, :1071-1079) */
void cuda_matvec_q4k(const void *weights, const float *x, float *y, int n_rows, int n_cols,
                     hipStream_t stream);
/* y = W x + residual (O-proj + skip)                      (kernels.cu:149, :1094-1102) */
void cuda_matvec_q4k_add(const void *weights, const float *x, const float *residual, float *y,
                         int n_rows, int n_cols, hipStream_t stream);
/* Q, K, V projections of one x in one launch              (kernels.cu:205, :1081-1092) */
void cuda_matvec_q4k_qkv(const void *w_q, const void *w_k, const void *w_v, const float *x,
                         float *out_q, float *out_k, float *out_v, int q_rows, int kv_rows,
                         int n_cols, hipStream_t stream);
/* y_a = A x, y_b = B x (K+V, gate+up), both Q4_K         (kernels.cu:278, :1104-1113) */
void cuda_matvec_q4k_dual(const void *wa, const void *wb, const float *x, float *ya, float *yb,
                          int n_rows, int n_cols, hipStream_t stream);
/* y += scale * (W x), W Q4_K (expert down-proj)           (kernels.cu:358, :1115-1124) */
void cuda_matvec_q4k_scaled_add(const void *weights, const float *x, float *y, int n_rows,
                                int n_cols, float scale, hipStream_t stream);
/* y = W x, W Q6_K                                          (kernels.cu:427, :1126-1135) */
void cuda_matvec_q6k(const void *weights, const float *x, float *y, int n_rows, int n_cols,
                     hipStream_t stream);

/* New: y += scale * (W x), W Q6_K, in one launch.  Replaces the reference's
 * cuda_matvec_q6k + cuda_scaled_add pair (forward.c:1137-1140). */
void mnemo_matvec_q6k_scaled_add(const void *weights, const float *x, float *y, int n_rows,
                                 int n_cols, float scale, hipStream_t stream);
/* New: y_a = A x, y_b = B x with independent GGUF types (12 or 14) for A and B, e.g. the
 * Q4_K K-proj + Q6_K V-proj of Q4_K_M models, which the reference runs as two launches
 * (forward.c:714-718). */
void mnemo_matvec_dual(const void *wa, int type_a, const void *wb, int type_b, const float *x,
                       float *ya, float *yb, int n_rows, int n_cols, hipStream_t stream);
/* New: cuda_matvec_q4k_qkv with a GGUF type per matrix.  Q4_K_M stores V as Q6_K, for
 * which the reference falls back to separate matvec() launches (src/forward.c:699-718);
 * this replaces that whole branch:
 * Q [q_rows], K and V [kv_rows] from one x, one launch. */
void mnemo_matvec_qkv(const void *wq, int tq, const void *wk, int tk, const void *wv, int tv,
                      const float *x, float *oq, float *ok, float *ov, int q_rows, int kv_rows,
                      int n_cols, hipStream_t stream);
/* New: the same with the pre-attention RMS norm folded in (forward.c:695-699 runs
 * cuda_rms_norm_residual first): the projections read x * rsqrt(mean(x^2) + eps) * norm_w,
 * which every workgroup computes from the raw x it loads anyway.  n_cols % 4 == 0. */
void mnemo_matvec_qkv_rmsnorm(const void *wq, int tq, const void *wk, int tk, const void *wv,
                              int tv, const float *x, const float *norm_w, float eps, float *q,
                              float *k, float *v, int q_rows, int kv_rows, int n_cols,
                              hipStream_t stream);
/* New: fused expert down projection of one expert:
 * y += scale * (W_down (silu(gate) * up)), W_down Q4_K or Q6_K [n_rows][n_cols].
 * Replaces cuda_swiglu + (cuda_matvec_q4k_scaled_add | cuda_matvec_q6k + cuda_scaled_add)
 * in expert_fwd (forward.c:1130-1141). */
void mnemo_matvec_swiglu_scaled_add(const void *w_down, int type_down, const float *gate,
                                    const float *up, float *y, int n_rows, int n_cols, float scale,
                                    hipStream_t stream);

/* ---------------------------------------------------------------- router */
/* y = W x, W fp32 row-major [n_rows][n_cols]               (kernels.cu:859, :1275-1281) */
void cuda_matvec_f32(const float *weights, const float *x, float *y, int n_rows, int n_cols,
                     hipStream_t stream);
/* top-k of n_experts scores, softmax over the k winners    (kernels.cu:993, :1301-1305)
 * k <= 16, n_experts <= 1024.  Winners are written in (score desc, index asc) order; the
 * reference writes them in an unspecified slot order, so consumers must only rely on the
 * (index, weight) pairing, which is what forward.c does. */
void cuda_topk_softmax(const float *scores, int *indices, float *weights, int n_experts, int k,
                       hipStream_t stream);

/* ---------------------------------------------------------------- glue */
/* out = silu(gate) * up                                    (kernels.cu:677, :1170-1176) */
void cuda_swiglu(const float *gate, const float *up, float *out, int n, hipStream_t stream);
/* out += scale * x                                         (kernels.cu:980, :1293-1299) */
void cuda_scaled_add(float *out, const float *x, float scale, int n, hipStream_t stream);

/* ---------------------------------------------------------------- prefill GEMM */
/* fp32 [N][K] -> Q8_1 MMQ blocks [N][K/128] x 144 B        (gemm_q4k.cu:327-364)
 * Byte-identical to the reference (including ds.y = half(d * sum(x))).  K % 128 == 0;
 * src and dst 16-byte aligned. */
void cuda_quantize_mmq_q8_1(const float *src, void *dst, int K, int N, hipStream_t stream);
/* out[j*M + i] = sum_k deq(W)[i][k] * deq(act)[j][k]      (gemm_q4k.cu:202, :272-324)
 * W Q4_K [M][K], act from cuda_quantize_mmq_q8_1 with N columns, out column-major [N][M].
 * K % 256 == 0. */
void cuda_gemm_q4k(const void *weights, const void *act_q8, float *output, int M, int K, int N,
                   hipStream_t stream);
/* New: the same for Q6_K weights (Q4_K_M expert down projections). */
void mnemo_gemm_q6k(const void *weights, const void *act_q8, float *output, int M, int K, int N,
                    hipStream_t stream);

/* ---- next token (kernels.cu:2208-2215, kernels.cu:2020-2174; forward.c:1703-1704) ------
 * temperature <= 0: argmax of logits[vocab_size] (exact ties go to the lower index);
 * else top-p sampling over the reference's 2048 candidates (8 per residue class mod 256),
 * drawn with xoroshiro128+ seeded from rng_state.  Writes one int to d_result. */
void cuda_sample_token(const float *logits, int vocab_size, float temperature, float top_p,
                       unsigned long long rng_state, int *d_result, hipStream_t stream);
/* New: the same selection with the vocabulary scan spread over 64 workgroups (two
 * launches, capture-safe): the class winners and partial sums go through a workspace of
 * mnemo_sample_workspace_bytes() bytes (16-byte aligned, no initialisation; calls sharing it
 * must not overlap).  vocab_size <= 262,144.  Same token as cuda_sample_token except when
 * the draw lies within fp32 rounding of a nucleus boundary (the total is summed in another
 * order).  Returns 0 or an MNEMO_ERR_* code. */
size_t mnemo_sample_workspace_bytes(void);
int mnemo_sample_token_ws(const float *logits, int vocab_size, float temperature, float top_p,
                          unsigned long long rng_state, void *workspace, size_t workspace_bytes,
                          int *d_result, hipStream_t stream);

/* ---- Grouped-expert prefill (no reference counterpart) ---------------------------------
 * The reference prefills MoE layers token by token through the decode chain
 * (src/forward.c:1783-1830; per expert src/forward.c:876-893).  This entry point computes
 * the same composition for T tokens at once:
 *   out[t] += sum_slot topk_w[t][slot] * W_down[e] (silu(W_gate[e] x_t) * W_up[e] x_t),
 *   e = topk_idx[t][slot]
 * with x_t and the SwiGLU activations quantized to Q8_1 (the GEMM semantics above).
 * Expert e's matrices sit at experts + e*expert_stride + {gate,up,down}_off, gate/up Q4_K
 * [eff][hidden], down Q4_K or Q6_K [hidden][eff] (the reference's expert file layout,
 * src/forward.c:866-872).  topk_idx / topk_w are [n_tokens][k] (cuda_topk_softmax's output
 * per token); ids outside [0, n_experts) are skipped.  hidden, eff % 256 == 0,
 * n_experts <= 512, n_tokens * k <= 4,194,304.  experts, expert_stride and the three
 * offsets 4-byte aligned (the weight blocks are copied into LDS by 16-byte DMA from 4-byte
 * aligned addresses).  workspace: device memory of at least
 * mnemo_moe_prefill_workspace_bytes(...) bytes, 16-byte aligned. */
size_t mnemo_moe_prefill_workspace_bytes(int n_tokens, int hidden, int eff, int n_experts, int k);
int mnemo_moe_prefill(const void *experts, size_t expert_stride, size_t gate_off, size_t up_off,
                      size_t down_off, int down_type, const float *x, const int *topk_idx,
                      const float *topk_w, int n_tokens, int hidden, int eff, int n_experts, int k,
                      void *workspace, size_t workspace_bytes, float *out, hipStream_t stream);

/* ---- Decode MoE block with device-side expert dispatch (no reference counterpart) --------
 * Replaces the reference's decode MoE block (src/forward.c:814-1077: router matvec, top-k,
 * a host synchronisation to read the expert ids, then expert_fwd per expert) for one token:
 *   z = W_router x;  (idx, w) = top-k softmax of z;
 *   out += sum_slot w[slot] * W_down[e] (silu(W_gate[e] x) * W_up[e] x),  e = idx[slot]
 * The ids stay on the device; three launches, no synchronisation, capture-safe.  Expert e's
 * matrices sit at experts + e*expert_stride + {gate,up,down}_off (gate/up Q4_K [eff][hidden],
 * down Q4_K or Q6_K [hidden][eff]); router_w is fp32 [n_experts][hidden].  topk_idx /
 * topk_w (may be NULL) receive the routing.  k <= 16, n_experts <= 1024, hidden and eff
 * multiples of 256.  workspace: mnemo_moe_decode_workspace_bytes(...) bytes, 16-byte
 * aligned, zero-filled once after allocation (each call leaves it reusable); calls that
 * share a workspace must not overlap. */
size_t mnemo_moe_decode_workspace_bytes(int hidden, int eff, int n_experts, int k);
int mnemo_moe_decode(const float *router_w, const void *experts, size_t expert_stride,
                     size_t gate_off, size_t up_off, size_t down_off, int down_type,
                     const float *x, int hidden, int eff, int n_experts, int k, void *workspace,
                     size_t workspace_bytes, float *out, int *topk_idx, float *topk_w,
                     hipStream_t stream);
/* New: mnemo_moe_decode with the pre-FFN RMS norm folded into the router and gate/up
 * launches (x is the raw hidden state; both compute x * rsqrt(mean(x^2) + eps) * norm_w as
 * forward.c:800-806's separate rms_norm launch would).  x may equal out. */
int mnemo_moe_decode_rmsnorm(const float *router_w, const void *experts, size_t expert_stride,
                             size_t gate_off, size_t up_off, size_t down_off, int down_type,
                             const float *x, const float *norm_w, float eps, int hidden, int eff,
                             int n_experts, int k, void *workspace, size_t workspace_bytes,
                             float *out, int *topk_idx, float *topk_w, hipStream_t stream);
/* New, no counterpart in the reference: mnemo_moe_decode_rmsnorm for callers that cannot
 * allocate or hold a workspace (code under hipGraph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  It allocates nothing: the workspace is a device array inside the
 * library, one copy per GPU kept until the process ends, set up by cuda_kernels_init (or by
 * the first call on a GPU).  Sizes must fit that array, 1,703,936 bytes of workspace
 * (mnemo_moe_decode_workspace_bytes(hidden, eff, n_experts, k) <= that: hidden 8192,
 * eff 4096, 1024 experts, k 16 fit); larger sizes are rejected with an error.  Every call on
 * a GPU shares that GPU's array, so calls that overlap on one GPU (other streams or host
 * threads) race. */
int mnemo_moe_decode_rmsnorm_noalloc(const float *router_w, const void *experts,
                                     size_t expert_stride, size_t gate_off, size_t up_off,
                                     size_t down_off, int down_type, const float *x,
                                     const float *norm_w, float eps, int hidden, int eff,
                                     int n_experts, int k, float *out, int *topk_idx,
                                     float *topk_w, hipStream_t stream);

/* ---- Attention chain around the projections (forward.c:687-786, graph form 1290-1420) ----
 * Reference entry points, same arguments and semantics: */
/* kernels.cu:1187-1193 (rms_norm_kernel :692-722): out = in * rsqrt(mean(in^2) + eps) * w. */
void cuda_rms_norm(const float *input, const float *weight, float *output, int n, float eps,
                   hipStream_t stream);
/* kernels.cu:1178-1185 (:725-749): the same plus residual_output = input. */
void cuda_rms_norm_residual(const float *input, const float *weight, float *normed_output,
                            float *residual_output, int n, float eps, hipStream_t stream);
/* kernels.cu:1221-1227 (:754-781): every head of head_dim values with the shared weight
 * [head_dim]; output may equal input. */
void cuda_rms_norm_batched(const float *input, const float *weight, float *output, int head_dim,
                           int n_heads, float eps, hipStream_t stream);
/* kernels.cu:1229-1236 (:1196-1219): q heads with q_weight, k heads with k_weight, in place. */
void cuda_rms_norm_qk(float *q, float *k, const float *q_weight, const float *k_weight,
                      int head_dim, int n_q, int n_k, float eps, hipStream_t stream);
/* kernels.cu:1238-1244 (:784-793): out = a + b. */
void cuda_residual_add(const float *a, const float *b, float *out, int n, hipStream_t stream);
/* kernels.cu:1256-1273 (:818-852): rotates the pairs (j, j + head_dim/2) of every q and k
 * head by pos / theta^(2j/head_dim), in place.  sin/cos are accurate (the reference's
 * __sincosf approximation loses accuracy as pos grows). */
void cuda_rope(float *q, float *k, int head_dim, int pos, float theta, int n_heads_q,
               int n_heads_k, hipStream_t stream);
/* kernels.cu:1328-1335 (:1320-1326): oa = f16(a), ob = f16(b), round to nearest even. */
void cuda_f32_to_f16_dual(const float *a, const float *b, void *oa, void *ob, int n,
                          hipStream_t stream);
/* kernels.cu:2243-2245: the kernels an engine finds in a captured graph by function pointer
 * (forward.c:1395-1412) and patches before every replay (forward.c:633-668).
 * cuda_get_rope_kernel_ptr: the kernel of cuda_rope, parameter 3 = pos.
 * cuda_get_f16dual_kernel_ptr: the kernel of cuda_f32_to_f16_dual, parameters 2 and 3 = the
 * f16 destinations.  cuda_get_attn_f16kv_kernel_ptr: the first kernel of cuda_attention_f16kv
 * (head_dim 128, gqa <= 16), parameter 6 = seq_len. */
void *cuda_get_rope_kernel_ptr(void);
void *cuda_get_f16dual_kernel_ptr(void);
void *cuda_get_attn_f16kv_kernel_ptr(void);
/* No counterpart in the reference: workspace slots of cuda_attention_f16kv / _int8kv.  Makes
 * at least n_slots free slots exist on the current GPU (allocates; call outside any graph
 * capture), for an engine that captures more attention calls than cuda_kernels_init's 16.
 * Returns 0 or an error code. */
int mnemo_attention_reserve(int n_slots);
/* bytes of one slot (device memory held until the process ends) */
size_t mnemo_attention_slot_bytes(void);
/* kernels.cu:1526-1534 (:1493-1524): per head absmax a, scale = a/127, q = rne(x*127/a)
 * clamped to +-127; out_* and *_scales point at the current position's row and slots. */
void cuda_f32_to_int8_kv_dual(const float *k, const float *v, void *out_k, void *out_v,
                              float *k_scales, float *v_scales, int head_dim, int n_kv_heads,
                              hipStream_t stream);
/* kernels.cu:1662-1673 (:1550-1660) and :1536-1546 (:1382-1481): softmax(scale q.k) v over
 * positions 0..seq_len-1 of the cache [pos][n_kv_heads][head_dim] for every query head
 * (kv head = head / gqa_ratio).  head_dim 64, 128 or 256.  With head_dim 128, gqa <= 16 and
 * n_kv_heads <= 256 the call is two launches: the split kernel (the function
 * cuda_get_attn_f16kv_kernel_ptr returns, with the reference kernel's parameters first and
 * seq_len as parameter 6, and a grid that does not depend on seq_len) and the merge of its
 * partials.  They run on a workspace slot of mnemo_attention_slot_bytes(): eager calls use a
 * slot bound to their stream, and a call made under graph capture takes a free slot of its own
 * (cuda_kernels_init reserves 16, mnemo_attention_reserve more), so a captured graph can be
 * replayed on any stream next to eager calls.  Other shapes run the per-head kernel.  The two
 * paths agree to ~1e-6 relative (not bit for bit). */
void cuda_attention_f16kv(const void *q, const void *kv_k, const void *kv_v, float *out,
                          int n_heads_q, int head_dim, int n_kv_heads, int seq_len, int gqa_ratio,
                          float scale, hipStream_t stream);
void cuda_attention_int8kv(const float *q, const void *kv_k, const void *kv_v,
                           const float *k_scales, const float *v_scales, float *out,
                           int n_heads_q, int head_dim, int n_kv_heads, int seq_len,
                           int gqa_ratio, float scale, hipStream_t stream);

/* ---- Token embedding (forward.c:1145-1280) ------------------------------------------
 * kernels.cu:2192-2198: output[0..hidden_size) = dequantised row token_id of a Q4_K table
 * with row_bytes per row.  Decodes the canonical GGUF layout (as the matvec kernels and the
 * reference's CPU fallback forward.c:1189-1229 do; the reference GPU kernel, kernels.cu:
 * 1901-1951, indexes the nibbles differently). */
void cuda_embedding_lookup_q4k(const void *embd_table, float *output, int token_id,
                               int hidden_size, int row_bytes, hipStream_t stream);
/* New: the same for F32 (0), Q4_K (12) or Q6_K (14) tables of n_vocab rows, the token id
 * read from device memory (e.g. cuda_sample_token's d_result) so a decode step's graph
 * chains sampling into the next embedding; ids outside the table read the nearest row. */
int mnemo_embedding_lookup(const void *table, int type_id, const int *token_dev, int n_vocab,
                           float *output, int hidden_size, hipStream_t stream);

/* New: the per-token steps 3-5 of forward.c:755-770 (QK norm, RoPE, KV store) in one launch
 * with the position read from device memory (*pos_dev), so a captured graph replays for
 * every token without the kernel-node updates of forward.c:638-666.  q [n_heads][head_dim]
 * and k [n_kv_heads][head_dim] are normalised (when both weights are given) and rotated in
 * place; k is stored at cache row *pos_dev ([pos][n_kv_heads][head_dim]), v likewise
 * (v_layout 0) or in the blocked layout of mnemo_attention_decode (v_layout 1:
 * [pos/64][n_kv_heads][head_dim][pos%64]).  kv_type 0 f16, 1 int8 with scales
 * [pos][n_kv_heads].  head_dim even, <= 512. */
int mnemo_attn_prep(float *q, float *k, const float *v, const float *q_norm_w,
                    const float *k_norm_w, int head_dim, int n_heads, int n_kv_heads, float eps,
                    float theta, const int *pos_dev, void *k_cache, void *v_cache,
                    float *k_scales, float *v_scales, int kv_type, int v_layout,
                    hipStream_t stream);
/* Bytes of a V cache for max_ctx positions in the given layout (blocked: rounded up to 64). */
size_t mnemo_v_cache_bytes(int n_kv_heads, int head_dim, int max_ctx, int kv_type, int v_layout);
/* New: cuda_attention_* over positions 0..*pos_dev (the length read from device memory). */
int mnemo_attention(const float *q, const void *k_cache, const void *v_cache,
                    const float *k_scales, const float *v_scales, int kv_type, float *out,
                    int n_heads, int head_dim, int n_kv_heads, const int *pos_dev, float scale,
                    hipStream_t stream);

/* New: the same attention for head_dim 128 and gqa <= 16 on the matrix cores, split over
 * 64-position chunks (each KV head is read once per chunk for all of its query heads; the
 * reference's attention_kernel_f16kv streams it once per query head, kernels.cu:1550-1660),
 * then merged per query head: two launches, capture-safe.  Positions 0..*pos_dev
 * (< max_ctx <= 65536).  K cache [pos][n_kv_heads][head_dim]; V cache in v_layout 0 (the
 * same rows) or 1 (blocked, mnemo_attn_prep's v_layout 1: the fast path; allocate
 * mnemo_v_cache_bytes and zero-fill it once, the rows past the sequence in the last block
 * are read with weight 0).  workspace: mnemo_attention_decode_workspace_bytes(n_kv_heads,
 * max_ctx) bytes, 16-byte aligned, no initialisation; calls sharing it must not overlap. */
size_t mnemo_attention_decode_workspace_bytes(int n_kv_heads, int max_ctx);
int mnemo_attention_decode(const float *q, const void *k_cache, const void *v_cache,
                           const float *k_scales, const float *v_scales, int kv_type, int v_layout,
                           float *out, int n_heads, int head_dim, int n_kv_heads, int max_ctx,
                           const int *pos_dev, float scale, void *workspace,
                           size_t workspace_bytes, hipStream_t stream);
/* New: mnemo_attn_prep and mnemo_attention_decode in the same two launches, for the
 * decode step's attention block (forward.c:720-775: QK norm, RoPE, cache store, attention).
 * q [n_heads][128], k and v [n_kv_heads][128] are the projections' raw outputs and are not
 * modified; every chunk normalises and rotates its query heads in registers, and the chunk
 * holding *pos_dev writes the new K / V rows (K normalised and rotated; int8: with their
 * scales) and uses them directly.  The caches and out are bit-identical to mnemo_attn_prep
 * followed by mnemo_attention_decode.  Nothing is stored when *pos_dev >= max_ctx. */
int mnemo_attention_decode_prep(const float *q, const float *k, const float *v,
                                const float *q_norm_w, const float *k_norm_w, float eps,
                                float theta, void *k_cache, void *v_cache, float *k_scales,
                                float *v_scales, int kv_type, int v_layout, float *out,
                                int n_heads, int head_dim, int n_kv_heads, int max_ctx,
                                const int *pos_dev, float scale, void *workspace,
                                size_t workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* MNEMO_KERNELS_H */
