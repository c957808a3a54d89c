/*
 * mnemo_oracle.h -- CPU restatement of MnemoCUDA's quantized-matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP kernels are
 * compared against; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.  The product library (mnemocuda_amd/libmnemo_hip.so) never links,
 * loads or falls back to it.
 *
 * Every routine cites the reference file:line whose arithmetic it restates
 * (paths relative to the MnemoCUDA source tree).
 *
 * Pinning (what fixes each routine independently of this code; see tests/test_oracle.py):
 *   mo_f16_to_f32        exhaustive over all 65536 patterns vs numpy float16 and x86 F16C.
 *   mo_f32_to_f16        edge cases + 2^20 random floats vs numpy astype(float16) (RNE).
 *   mo_get_scale_min_k4  exhaustive round trip through an independent packer, and the
 *                        packed-int form of gemm_q4k.cu:53-56 restated in numpy.
 *   mo_dequant_q4k/q6k   one-hot brute force over all 256 positions, closed forms
 *                        (all-zero / all-max quants), linearity in d and dmin, and an
 *                        independent numpy restatement written from the layout text.
 *   mo_gemv_*            fp64 brute force of numpy-dequantised weights.
 *   mo_quantize_q8_1     closed forms per block (zero block, +-amax maps to +-127,
 *                        round-half-even ties) and an independent numpy restatement.
 *   mo_topk_softmax      numpy argsort (stable) + fp64 softmax.
 *   mo_gemm_*            an independent numpy restatement (main part from the decoded
 *                        integers, min term from the ds field); d = 0 weights leave the min
 *                        term alone; the identity split - full dequant product =
 *                        sum_s dmin*m_s * (d8 * sum q8 - ds).
 *   mo_xoroshiro_next    an independent Python restatement of xoroshiro128+ (64-bit
 *                        wrap-around arithmetic) over many seeds.
 *   mo_sample_token      greedy = numpy argmax; top_p -> 0 draws the argmax for every
 *                        seed; draw frequencies over many seeds match the renormalised
 *                        nucleus distribution (chi-square); a numpy restatement.
 *   mo_rms_norm*         closed form for constant vectors, scale invariance, numpy.
 *   mo_rope              pos 0 is the identity, per-pair norms are preserved, two
 *                        rotations compose, numpy restatement (mnemo_oracle_attn.c).
 *   mo_kv_quant_int8     closed forms (the absmax element maps to +-127, zero heads),
 *                        round-half-even ties, numpy restatement.
 *   mo_attention         one position returns v exactly, q = 0 gives the mean of v, a
 *                        dominant score picks its v, numpy softmax restatement.
 */
#ifndef MNEMO_ORACLE_H
#define MNEMO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MO_QK_K 256
#define MO_Q4K_BYTES 144
#define MO_Q6K_BYTES 210
#define MO_Q8_1_MMQ_BYTES 144 /* 4 x half2 + 128 int8, covers 128 values */

/* GGUF type ids used by the reference dispatcher (forward.c:160-173). */
#define MO_TYPE_F32 0
#define MO_TYPE_Q4K 12
#define MO_TYPE_Q6K 14

float mo_f16_to_f32(uint16_t h);
uint16_t mo_f32_to_f16(float f);
void mo_get_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m);

/* Dequantise n_rows x n_cols (row-major, ceil(n_cols/256) blocks per row). */
void mo_dequant_q4k(const void *w, float *out, int n_rows, int n_cols);
void mo_dequant_q6k(const void *w, float *out, int n_rows, int n_cols);
int mo_dequant(int type_id, const void *w, float *out, int n_rows, int n_cols);

/* y = W x accumulated in fp64 over fp32 dequantised weights. */
int mo_gemv(int type_id, const void *w, const float *x, double *y, int n_rows, int n_cols);

/* CPU baseline: the reference GPU kernel's arithmetic (fp32 dequant, fp32 accumulate),
 * rows split over nthreads OpenMP threads. */
int mo_gemv_f32acc(int type_id, const void *w, const float *x, float *y, int n_rows,
                   int n_cols, int nthreads);

void mo_matvec_f32(const float *w, const float *x, double *y, int n_rows, int n_cols);
void mo_topk_softmax(const float *scores, int n_experts, int k, int *idx, float *wts);
void mo_swiglu(const float *g, const float *u, float *out, int n);
void mo_scaled_add(float *out, const float *x, float scale, int n);

/* Q8_1 "MMQ" activation blocks, [N][K/128] blocks of 144 B. */
void mo_quantize_q8_1_mmq(const float *src, void *dst, int K, int N);
void mo_dequant_q8_1_mmq(const void *src, float *out, int K, int N);

/* out[j*M + i] = sum_k deq(W)[i][k] * deq(A)[j][k] in fp64 (column-major [N][M]). */
int mo_gemm_q8_1(int type_id, const void *w, const void *act, double *out, int M, int K, int N);

/* Next-token selection of kernels.cu:2020-2174: greedy argmax for temperature <= 0, else
 * top-p over 2048 per-class candidates with the reference's fp32 summation orders and
 * selection sort, xoroshiro128+ draw.  Returns the token; *u_out (may be NULL) gets the
 * uniform draw, *nsum_out the renormalised nucleus mass. */
int mo_sample_token(const float *logits, int V, float temperature, float top_p,
                    unsigned long long seed, float *u_out, float *nsum_out);
uint64_t mo_xoroshiro_next(uint64_t *s0, uint64_t *s1);

/* Decode attention chain (mnemo_oracle_attn.c). */
void mo_rms_norm(const float *in, const float *w, float *out, int n, float eps);
void mo_rms_norm_residual(const float *in, const float *w, float *normed, float *residual, int n, float eps);
void mo_rms_norm_heads(const float *in, const float *w, float *out, int head_dim, int n_heads, float eps);
void mo_residual_add(const float *a, const float *b, float *out, int n);
float mo_rope_freq(int j, int head_dim, float theta);
void mo_rope(float *q, float *k, int head_dim, int pos, float theta, int n_heads_q, int n_heads_k);
void mo_kv_quant_int8(const float *in, int8_t *out, float *scales, int head_dim, int n_kv_heads);
#define MO_ATTN_MAX_HD 1024
int mo_attention(const float *q, const void *kv_k, const void *kv_v, const float *k_scales,
                 const float *v_scales, int kv_type, float *out, int n_heads, int head_dim,
                 int n_kv_heads, int seq_len, int gqa, float scale);

#ifdef __cplusplus
}
#endif
#endif
