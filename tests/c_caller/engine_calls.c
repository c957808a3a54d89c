/*
 * engine_calls.c -- a C caller of the library's C-ABI, written the way the reference engine
 * calls its kernels (MnemoCUDA src/forward.c:160-173 matvec dispatch, :687-823 one decode
 * layer): plain C, the HIP runtime's C API for device memory, the extern "C" entry points
 * of include/mnemo_kernels.h with the reference's argument lists, one stream.
 *
 * It fills seeded GGUF blocks and activations, runs the decode-path entry points, and
 * writes every input and output to one binary file that tests/test_gpu_c_caller.py checks
 * against the oracle.  Exit status: 0 on success, 1 on a library or HIP error.
 *
 * File layout (little endian): int32 R, RK, C, E, K, NT, then the bytes of Wq4 (R x C Q4_K),
 * Wq6 (R x C Q6_K), Wk (RK x C Q4_K), Wv (RK x C Q6_K), fp32 x[C], res[R], router[E][C],
 * x2[C], act[NT][C], then the outputs y4[R], y6[R], yadd[R], ya[R], yb[R], q[R], k[RK],
 * v[RK], logits[E], int32 idx[K], fp32 w[K], then q2[R], k2[RK], v2[RK] (all-Q4_K QKV),
 * ysa[R] (res + 0.37 Wq4 x), sw[C] (silu(x) * x2), ysc[R] (res + 0.5 y4), the Q8_1 bytes of
 * act [NT][C/128][144] and the GEMM output gout[NT][R] of Wq4 with them.  Then the attention
 * chain: int32 HH, NH, NKV, HD, SEQ, VOC, VT, the inputs xin[HH], anorm[HH], q[NH*HD],
 * k[NKV*HD], v[NKV*HD], qw[HD], kw[HD], the f16 caches K, V [SEQ][NKV][HD] and the int8
 * caches K, V with their scales [SEQ][NKV] before the call, logits[VOC], the Q4_K embedding
 * table [VT][HH], and the outputs normed, resid, normed2, radd [HH], att, att8 [NH*HD],
 * emb[HH], q and k after the QK norm and RoPE, the four caches and two scale arrays after
 * the stores, the sampled token, and the head-wise RMS norm of the raw q [NH*HD].
 */
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/mnemo_kernels.h"

#define R 512
#define RK 128
#define C 4096
#define E 64
#define K 8
#define NT 32
#define Q4_BYTES ((size_t)(C / 256) * 144)
#define Q6_BYTES ((size_t)(C / 256) * 210)
/* the attention chain (forward.c:725-823, :1145-1280 embedding, :1702-1707 sampling) */
#define HH 512   /* hidden size of the norms and the embedding */
#define NH 8     /* query heads */
#define NKV 2    /* KV heads */
#define HD 128   /* head_dim */
#define SEQ 70   /* positions attended: the new token at POS = SEQ - 1 */
#define POS (SEQ - 1)
#define VOC 3000 /* vocabulary of the sampled logits */
#define VT 16    /* rows of the Q4_K embedding table */

static uint64_t lcg = 0x9E3779B97F4A7C15ull;
static uint32_t next32(void) {
    lcg = lcg * 6364136223846793005ull + 1442695040888963407ull;
    return (uint32_t)(lcg >> 32);
}
static float uniform(void) { return (float)(next32() >> 8) * (1.0f / 16777216.0f); }

/* f16 bits of a small positive value (d, dmin, Q6_K d): exponent 2^-8..2^-7 range */
static uint16_t small_f16(void) { return (uint16_t)(0x1C00 | (next32() & 0x3FF)); }

static void fill_q4k(uint8_t *w, size_t rows) {
    for (size_t b = 0; b < rows * (C / 256); b++) {
        uint8_t *blk = w + b * 144;
        uint16_t d = small_f16(), dmin = small_f16();
        memcpy(blk, &d, 2);
        memcpy(blk + 2, &dmin, 2);
        for (int i = 4; i < 144; i++) blk[i] = (uint8_t)next32();
    }
}
static void fill_q6k(uint8_t *w, size_t rows) {
    for (size_t b = 0; b < rows * (C / 256); b++) {
        uint8_t *blk = w + b * 210;
        for (int i = 0; i < 192; i++) blk[i] = (uint8_t)next32();
        for (int i = 192; i < 208; i++) blk[i] = (uint8_t)(int8_t)((int)(next32() % 61) - 30);
        uint16_t d = small_f16();
        memcpy(blk + 208, &d, 2);
    }
}

/* f16 bits of a value in +-[0.125, 1) */
static uint16_t kv_f16(void) { return (uint16_t)((next32() & 0x8000u) | (0x3000u + next32() % 0x0C00u)); }
static float sym(float a) { return a * (2.0f * uniform() - 1.0f); }

static void *dev_copy(const void *h, size_t n) {
    void *d = NULL;
    if (hipMalloc(&d, n) != hipSuccess || hipMemcpy(d, h, n, hipMemcpyHostToDevice) != hipSuccess) return NULL;
    return d;
}

int main(int argc, char **argv) {
    if (argc != 2) {
        fprintf(stderr, "usage: %s <out.bin>\n", argv[0]);
        return 1;
    }
    cuda_kernels_init();
    uint8_t *wq4 = malloc(R * Q4_BYTES), *wq6 = malloc(R * Q6_BYTES);
    uint8_t *wk = malloc(RK * Q4_BYTES), *wv = malloc(RK * Q6_BYTES);
    float *x = malloc(C * 4), *res = malloc(R * 4), *router = malloc((size_t)E * C * 4);
    float *x2 = malloc(C * 4), *act = malloc((size_t)NT * C * 4);
    fill_q4k(wq4, R);
    fill_q6k(wq6, R);
    fill_q4k(wk, RK);
    fill_q6k(wv, RK);
    for (int i = 0; i < C; i++) x[i] = 2.0f * uniform() - 1.0f;
    for (int i = 0; i < R; i++) res[i] = 2.0f * uniform() - 1.0f;
    for (int i = 0; i < E * C; i++) router[i] = (2.0f * uniform() - 1.0f) * 0.03f;
    for (int i = 0; i < C; i++) x2[i] = 2.0f * uniform() - 1.0f;
    for (int i = 0; i < NT * C; i++) act[i] = 4.0f * uniform() - 2.0f;

    void *d_wq4 = dev_copy(wq4, R * Q4_BYTES), *d_wq6 = dev_copy(wq6, R * Q6_BYTES);
    void *d_wk = dev_copy(wk, RK * Q4_BYTES), *d_wv = dev_copy(wv, RK * Q6_BYTES);
    float *d_x = dev_copy(x, C * 4), *d_res = dev_copy(res, R * 4), *d_router = dev_copy(router, (size_t)E * C * 4);
    float *d_x2 = dev_copy(x2, C * 4), *d_act = dev_copy(act, (size_t)NT * C * 4);
    float *d_out = NULL, *d_out2 = NULL;
    int *d_idx = NULL;
    void *d_q8 = NULL;
    const size_t n_out = 5 * R + R + 2 * RK + E + K;
    const size_t n_out2 = R + 2 * RK + R + C + R + (size_t)NT * R;
    const size_t q8_bytes = (size_t)NT * (C / 128) * 144;
    if (!d_wq4 || !d_wq6 || !d_wk || !d_wv || !d_x || !d_res || !d_router || !d_x2 || !d_act ||
        hipMalloc((void **)&d_out, n_out * 4) != hipSuccess || hipMalloc((void **)&d_idx, K * 4) != hipSuccess ||
        hipMalloc((void **)&d_out2, n_out2 * 4) != hipSuccess || hipMalloc(&d_q8, q8_bytes) != hipSuccess) {
        fprintf(stderr, "hip allocation or copy failed\n");
        return 1;
    }
    float *y4 = d_out, *y6 = y4 + R, *yadd = y6 + R, *ya = yadd + R, *yb = ya + R, *q = yb + R;
    float *k = q + R, *v = k + RK, *logits = v + RK, *w = logits + E;
    float *q2 = d_out2, *k2 = q2 + R, *v2 = k2 + RK, *ysa = v2 + RK, *sw = ysa + R, *ysc = sw + C, *gout = ysc + R;
    hipStream_t s;
    if (hipStreamCreate(&s) != hipSuccess) return 1;
    if (hipMemcpy(ysa, d_res, R * 4, hipMemcpyDeviceToDevice) != hipSuccess ||
        hipMemcpy(ysc, d_res, R * 4, hipMemcpyDeviceToDevice) != hipSuccess)
        return 1;

    /* the engine's calls (reference argument lists) */
    cuda_matvec_q4k(d_wq4, d_x, y4, R, C, s);
    cuda_matvec_q6k(d_wq6, d_x, y6, R, C, s);
    cuda_matvec_q4k_add(d_wq4, d_x, d_res, yadd, R, C, s);
    cuda_matvec_q4k_dual(d_wq4, d_wq4, d_x, ya, yb, R, C, s);
    mnemo_matvec_qkv(d_wq4, 12, d_wk, 12, d_wv, 14, d_x, q, k, v, R, RK, C, s);
    cuda_matvec_f32(d_router, d_x, logits, E, C, s);
    cuda_topk_softmax(logits, d_idx, w, E, K, s);
    cuda_matvec_q4k_qkv(d_wq4, d_wk, d_wk, d_x, q2, k2, v2, R, RK, C, s);  /* forward.c:701 */
    cuda_matvec_q4k_scaled_add(d_wq4, d_x, ysa, R, C, 0.37f, s);          /* forward.c:1134 */
    cuda_swiglu(d_x, d_x2, sw, C, s);                                      /* forward.c:1130 */
    cuda_scaled_add(ysc, y4, 0.5f, R, s);                                  /* forward.c:1140 */
    cuda_quantize_mmq_q8_1(d_act, d_q8, C, NT, s);                         /* forward.c:691 */
    cuda_gemm_q4k(d_wq4, d_q8, gout, R, C, NT, s);                         /* forward.c:693-697 */
    if (hipStreamSynchronize(s) != hipSuccess) return 1;
    if (mnemo_last_error() != MNEMO_OK) {
        fprintf(stderr, "library error: %s\n", mnemo_last_error_string());
        return 1;
    }

    float *out = malloc(n_out * 4), *out2 = malloc(n_out2 * 4);
    uint8_t *q8 = malloc(q8_bytes);
    int idx[K];
    if (hipMemcpy(out, d_out, n_out * 4, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(idx, d_idx, K * 4, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(out2, d_out2, n_out2 * 4, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(q8, d_q8, q8_bytes, hipMemcpyDeviceToHost) != hipSuccess)
        return 1;
    FILE *f = fopen(argv[1], "wb");
    if (!f) return 1;
    const int32_t hdr[6] = {R, RK, C, E, K, NT};
    fwrite(hdr, 4, 6, f);
    fwrite(wq4, 1, R * Q4_BYTES, f);
    fwrite(wq6, 1, R * Q6_BYTES, f);
    fwrite(wk, 1, RK * Q4_BYTES, f);
    fwrite(wv, 1, RK * Q6_BYTES, f);
    fwrite(x, 4, C, f);
    fwrite(res, 4, R, f);
    fwrite(router, 4, (size_t)E * C, f);
    fwrite(x2, 4, C, f);
    fwrite(act, 4, (size_t)NT * C, f);
    fwrite(out, 4, 5 * R + R + 2 * RK + E, f);
    fwrite(idx, 4, K, f);
    fwrite(out + 5 * R + R + 2 * RK + E, 4, K, f);
    fwrite(out2, 4, R + 2 * RK + R + C + R, f);
    fwrite(q8, 1, q8_bytes, f);
    fwrite(out2 + (gout - d_out2), 4, (size_t)NT * R, f);

    /* ---- the attention chain of one decode layer, then sampling and the embedding ---- */
    const size_t nkv = (size_t)SEQ * NKV * HD;
    float *xin = malloc(HH * 4), *anorm = malloc(HH * 4), *qraw = malloc(NH * HD * 4);
    float *knraw = malloc(NKV * HD * 4), *vnraw = malloc(NKV * HD * 4), *qw = malloc(HD * 4), *kw = malloc(HD * 4);
    uint16_t *kc = malloc(nkv * 2), *vc = malloc(nkv * 2);
    int8_t *kc8 = malloc(nkv), *vc8 = malloc(nkv);
    float *ksc = malloc(SEQ * NKV * 4), *vsc = malloc(SEQ * NKV * 4), *lg = malloc(VOC * 4);
    uint8_t *table = malloc((size_t)VT * (HH / 256) * 144);
    for (int i = 0; i < HH; i++) { xin[i] = sym(2.0f); anorm[i] = 1.0f + sym(0.1f); }
    for (int i = 0; i < NH * HD; i++) qraw[i] = sym(2.0f);
    for (int i = 0; i < NKV * HD; i++) { knraw[i] = sym(2.0f); vnraw[i] = sym(2.0f); }
    for (int i = 0; i < HD; i++) { qw[i] = 1.0f + sym(0.1f); kw[i] = 1.0f + sym(0.1f); }
    for (size_t i = 0; i < nkv; i++) {
        kc[i] = kv_f16();
        vc[i] = kv_f16();
        kc8[i] = (int8_t)((int)(next32() % 255) - 127);
        vc8[i] = (int8_t)((int)(next32() % 255) - 127);
    }
    for (int i = 0; i < SEQ * NKV; i++) { ksc[i] = 0.001f + 0.01f * uniform(); vsc[i] = 0.001f + 0.01f * uniform(); }
    for (int i = 0; i < VOC; i++) lg[i] = sym(6.0f);
    fill_q4k(table, (size_t)VT * (HH / 256) / (C / 256)); /* VT rows of HH/256 blocks */
    float *d_xin = dev_copy(xin, HH * 4), *d_anorm = dev_copy(anorm, HH * 4), *d_q = dev_copy(qraw, NH * HD * 4);
    float *d_kn = dev_copy(knraw, NKV * HD * 4), *d_vn = dev_copy(vnraw, NKV * HD * 4);
    float *d_qw = dev_copy(qw, HD * 4), *d_kw = dev_copy(kw, HD * 4), *d_lg = dev_copy(lg, VOC * 4);
    uint16_t *d_kc = dev_copy(kc, nkv * 2), *d_vc = dev_copy(vc, nkv * 2);
    int8_t *d_kc8 = dev_copy(kc8, nkv), *d_vc8 = dev_copy(vc8, nkv);
    float *d_ksc = dev_copy(ksc, SEQ * NKV * 4), *d_vsc = dev_copy(vsc, SEQ * NKV * 4);
    void *d_table = dev_copy(table, (size_t)VT * (HH / 256) * 144);
    float *d_chain = NULL; /* normed, resid, normed2, radd [HH], att, att8 [NH*HD], emb [HH] */
    int *d_tok = NULL;
    const size_t n_chain = 5 * (size_t)HH + 2 * NH * HD;
    if (!d_xin || !d_anorm || !d_q || !d_kn || !d_vn || !d_qw || !d_kw || !d_lg || !d_kc || !d_vc || !d_kc8 ||
        !d_vc8 || !d_ksc || !d_vsc || !d_table || hipMalloc((void **)&d_chain, n_chain * 4) != hipSuccess ||
        hipMalloc((void **)&d_tok, 4) != hipSuccess) {
        fprintf(stderr, "hip allocation or copy failed (attention chain)\n");
        return 1;
    }
    float *normed = d_chain, *resid = normed + HH, *normed2 = resid + HH, *radd = normed2 + HH;
    float *att = radd + HH, *att8 = att + NH * HD, *emb = att8 + NH * HD;
    const float scale = 0.08838834764831845f; /* 1 / sqrt(128) */
    cuda_rms_norm_residual(d_xin, d_anorm, normed, resid, HH, 1e-6f, s);           /* forward.c:727 */
    cuda_rms_norm(d_xin, d_anorm, normed2, HH, 1e-6f, s);
    cuda_residual_add(d_xin, d_anorm, radd, HH, s);
    cuda_rms_norm_qk(d_q, d_kn, d_qw, d_kw, HD, NH, NKV, 1e-6f, s);                 /* forward.c:742 */
    cuda_rope(d_q, d_kn, HD, POS, 1e6f, NH, NKV, s);                                /* forward.c:748 */
    cuda_f32_to_f16_dual(d_kn, d_vn, d_kc + (size_t)POS * NKV * HD, d_vc + (size_t)POS * NKV * HD, NKV * HD, s);
    cuda_attention_f16kv(d_q, d_kc, d_vc, att, NH, HD, NKV, SEQ, NH / NKV, scale, s); /* forward.c:772 */
    cuda_f32_to_int8_kv_dual(d_kn, d_vn, d_kc8 + (size_t)POS * NKV * HD, d_vc8 + (size_t)POS * NKV * HD,
                             d_ksc + POS * NKV, d_vsc + POS * NKV, HD, NKV, s);
    cuda_attention_int8kv(d_q, d_kc8, d_vc8, d_ksc, d_vsc, att8, NH, HD, NKV, SEQ, NH / NKV, scale, s);
    float *d_qb = dev_copy(qraw, NH * HD * 4), *d_qbo = NULL;
    if (!d_qb || hipMalloc((void **)&d_qbo, NH * HD * 4) != hipSuccess) return 1;
    cuda_rms_norm_batched(d_qb, d_qw, d_qbo, HD, NH, 1e-6f, s);
    cuda_sample_token(d_lg, VOC, 0.8f, 0.9f, 12345ull, d_tok, s);                  /* forward.c:1703 */
    cuda_embedding_lookup_q4k(d_table, emb, 5, HH, (HH / 256) * 144, s);           /* forward.c:1160 */
    if (hipStreamSynchronize(s) != hipSuccess) return 1;
    if (mnemo_last_error() != MNEMO_OK) {
        fprintf(stderr, "library error: %s\n", mnemo_last_error_string());
        return 1;
    }
    float *chain = malloc(n_chain * 4), *qpost = malloc(NH * HD * 4), *kpost = malloc(NKV * HD * 4);
    uint16_t *kc_o = malloc(nkv * 2), *vc_o = malloc(nkv * 2);
    int8_t *kc8_o = malloc(nkv), *vc8_o = malloc(nkv);
    float *ksc_o = malloc(SEQ * NKV * 4), *vsc_o = malloc(SEQ * NKV * 4);
    int tok = -1;
    if (hipMemcpy(chain, d_chain, n_chain * 4, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(qpost, d_q, NH * HD * 4, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(kpost, d_kn, NKV * HD * 4, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(kc_o, d_kc, nkv * 2, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(vc_o, d_vc, nkv * 2, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(kc8_o, d_kc8, nkv, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(vc8_o, d_vc8, nkv, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(ksc_o, d_ksc, SEQ * NKV * 4, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(vsc_o, d_vsc, SEQ * NKV * 4, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(&tok, d_tok, 4, hipMemcpyDeviceToHost) != hipSuccess)
        return 1;
    float *qb = malloc(NH * HD * 4);
    if (hipMemcpy(qb, d_qbo, NH * HD * 4, hipMemcpyDeviceToHost) != hipSuccess) return 1;
    const int32_t hdr2[7] = {HH, NH, NKV, HD, SEQ, VOC, VT};
    fwrite(hdr2, 4, 7, f);
    fwrite(xin, 4, HH, f);
    fwrite(anorm, 4, HH, f);
    fwrite(qraw, 4, NH * HD, f);
    fwrite(knraw, 4, NKV * HD, f);
    fwrite(vnraw, 4, NKV * HD, f);
    fwrite(qw, 4, HD, f);
    fwrite(kw, 4, HD, f);
    fwrite(kc, 2, nkv, f);
    fwrite(vc, 2, nkv, f);
    fwrite(kc8, 1, nkv, f);
    fwrite(vc8, 1, nkv, f);
    fwrite(ksc, 4, SEQ * NKV, f);
    fwrite(vsc, 4, SEQ * NKV, f);
    fwrite(lg, 4, VOC, f);
    fwrite(table, 1, (size_t)VT * (HH / 256) * 144, f);
    fwrite(chain, 4, n_chain, f);
    fwrite(qpost, 4, NH * HD, f);
    fwrite(kpost, 4, NKV * HD, f);
    fwrite(kc_o, 2, nkv, f);
    fwrite(vc_o, 2, nkv, f);
    fwrite(kc8_o, 1, nkv, f);
    fwrite(vc8_o, 1, nkv, f);
    fwrite(ksc_o, 4, SEQ * NKV, f);
    fwrite(vsc_o, 4, SEQ * NKV, f);
    fwrite(&tok, 4, 1, f);
    fwrite(qb, 4, NH * HD, f);
    fclose(f);
    printf("%s: ok\n", mnemo_version());
    return 0;
}
