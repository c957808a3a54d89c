/*
 * mnemo_oracle_attn.c -- CPU restatement of MnemoCUDA's decode attention chain
 * (RMS norms, RoPE, KV-cache stores, attention over the cache).
 *
 * TEST INFRASTRUCTURE ONLY (see mnemo_oracle.h): the product library never loads it.
 *
 * Accumulations run in fp64 so that this is a reference for the fp32 kernels, not a
 * copy of their rounding.  Where the reference's arithmetic fixes an fp32 value that a
 * later step depends on discretely (RoPE frequencies and angles, the int8 KV scale and
 * its rounding), that step is restated in fp32 exactly as the reference writes it.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "mnemo_oracle.h"

/* rms_norm_kernel (kernels.cu:692-722): out = in * rsqrt(mean(in^2) + eps) * w. */
void mo_rms_norm(const float *in, const float *w, float *out, int n, float eps) {
    double ss = 0.0;
    for (int i = 0; i < n; i++) ss += (double)in[i] * in[i];
    const double scale = 1.0 / sqrt(ss / n + (double)eps);
    for (int i = 0; i < n; i++) out[i] = (float)((double)in[i] * scale * w[i]);
}

/* rms_norm_residual_kernel (kernels.cu:725-749): the norm plus a copy of the input. */
void mo_rms_norm_residual(const float *in, const float *w, float *normed, float *residual, int n, float eps) {
    memcpy(residual, in, (size_t)n * sizeof(float));
    mo_rms_norm(in, w, normed, n, eps);
}

/* rms_norm_batched_kernel (kernels.cu:754-781) / rms_norm_qk_kernel (kernels.cu:1196-1219):
 * every head of head_dim values normalised with the shared weight vector. */
void mo_rms_norm_heads(const float *in, const float *w, float *out, int head_dim, int n_heads, float eps) {
    for (int h = 0; h < n_heads; h++) mo_rms_norm(in + (size_t)h * head_dim, w, out + (size_t)h * head_dim, head_dim, eps);
}

/* residual_add_kernel (kernels.cu:784-793). */
void mo_residual_add(const float *a, const float *b, float *out, int n) {
    for (int i = 0; i < n; i++) out[i] = a[i] + b[i];
}

/* RoPE (kernels.cu:818-852, frequencies kernels.cu:1256-1266): pairs (j, j + hd/2) of every
 * head rotated by angle pos * freq_j, freq_j = 1 / powf(theta, 2j / hd).  The frequency
 * and the angle are fp32 values as the reference computes them; the rotation is done in
 * fp64 with libm sin/cos of that fp32 angle. */
float mo_rope_freq(int j, int head_dim, float theta) {
    return 1.0f / powf(theta, (float)(2 * j) / (float)head_dim);
}
static void rope_vec(float *v, int n_heads, int head_dim, int pos, float theta) {
    const int half = head_dim / 2;
    for (int j = 0; j < half; j++) {
        const float angle = (float)pos * mo_rope_freq(j, head_dim, theta);
        const double c = cos((double)angle), s = sin((double)angle);
        for (int h = 0; h < n_heads; h++) {
            float *x = v + (size_t)h * head_dim;
            const double a = x[j], b = x[j + half];
            x[j] = (float)(a * c - b * s);
            x[j + half] = (float)(a * s + b * c);
        }
    }
}
void mo_rope(float *q, float *k, int head_dim, int pos, float theta, int n_heads_q, int n_heads_k) {
    rope_vec(q, n_heads_q, head_dim, pos, theta);
    rope_vec(k, n_heads_k, head_dim, pos, theta);
}

/* f32_to_int8_kv_kernel (kernels.cu:1339-1377): per head, absmax a; inv = 127.0f / a and
 * scale = a / 127.0f in fp32; q = round-half-even(x * inv) clamped to [-127, 127]. */
void mo_kv_quant_int8(const float *in, int8_t *out, float *scales, int head_dim, int n_kv_heads) {
    for (int h = 0; h < n_kv_heads; h++) {
        const float *x = in + (size_t)h * head_dim;
        float a = 0.0f;
        for (int d = 0; d < head_dim; d++) a = fmaxf(a, fabsf(x[d]));
        const float inv = a > 0.0f ? 127.0f / a : 0.0f;
        scales[h] = a > 0.0f ? a / 127.0f : 0.0f;
        for (int d = 0; d < head_dim; d++) {
            const float p = x[d] * inv;
            float r = nearbyintf(p); /* default rounding mode: to nearest, ties to even */
            if (r > 127.0f) r = 127.0f;
            if (r < -127.0f) r = -127.0f;
            out[(size_t)h * head_dim + d] = (int8_t)r;
        }
    }
}

/* attention_kernel_f16kv (kernels.cu:1550-1660) and attention_kernel_int8kv
 * (kernels.cu:1382-1481): for every query head h (kv head h / gqa), exact softmax over
 * positions 0..seq_len-1 of scale * q.k_p, out = sum_p softmax_p v_p.  The cache is
 * [pos][n_kv_heads][head_dim]; kv_type 0 = f16 bits, 1 = int8 with per (pos, kv head)
 * scales in k_scales / v_scales. */
int mo_attention(const float *q, const void *kv_k, const void *kv_v, const float *k_scales,
                 const float *v_scales, int kv_type, float *out, int n_heads, int head_dim,
                 int n_kv_heads, int seq_len, int gqa, float scale) {
    if (head_dim <= 0 || head_dim > MO_ATTN_MAX_HD || gqa <= 0) return -1;
    const size_t stride = (size_t)n_kv_heads * head_dim;
    for (int h = 0; h < n_heads; h++) {
        const int kvh = h / gqa;
        const float *qh = q + (size_t)h * head_dim;
        double mx = -INFINITY;
        /* two passes over the positions: max, then sum and weighted V */
        for (int p = 0; p < seq_len; p++) {
            double s = 0.0;
            for (int d = 0; d < head_dim; d++) {
                const size_t o = (size_t)p * stride + (size_t)kvh * head_dim + d;
                const double kd = kv_type == 0 ? mo_f16_to_f32(((const uint16_t *)kv_k)[o])
                                               : (double)((const int8_t *)kv_k)[o] * k_scales[(size_t)p * n_kv_heads + kvh];
                s += qh[d] * kd;
            }
            s *= scale;
            if (s > mx) mx = s;
        }
        double sum = 0.0;
        double acc[MO_ATTN_MAX_HD];
        for (int d = 0; d < head_dim; d++) acc[d] = 0.0;
        for (int p = 0; p < seq_len; p++) {
            double s = 0.0;
            for (int d = 0; d < head_dim; d++) {
                const size_t o = (size_t)p * stride + (size_t)kvh * head_dim + d;
                const double kd = kv_type == 0 ? mo_f16_to_f32(((const uint16_t *)kv_k)[o])
                                               : (double)((const int8_t *)kv_k)[o] * k_scales[(size_t)p * n_kv_heads + kvh];
                s += qh[d] * kd;
            }
            const double e = exp(s * scale - mx);
            sum += e;
            for (int d = 0; d < head_dim; d++) {
                const size_t o = (size_t)p * stride + (size_t)kvh * head_dim + d;
                const double vd = kv_type == 0 ? mo_f16_to_f32(((const uint16_t *)kv_v)[o])
                                               : (double)((const int8_t *)kv_v)[o] * v_scales[(size_t)p * n_kv_heads + kvh];
                acc[d] += e * vd;
            }
        }
        for (int d = 0; d < head_dim; d++) out[(size_t)h * head_dim + d] = seq_len > 0 ? (float)(acc[d] / sum) : 0.0f;
    }
    return 0;
}
