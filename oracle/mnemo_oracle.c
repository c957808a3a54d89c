/*
 * mnemo_oracle.c -- CPU restatement of MnemoCUDA's quantized-matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product).  See mnemo_oracle.h for
 * how each routine is pinned.  Reference citations are file:line in MnemoCUDA's tree.
 */
#include "mnemo_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* IEEE binary16 -> binary32, exact for every pattern.  Same value as the GPU decoder
 * f16_to_f32 (kernels.cu:41-43, __half2float).  The reference's software decoder
 * (forward.c:1197-1208) agrees for all finite patterns; it has no Inf/NaN branch,
 * which the GPU path does have, so the GPU behaviour is followed for exp == 31. */
float mo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            /* subnormal: mant * 2^-24, exactly representable in fp32 */
            float f = (float)mant * (1.0f / 16777216.0f);
            memcpy(&bits, &f, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (mant << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

/* binary32 -> binary16, round to nearest even (the rounding of __float2half used by
 * the Q8_1 quantizer, gemm_q4k.cu:356). */
uint16_t mo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t absx = x & 0x7FFFFFFFu;
    if (absx >= 0x7F800000u) { /* Inf / NaN */
        if (absx == 0x7F800000u) return sign | 0x7C00u;
        return sign | 0x7E00u | (uint16_t)((absx >> 13) & 0x3FFu);
    }
    if (absx >= 0x477FF000u) /* rounds to >= 65520 -> Inf */
        return sign | 0x7C00u;
    int e = (int)(absx >> 23) - 127;
    if (e < -25) return sign; /* below half the smallest subnormal */
    if (e < -14) {
        /* subnormal result: value = m * 2^-24, m = round(abs * 2^24) */
        uint32_t m = (absx & 0x7FFFFFu) | 0x800000u; /* 24-bit significand, value m*2^(e-23) */
        int shift = -e - 1;                             /* (e-23) + 24 = e + 1 -> shift right by -(e+1) */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (q & 1u))) q++;
        return sign | (uint16_t)q;
    }
    uint32_t mant = absx & 0x7FFFFFu;
    uint32_t q = ((uint32_t)(e + 15) << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++; /* carry may bump the exponent */
    return sign | (uint16_t)q;
}

/* 6-bit (scale, min) of sub-block j from the 12 packed bytes.
 * Restates get_scale_min_k4, kernels.cu:45-53 (same logic forward.c:1213-1224). */
void mo_get_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* One Q4_K super-block (144 B: f16 d, f16 dmin, 12 B scales, 128 B qs) -> 256 floats.
 * Value v: pair g = v/64 uses qs[32g + v%32]; low nibble for v%64 < 32 (sub-block 2g),
 * high nibble otherwise (sub-block 2g+1); w = (d*sc)*q - (dmin*m) in fp32.
 * Restates kernels.cu:20-25 (layout), kernels.cu:114-136 (index/arith) and the linear
 * form forward.c:1212-1228.  d*sc, (d*sc)*q and dmin*m are exact in fp32, so the single
 * rounding is the final subtraction whether or not it is fused. */
static void deq_q4k_block(const uint8_t *b, float *out) {
    float d = mo_f16_to_f32(rd16(b));
    float dmin = mo_f16_to_f32(rd16(b + 2));
    const uint8_t *scales = b + 4;
    const uint8_t *qs = b + 16;
    for (int g = 0; g < 4; g++) {
        uint8_t sc0, m0, sc1, m1;
        mo_get_scale_min_k4(2 * g, scales, &sc0, &m0);
        mo_get_scale_min_k4(2 * g + 1, scales, &sc1, &m1);
        float d0 = d * (float)sc0, mf0 = dmin * (float)m0;
        float d1 = d * (float)sc1, mf1 = dmin * (float)m1;
        for (int l = 0; l < 32; l++) {
            uint8_t byte = qs[32 * g + l];
            out[64 * g + l] = d0 * (float)(byte & 0x0F) - mf0;
            out[64 * g + 32 + l] = d1 * (float)(byte >> 4) - mf1;
        }
    }
}

/* One Q6_K super-block (210 B: ql[128], qh[64], int8 scales[16], f16 d) -> 256 floats.
 * Value v: half h = v/128, u = v%128, grp = u/32, l = u%32;
 *   lo4 = (ql[64h + 32(grp&1) + l] >> (grp>=2 ? 4 : 0)) & 15
 *   hi2 = (qh[32h + l] >> 2grp) & 3
 *   w   = (d * scales[v/16]) * ((hi2<<4 | lo4) - 32)
 * Restates kernels.cu:27-32, 455-486 and tools/validate_dequant.py:253-319. */
static void deq_q6k_block(const uint8_t *b, float *out) {
    const uint8_t *ql = b;
    const uint8_t *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    float d = mo_f16_to_f32(rd16(b + 208));
    for (int v = 0; v < 256; v++) {
        int h = v / 128, u = v % 128, grp = u / 32, l = u % 32;
        int lo4 = (ql[64 * h + 32 * (grp & 1) + l] >> (grp >= 2 ? 4 : 0)) & 15;
        int hi2 = (qh[32 * h + l] >> (2 * grp)) & 3;
        int q = ((hi2 << 4) | lo4) - 32;
        float s = d * (float)sc[v / 16];
        out[v] = s * (float)q;
    }
}

static void deq_rows(const void *w, float *out, int n_rows, int n_cols, int blk_bytes,
                     void (*blk)(const uint8_t *, float *)) {
    int bpr = (n_cols + 255) / 256;
    float tmp[256];
    const uint8_t *p = (const uint8_t *)w;
    for (int r = 0; r < n_rows; r++) {
        for (int b = 0; b < bpr; b++) {
            blk(p + ((size_t)r * bpr + b) * blk_bytes, tmp);
            int n = n_cols - b * 256;
            if (n > 256) n = 256;
            memcpy(out + (size_t)r * n_cols + (size_t)b * 256, tmp, (size_t)n * sizeof(float));
        }
    }
}

void mo_dequant_q4k(const void *w, float *out, int n_rows, int n_cols) {
    deq_rows(w, out, n_rows, n_cols, MO_Q4K_BYTES, deq_q4k_block);
}

void mo_dequant_q6k(const void *w, float *out, int n_rows, int n_cols) {
    deq_rows(w, out, n_rows, n_cols, MO_Q6K_BYTES, deq_q6k_block);
}

int mo_dequant(int type_id, const void *w, float *out, int n_rows, int n_cols) {
    switch (type_id) {
    case MO_TYPE_F32:
        memcpy(out, w, (size_t)n_rows * n_cols * sizeof(float));
        return 0;
    case MO_TYPE_Q4K: mo_dequant_q4k(w, out, n_rows, n_cols); return 0;
    case MO_TYPE_Q6K: mo_dequant_q6k(w, out, n_rows, n_cols); return 0;
    default: return -1;
    }
}

static size_t row_bytes(int type_id, int n_cols) {
    int bpr = (n_cols + 255) / 256;
    switch (type_id) {
    case MO_TYPE_F32: return (size_t)n_cols * 4;
    case MO_TYPE_Q4K: return (size_t)bpr * MO_Q4K_BYTES;
    case MO_TYPE_Q6K: return (size_t)bpr * MO_Q6K_BYTES;
    default: return 0;
    }
}

/* y = W x in fp64 over the fp32 dequantised weights (the exact value every GEMV
 * entry point -- kernels.cu:66, 149, 205, 278, 358, 427 -- approximates). */
int mo_gemv(int type_id, const void *w, const float *x, double *y, int n_rows, int n_cols) {
    size_t rb = row_bytes(type_id, n_cols);
    if (!rb) return -1;
    float *row = (float *)malloc((size_t)n_cols * sizeof(float));
    if (!row) return -2;
    for (int r = 0; r < n_rows; r++) {
        mo_dequant(type_id, (const uint8_t *)w + (size_t)r * rb, row, 1, n_cols);
        double acc = 0.0;
        for (int c = 0; c < n_cols; c++) acc += (double)row[c] * (double)x[c];
        y[r] = acc;
    }
    free(row);
    return 0;
}

/* CPU baseline with the reference GPU kernel's arithmetic: per weight
 * (d*sc*q - dmin*m) * x accumulated in fp32 (kernels.cu:114-136 / 455-486), one
 * accumulator per row, rows split over OpenMP threads. */
int mo_gemv_f32acc(int type_id, const void *w, const float *x, float *y, int n_rows,
                   int n_cols, int nthreads) {
    size_t rb = row_bytes(type_id, n_cols);
    if (!rb || type_id == MO_TYPE_F32) return -1;
    int bpr = (n_cols + 255) / 256;
    if (n_cols % 256) return -3; /* baseline is only timed on whole super-blocks */
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
#endif
    for (int r = 0; r < n_rows; r++) {
        const uint8_t *p = (const uint8_t *)w + (size_t)r * rb;
        float tmp[256];
        float acc = 0.0f;
        for (int b = 0; b < bpr; b++) {
            if (type_id == MO_TYPE_Q4K)
                deq_q4k_block(p + (size_t)b * MO_Q4K_BYTES, tmp);
            else
                deq_q6k_block(p + (size_t)b * MO_Q6K_BYTES, tmp);
            const float *xb = x + (size_t)b * 256;
            float s = 0.0f;
            for (int i = 0; i < 256; i++) s += tmp[i] * xb[i];
            acc += s;
        }
        y[r] = acc;
    }
    return 0;
}

/* Router logits z = W_r x, W_r fp32 row-major [n_rows][n_cols] (kernels.cu:859-880). */
void mo_matvec_f32(const float *w, const float *x, double *y, int n_rows, int n_cols) {
    for (int r = 0; r < n_rows; r++) {
        double acc = 0.0;
        for (int c = 0; c < n_cols; c++) acc += (double)w[(size_t)r * n_cols + c] * (double)x[c];
        y[r] = acc;
    }
}

/* Top-k of n_experts scores, then softmax over the k selected (normalised top-k).
 * Restates topk_softmax_kernel, kernels.cu:993-1057.  Selection order is defined as
 * (value descending, index ascending); the reference emits its k winners in an
 * implementation-dependent slot order, so only the index SET and the (index, weight)
 * pairing are comparable with it.  As in the reference, candidates <= -1e30 are never
 * selected and unfilled slots give index -1, weight 0. */
void mo_topk_softmax(const float *scores, int n_experts, int k, int *idx, float *wts) {
    float vals[64];
    int ids[64];
    if (k > 64) k = 64;
    for (int i = 0; i < k; i++) { vals[i] = -1e30f; ids[i] = -1; }
    for (int j = 0; j < n_experts; j++) {
        float v = scores[j];
        if (!(v > -1e30f)) continue;
        /* insertion into a list sorted by (value desc, index asc) */
        int pos = k;
        for (int i = 0; i < k; i++) {
            if (ids[i] < 0 || v > vals[i]) { pos = i; break; }
        }
        if (pos == k) continue;
        for (int i = k - 1; i > pos; i--) { vals[i] = vals[i - 1]; ids[i] = ids[i - 1]; }
        vals[pos] = v;
        ids[pos] = j;
    }
    double mx = -1e300;
    for (int i = 0; i < k; i++) if (ids[i] >= 0 && vals[i] > mx) mx = vals[i];
    double e[64], sum = 0.0;
    for (int i = 0; i < k; i++) {
        e[i] = ids[i] >= 0 ? exp((double)vals[i] - mx) : 0.0;
        sum += e[i];
    }
    for (int i = 0; i < k; i++) {
        idx[i] = ids[i];
        wts[i] = sum > 0.0 ? (float)(e[i] / sum) : 0.0f;
    }
}

/* out = silu(g) * u with the reference's fp32 expression (kernels.cu:677-688). */
void mo_swiglu(const float *g, const float *u, float *out, int n) {
    for (int i = 0; i < n; i++) {
        float gi = g[i];
        float silu = gi / (1.0f + expf(-gi));
        out[i] = silu * u[i];
    }
}

/* out += scale * x (kernels.cu:980-988). */
void mo_scaled_add(float *out, const float *x, float scale, int n) {
    for (int i = 0; i < n; i++) out[i] += scale * x[i];
}

/* fp32 [N][K] -> Q8_1 MMQ blocks [N][K/128] (144 B each: half2 ds4[4] then int8 qs[128]).
 * Per 32 values: amax, d = amax/127, id = 127/amax (0 if amax == 0),
 * q = rint_half_even(x*id) clamped to +-127, sum = sequential fp32 sum of x,
 * ds = (half(d), half(d*sum)).  Restates quantize_mmq_q8_1_kernel, gemm_q4k.cu:327-358,
 * including its second half2 component d*sum (llama.cpp's MMQ layout stores the plain
 * sum there; consumers in this project recompute the block sum from qs instead). */
void mo_quantize_q8_1_mmq(const float *src, void *dst, int K, int N) {
    int nsb = K / 128;
    uint8_t *out = (uint8_t *)dst;
    for (int col = 0; col < N; col++) {
        for (int sb = 0; sb < nsb; sb++) {
            const float *xs = src + (size_t)col * K + (size_t)sb * 128;
            uint8_t *blk = out + ((size_t)col * nsb + sb) * MO_Q8_1_MMQ_BYTES;
            for (int sub = 0; sub < 4; sub++) {
                const float *xb = xs + sub * 32;
                float amax = 0.0f;
                for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(xb[i]));
                float d = amax / 127.0f;
                float id = (amax > 0.0f) ? 127.0f / amax : 0.0f;
                float sum = 0.0f;
                for (int i = 0; i < 32; i++) {
                    float v = rintf(xb[i] * id); /* default FE_TONEAREST: half-even */
                    if (v > 127.0f) v = 127.0f;
                    if (v < -127.0f) v = -127.0f;
                    blk[16 + sub * 32 + i] = (uint8_t)(int8_t)(int)v;
                    sum += xb[i];
                }
                uint16_t hd = mo_f32_to_f16(d);
                uint16_t hs = mo_f32_to_f16(d * sum);
                blk[sub * 4 + 0] = (uint8_t)(hd & 0xFF);
                blk[sub * 4 + 1] = (uint8_t)(hd >> 8);
                blk[sub * 4 + 2] = (uint8_t)(hs & 0xFF);
                blk[sub * 4 + 3] = (uint8_t)(hs >> 8);
            }
        }
    }
}

/* dequant(Q8_1) value = float(half d) * q (gemm_q4k.cu:106-111 multiplies by ds.x). */
void mo_dequant_q8_1_mmq(const void *src, float *out, int K, int N) {
    int nsb = K / 128;
    const uint8_t *in = (const uint8_t *)src;
    for (int col = 0; col < N; col++)
        for (int sb = 0; sb < nsb; sb++) {
            const uint8_t *blk = in + ((size_t)col * nsb + sb) * MO_Q8_1_MMQ_BYTES;
            for (int sub = 0; sub < 4; sub++) {
                float d = mo_f16_to_f32(rd16(blk + sub * 4));
                for (int i = 0; i < 32; i++)
                    out[(size_t)col * K + sb * 128 + sub * 32 + i] =
                        d * (float)(int8_t)blk[16 + sub * 32 + i];
            }
        }
}

/* The Q4_K x Q8_1 product of gemm_q4k.cu:103-112, 164-166 in fp64, per 32-value
 * sub-block s of weight row i and token j:
 *     (d*sc_s) * d8_js * sum_{k in s} q_ik * q8_jk  -  (dmin*m_s) * ds_js
 * with ds_js the block's second half (d8 * sum of the unquantized values, the field
 * gemm_q4k.cu:166 multiplies by dmA.y).  d*sc and dmin*m are taken exactly (the reference
 * rounds them to f16, gemm_q4k.cu:106-111; the GEMV path keeps them in fp32,
 * kernels.cu:114-136). */
static void gemm_q4k_split(const uint8_t *w, const uint8_t *act, double *out, int M, int K, int N) {
    const int nb = K / 256, na = K / 128;
    for (int j = 0; j < N; j++)
        for (int i = 0; i < M; i++) {
            double acc = 0.0;
            for (int b = 0; b < nb; b++) {
                const uint8_t *blk = w + ((size_t)i * nb + b) * MO_Q4K_BYTES;
                const double d = mo_f16_to_f32(rd16(blk)), dmin = mo_f16_to_f32(rd16(blk + 2));
                for (int s = 0; s < 8; s++) {
                    uint8_t sc, m;
                    mo_get_scale_min_k4(s, blk + 4, &sc, &m);
                    const int sb = 2 * b + s / 4, sub = s % 4; /* Q8_1 block and sub-block */
                    const uint8_t *ab = act + ((size_t)j * na + sb) * MO_Q8_1_MMQ_BYTES;
                    const double d8 = mo_f16_to_f32(rd16(ab + 4 * sub));
                    const double ds = mo_f16_to_f32(rd16(ab + 4 * sub + 2));
                    long isum = 0;
                    for (int l = 0; l < 32; l++) {
                        const int q = (blk[16 + 32 * (s / 2) + l] >> (4 * (s % 2))) & 15;
                        isum += (long)q * (int8_t)ab[16 + 32 * sub + l];
                    }
                    acc += d * sc * d8 * (double)isum - dmin * m * ds;
                }
            }
            out[(size_t)j * M + i] = acc;
        }
}

/* out[j*M + i] (column-major [N][M] as gemm_q4k.cu:194): Q4_K in the split form above;
 * Q6_K (no min term) as the fp64 product of the dequantised operands,
 * sum_k deq(W)[i][k] * d8_j * q8_jk. */
int mo_gemm_q8_1(int type_id, const void *w, const void *act, double *out, int M, int K, int N) {
    if (K % 256) return -3;
    if (type_id == MO_TYPE_Q4K) {
        gemm_q4k_split((const uint8_t *)w, (const uint8_t *)act, out, M, K, N);
        return 0;
    }
    float *wd = (float *)malloc((size_t)M * K * sizeof(float));
    float *ad = (float *)malloc((size_t)N * K * sizeof(float));
    if (!wd || !ad) { free(wd); free(ad); return -2; }
    if (mo_dequant(type_id, w, wd, M, K)) { free(wd); free(ad); return -1; }
    mo_dequant_q8_1_mmq(act, ad, K, N);
    for (int j = 0; j < N; j++)
        for (int i = 0; i < M; i++) {
            const float *wr = wd + (size_t)i * K;
            const float *ar = ad + (size_t)j * K;
            double acc = 0.0;
            for (int k = 0; k < K; k++) acc += (double)wr[k] * (double)ar[k];
            out[(size_t)j * M + i] = acc;
        }
    free(wd);
    free(ad);
    return 0;
}

/* ---- next-token selection (kernels.cu:2020-2174) ---------------------------------------- */
uint64_t mo_xoroshiro_next(uint64_t *s0, uint64_t *s1) {
    /* kernels.cu:2134-2143: t = s0 ^ (s0 << 23); s0 = s1; s1 = t ^ s1 ^ (t >> 17) ^ (s1 >> 26) */
    const uint64_t t = *s0 ^ (*s0 << 23);
    *s0 = *s1;
    *s1 = t ^ *s1 ^ (t >> 17) ^ (*s1 >> 26);
    return *s0 + *s1;
}

int mo_sample_token(const float *logits, int V, float temperature, float top_p,
                    unsigned long long seed, float *u_out, float *nsum_out) {
    enum { BLOCK = 256, LK = 8, NC = BLOCK * LK };
    float gmax = -1e30f;                        /* kernels.cu:2038-2047 */
    for (int i = 0; i < V; i++) gmax = fmaxf(gmax, logits[i]);
    if (temperature <= 0.0f) {                  /* argmax, ties to the lower index */
        float bv = -1e30f;
        int bi = 0;
        for (int i = 0; i < V; i++)
            if (logits[i] > bv) { bv = logits[i]; bi = i; }
        return bi;
    }
    float csum[BLOCK];
    static float cand_p[NC];
    static int cand_id[NC];
    for (int t = 0; t < BLOCK; t++) {           /* kernels.cu:2075-2104: per thread t */
        float sum = 0.0f, hv[LK];
        int hid[LK];
        for (int k = 0; k < LK; k++) { hv[k] = -1.0f; hid[k] = -1; }
        for (int i = t; i < V; i += BLOCK) {
            const float p = expf((logits[i] - gmax) / temperature);
            sum += p;
            int mi = 0;
            for (int k = 1; k < LK; k++)
                if (hv[k] < hv[mi]) mi = k;
            if (p > hv[mi]) { hv[mi] = p; hid[mi] = i; }
        }
        csum[t] = sum;
        for (int k = 0; k < LK; k++) { cand_p[t * LK + k] = hv[k]; cand_id[t * LK + k] = hid[k]; }
    }
    for (int s = BLOCK / 2; s > 0; s >>= 1)     /* the tree of kernels.cu:2079-2083 */
        for (int t = 0; t < s; t++) csum[t] += csum[t + s];
    const float total = csum[0];
    uint64_t s0 = seed, s1 = seed ^ 0xDEADBEEFCAFEBABEull;  /* kernels.cu:2127-2143 */
    for (int w = 0; w < 3; w++) mo_xoroshiro_next(&s0, &s1);
    const float r = (float)(mo_xoroshiro_next(&s0, &s1) >> 11) * (1.0f / 9007199254740992.0f);
    const float mass = top_p * total;           /* kernels.cu:2145-2166: selection sort */
    float cumul = 0.0f;
    int n = 0;
    for (int pick = 0; pick < NC; pick++) {
        int best = pick;
        for (int j = pick + 1; j < NC; j++)
            if (cand_p[j] > cand_p[best]) best = j;
        if (cand_p[best] <= 0.0f) break;
        const float tp = cand_p[pick];
        const int ti = cand_id[pick];
        cand_p[pick] = cand_p[best]; cand_id[pick] = cand_id[best];
        cand_p[best] = tp; cand_id[best] = ti;
        cumul += cand_p[pick];
        n = pick + 1;
        if (cumul >= mass) break;
    }
    float nsum = 0.0f;                          /* kernels.cu:2168-2177 */
    for (int i = 0; i < n; i++) nsum += cand_p[i];
    const float target = r * nsum;
    float acc = 0.0f;
    int id = cand_id[0];
    for (int i = 0; i < n; i++) {
        acc += cand_p[i];
        if (acc >= target) { id = cand_id[i]; break; }
    }
    if (u_out) *u_out = r;
    if (nsum_out) *nsum_out = nsum;
    return id;
}
