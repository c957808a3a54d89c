/* cpu_baseline.c -- the CPU baseline bench.py times beside the GPU (a reported baseline,
 * never a checker and never the product).
 *
 * The reference has no CPU GEMV; this is the fused dequant+dot of its GPU kernels' arithmetic
 * (kernels.cu:114-136 for Q4_K: w = (d*sc)*q - dmin*m per weight; kernels.cu:455-486 for
 * Q6_K: w = (d*sc)*(q - 32)) with fp32 accumulation, written so that the compiler
 * vectorises it: 32 independent partial sums per row (one per value of a sub-block),
 * unsigned-byte unpacking in plain loops, FMA contraction allowed.  The build compiles it
 * twice, for x86-64-v3 (AVX2) and x86-64-v4 (AVX-512); the loader picks what the host CPU
 * supports.  Rows are split over OpenMP threads.
 *
 * Unlike mnemo_oracle.c (the checker: no contraction, serial sums), results differ from
 * the IEEE restatement in the last bits; tests only hold them to a relative 1e-5.
 */
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define LANES 32 /* one sub-block: two AVX-512 (four AVX2) registers of fp32 partial sums */

static inline float f16_to_f32(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
    uint32_t u;
    if (e == 0) {
        float f = (float)m * (1.0f / 16777216.0f); /* 2^-24 */
        memcpy(&u, &f, 4);
        u |= s;
    } else if (e == 31) {
        u = s | 0x7F800000u | (m << 13);
    } else {
        u = s | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* the 6-bit scale and min of sub-block j (get_scale_min_k4, kernels.cu:45-53) */
static inline void scale_min(int j, const uint8_t *q, int *sc, int *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

static float dot_q4k_row(const uint8_t *p, const float *x, int bpr) {
    float part[LANES] = {0};
    for (int b = 0; b < bpr; b++, p += 144, x += 256) {
        const float d = f16_to_f32(rd16(p)), dmin = f16_to_f32(rd16(p + 2));
        const uint8_t *qs = p + 16;
        for (int g = 0; g < 4; g++) {
            int sc0, m0, sc1, m1;
            scale_min(2 * g, p + 4, &sc0, &m0);
            scale_min(2 * g + 1, p + 4, &sc1, &m1);
            const float d0 = d * (float)sc0, mf0 = dmin * (float)m0;
            const float d1 = d * (float)sc1, mf1 = dmin * (float)m1;
            const uint8_t *q = qs + 32 * g;
            const float *xa = x + 64 * g, *xb = xa + 32;
            for (int l = 0; l < LANES; l++) part[l] += (d0 * (float)(q[l] & 15) - mf0) * xa[l];
            for (int l = 0; l < LANES; l++) part[l] += (d1 * (float)(q[l] >> 4) - mf1) * xb[l];
        }
    }
    float s = 0.0f;
    for (int l = 0; l < LANES; l++) s += part[l];
    return s;
}

static float dot_q6k_row(const uint8_t *p, const float *x, int bpr) {
    float part[LANES] = {0};
    for (int b = 0; b < bpr; b++, p += 210, x += 256) {
        const uint8_t *ql = p, *qh = p + 128;
        const int8_t *sc = (const int8_t *)(p + 192);
        const float d = f16_to_f32(rd16(p + 208));
        for (int h = 0; h < 2; h++)
            for (int grp = 0; grp < 4; grp++) {
                const uint8_t *lq = ql + 64 * h + 32 * (grp & 1), *hq = qh + 32 * h;
                const int sh = grp >= 2 ? 4 : 0;
                const float *xv = x + 128 * h + 32 * grp;
                /* 16 values per scale */
                const float s0 = d * (float)sc[8 * h + 2 * grp], s1 = d * (float)sc[8 * h + 2 * grp + 1];
                for (int l = 0; l < 16; l++) {
                    const int q = (((hq[l] >> (2 * grp)) & 3) << 4 | ((lq[l] >> sh) & 15)) - 32;
                    part[l] += (s0 * (float)q) * xv[l];
                }
                for (int l = 16; l < 32; l++) {
                    const int q = (((hq[l] >> (2 * grp)) & 3) << 4 | ((lq[l] >> sh) & 15)) - 32;
                    part[l] += (s1 * (float)q) * xv[l];
                }
            }
    }
    float s = 0.0f;
    for (int l = 0; l < LANES; l++) s += part[l];
    return s;
}

/* y[r] = W[r] . x for Q4_K (12) or Q6_K (14) rows of n_cols (a multiple of 256) */
int mo_base_gemv(int type_id, const void *w, const float *x, float *y, int n_rows, int n_cols, int nthreads) {
    if (n_cols % 256 || (type_id != 12 && type_id != 14)) return -1;
    const int bpr = n_cols / 256;
    const size_t rb = (size_t)bpr * (type_id == 12 ? 144 : 210);
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
#endif
    for (int r = 0; r < n_rows; r++) {
        const uint8_t *p = (const uint8_t *)w + (size_t)r * rb;
        y[r] = type_id == 12 ? dot_q4k_row(p, x, bpr) : dot_q6k_row(p, x, bpr);
    }
    return 0;
}
