// gemm.hip -- Q4_K / Q6_K x Q8_1 GEMM for prefill and batched experts (gfx950 MFMA).
//
// Semantics (MnemoCUDA gemm_q4k.cu:103-112, 164-166, 194):
//   out[j*M + i] = sum_k deq(W)[i][k] * deq(A)[j][k]
// with W GGUF blocks [M][K] and A the Q8_1 MMQ activations [N][K/128] x 144 B.
//
// Design: both operands are dequantised on the fly into f16 tiles in LDS and multiplied
// with v_mfma_f32_16x16x32_f16 (fp32 accumulate).  Per-32 scales of both operands are
// thereby folded into the values, so the MFMA accumulates across the whole K without any
// per-sub-block fp32 rescale in VALU (an int8 MFMA would need one cvt + two FMAs per
// output per 32-K step, which costs more VALU time than the MFMA saves).
//   * W value w = d*sc*q - dmin*m (Q4_K) or d*sc*(q-32) (Q6_K) is computed exactly in fp32
//     and rounded once to f16; A value d8*q8 likewise.  Expected relative L2 error vs the
//     fp64 product: ~4e-4 (two independent f16 roundings).
//   * Workgroup tile 128 weight rows x 128 tokens, 4 waves each owning 64 x 64
//     (4 x 4 MFMA tiles), K step 64 (= one Q4_K nibble group / one Q6_K ql group).
//   * LDS rows padded by 8 halves so the 16 lanes of an MFMA fragment read hit
//     different banks.
#include "mnemo_common.hpp"
#include "mnemo_internal.hpp"

namespace mnemo {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128;  // weight rows per workgroup
constexpr int kBN = 128;  // tokens per workgroup
constexpr int kKS = 64;   // K per step
constexpr int kLdsStride = kKS + 8;  // halves

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    h2 v = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, v);
}

// 32 weights of row `row` for K step `ks` (super-block ks/4, group g = ks%4), half `h`,
// written as f16 to dst (row of the LDS tile).  Q4_K: bytes [32g+16h, +16) of qs give
// 16 weights of sub-block 2g (columns 16h..16h+15 of the step) and 16 of sub-block 2g+1
// (columns 32+16h..).
__device__ __forceinline__ void deq_w_q4k(const uint8_t *__restrict__ wrow, int ks, int h,
                                          _Float16 *dst) {
    const uint8_t *blk = wrow + (size_t)(ks >> 2) * kQ4KBytes;
    const int g = ks & 3;
    const uint4 hdr = ld16(blk);
    const uint4 q = ld16(blk + 16 + 32 * g + 16 * h);
    const uint32_t s0 = hdr.y, s1 = hdr.z, s2 = hdr.w;
    uint32_t sc0, m0, sc1, m1;
    if (g < 2) {
        const int sh = 16 * g;
        sc0 = (s0 >> sh) & 63; m0 = (s1 >> sh) & 63;
        sc1 = (s0 >> (sh + 8)) & 63; m1 = (s1 >> (sh + 8)) & 63;
    } else {
        const int sh = 16 * (g - 2);
        sc0 = ((s2 >> sh) & 15) | (((s0 >> (sh + 6)) & 3) << 4);
        m0 = ((s2 >> (sh + 4)) & 15) | (((s1 >> (sh + 6)) & 3) << 4);
        sc1 = ((s2 >> (sh + 8)) & 15) | (((s0 >> (sh + 14)) & 3) << 4);
        m1 = ((s2 >> (sh + 12)) & 15) | (((s1 >> (sh + 14)) & 3) << 4);
    }
    const float d = h2f(hdr.x & 0xFFFFu), dmin = h2f(hdr.x >> 16);
    const float a0 = d * (float)sc0, b0 = dmin * (float)m0;
    const float a1 = d * (float)sc1, b1 = dmin * (float)m1;
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t v = w[k];
        float l0 = a0 * (float)(v & 15) - b0, l1 = a0 * (float)((v >> 8) & 15) - b0;
        float l2 = a0 * (float)((v >> 16) & 15) - b0, l3 = a0 * (float)((v >> 24) & 15) - b0;
        float h0 = a1 * (float)((v >> 4) & 15) - b1, h1 = a1 * (float)((v >> 12) & 15) - b1;
        float h2_ = a1 * (float)((v >> 20) & 15) - b1, h3 = a1 * (float)((v >> 28) & 15) - b1;
        lo[2 * k] = pack_h2(l0, l1); lo[2 * k + 1] = pack_h2(l2, l3);
        hi[2 * k] = pack_h2(h0, h1); hi[2 * k + 1] = pack_h2(h2_, h3);
    }
    uint4 *dl = (uint4 *)(dst + 16 * h);
    uint4 *dh = (uint4 *)(dst + 32 + 16 * h);
    dl[0] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    dl[1] = make_uint4(lo[4], lo[5], lo[6], lo[7]);
    dh[0] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    dh[1] = make_uint4(hi[4], hi[5], hi[6], hi[7]);
}

// Q6_K: K step ks covers values 64*(ks%4) .. +63 of super-block ks/4, i.e. half
// hh = (ks%4)/2 and groups 2*(ks%2), 2*(ks%2)+1.  Half h takes group grp = 2*(ks%2) + h:
// ql bytes [64hh + 32h, +32) (low nibbles if grp < 2 else high), qh bytes [32hh, +32)
// shifted by 2*grp; columns 32h .. 32h+31 of the step.
__device__ __forceinline__ void deq_w_q6k(const uint8_t *__restrict__ wrow, int ks, int h,
                                          _Float16 *dst) {
    const uint8_t *blk = wrow + (size_t)(ks >> 2) * kQ6KBytes;
    const int g = ks & 3, hh = g >> 1, grp = 2 * (g & 1) + h;
    const uint4 l0 = ld16(blk + 64 * hh + 32 * h), l1 = ld16(blk + 64 * hh + 32 * h + 16);
    const uint4 q0 = ld16(blk + 128 + 32 * hh), q1 = ld16(blk + 128 + 32 * hh + 16);
    const int8_t *sc = (const int8_t *)(blk + 192 + 8 * hh + 2 * grp);
    const float d = h2f((uint32_t)blk[208] | ((uint32_t)blk[209] << 8));
    const float s0 = d * (float)sc[0], s1 = d * (float)sc[1];
    const uint32_t ql[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
    const uint32_t qh[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    const int shl = grp >= 2 ? 4 : 0, shh = 2 * grp;
    uint32_t o[16];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const float s = k < 4 ? s0 : s1;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int lo4 = (ql[k] >> (8 * e + shl)) & 15;
            const int hi2 = (qh[k] >> (8 * e + shh)) & 3;
            v[e] = s * (float)(((hi2 << 4) | lo4) - 32);
        }
        o[2 * k] = pack_h2(v[0], v[1]);
        o[2 * k + 1] = pack_h2(v[2], v[3]);
    }
    uint4 *dd = (uint4 *)(dst + 32 * h);
#pragma unroll
    for (int k = 0; k < 4; k++) dd[k] = make_uint4(o[4 * k], o[4 * k + 1], o[4 * k + 2], o[4 * k + 3]);
}

// 32 activations (one Q8_1 sub-block) of token row `arow` for K step ks, half h:
// values ks*64 + 32h .. +31 -> columns 32h.. of the step.
__device__ __forceinline__ void deq_a_q81(const uint8_t *__restrict__ arow, int ks, int h, _Float16 *dst) {
    const int v0 = ks * kKS + 32 * h;
    const uint8_t *blk = arow + (size_t)(v0 >> 7) * kQ81Bytes;
    const int sub = (v0 >> 5) & 3;
    const float d = h2f(*(const uint16_t *)(blk + 4 * sub));
    const uint4 a = ld16(blk + 16 + 32 * sub), b = ld16(blk + 32 + 32 * sub);
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t o[16];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int x0 = (int8_t)(w[k] & 0xFF), x1 = (int8_t)((w[k] >> 8) & 0xFF);
        const int x2 = (int8_t)((w[k] >> 16) & 0xFF), x3 = (int8_t)(w[k] >> 24);
        o[2 * k] = pack_h2(d * (float)x0, d * (float)x1);
        o[2 * k + 1] = pack_h2(d * (float)x2, d * (float)x3);
    }
    uint4 *dd = (uint4 *)(dst + 32 * h);
#pragma unroll
    for (int k = 0; k < 4; k++) dd[k] = make_uint4(o[4 * k], o[4 * k + 1], o[4 * k + 2], o[4 * k + 3]);
}

template <int TYPE>
__global__ void __launch_bounds__(256) gemm_q8_1_kernel(const uint8_t *__restrict__ W,
                                                         const uint8_t *__restrict__ A,
                                                         float *__restrict__ out, int M, int K, int N) {
    __shared__ __align__(16) _Float16 As[kBM * kLdsStride];
    __shared__ __align__(16) _Float16 Bs[kBN * kLdsStride];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int i0 = blockIdx.x * kBM, j0 = blockIdx.y * kBN;
    const int wi = (wave & 1) * 64, wj = (wave >> 1) * 64;
    const int bpr = K / 256;
    const size_t wrow_bytes = (size_t)bpr * (TYPE == kTypeQ4K ? kQ4KBytes : kQ6KBytes);
    const size_t arow_bytes = (size_t)(K / 128) * kQ81Bytes;

    // loader roles: thread -> (row, half)
    const int lr = tid >> 1, lh = tid & 1;
    const int wr = min(i0 + lr, M - 1), ar = min(j0 + lr, N - 1);
    const uint8_t *wrow = W + (size_t)wr * wrow_bytes;
    const uint8_t *arow = A + (size_t)ar * arow_bytes;

    f4 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};

    const int nks = K / kKS;
    for (int ks = 0; ks < nks; ks++) {
        if (TYPE == kTypeQ4K) deq_w_q4k(wrow, ks, lh, As + lr * kLdsStride);
        else deq_w_q6k(wrow, ks, lh, As + lr * kLdsStride);
        deq_a_q81(arow, ks, lh, Bs + lr * kLdsStride);
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kKS; kk += 32) {
            h8 af[4], bf[4];
            const int ko = kk + 8 * (lane >> 4);
#pragma unroll
            for (int t = 0; t < 4; t++) {
                af[t] = *(const h8 *)(As + (wi + 16 * t + (lane & 15)) * kLdsStride + ko);
                bf[t] = *(const h8 *)(Bs + (wj + 16 * t + (lane & 15)) * kLdsStride + ko);
            }
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < 4; b++)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[a], bf[b], acc[a][b], 0, 0, 0);
        }
        __syncthreads();
    }
    // D layout (16x16 f32): lane l holds rows 4*(l/16)+e, column l%16.
    // Rows index weights i (A operand), columns tokens j (B operand).
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int j = j0 + wj + 16 * b + (lane & 15);
            const int ib = i0 + wi + 16 * a + 4 * (lane >> 4);
            if (j >= N) continue;
            float *o = out + (size_t)j * M + ib;
            if (ib + 3 < M && ((M & 3) == 0)) {
                *(f4 *)o = acc[a][b];
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (ib + e < M) o[e] = acc[a][b][e];
            }
        }
}

int launch_gemm_q8_1(int type, const void *w, const void *act, float *out, int M, int K, int N,
                     hipStream_t stream) {
    if (!w || !act || !out || M <= 0 || N <= 0 || K <= 0 || K % 256 != 0)
        return set_error(kErrBadArg, "gemm: need non-null pointers, M, N > 0 and K %% 256 == 0");
    if (type != kTypeQ4K && type != kTypeQ6K) return set_error(kErrUnsupportedType, "gemm: unsupported type %d", type);
    if (((uintptr_t)out & 15) != 0 && (M & 3) == 0)
        return set_error(kErrBadArg, "gemm: output must be 16-byte aligned");
    dim3 grid((M + kBM - 1) / kBM, (N + kBN - 1) / kBN);
    if (type == kTypeQ4K)
        hipLaunchKernelGGL(gemm_q8_1_kernel<kTypeQ4K>, grid, dim3(256), 0, stream, (const uint8_t *)w,
                           (const uint8_t *)act, out, M, K, N);
    else
        hipLaunchKernelGGL(gemm_q8_1_kernel<kTypeQ6K>, grid, dim3(256), 0, stream, (const uint8_t *)w,
                           (const uint8_t *)act, out, M, K, N);
    return check_launch("gemm_q8_1");
}

}  // namespace mnemo
