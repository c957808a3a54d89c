// router.hip -- fp32 router matvec, top-k softmax, expert glue and the Q8_1 quantizer.
//
//  * matvec_f32      (MnemoCUDA kernels.cu:859-880): one wave per router row, 16-byte
//                    loads, fp32 FMA, DPP row reduction.
//  * topk_softmax    (kernels.cu:993-1057): one wave; k rounds of a wave-wide arg-max
//                    ordered by (value desc, index asc), then softmax over the winners.
//                    Winners are written in that order (the reference's order is its
//                    slot order, so only the (index, weight) pairs are comparable).
//  * swiglu / scaled_add (kernels.cu:677-688, 980-988): elementwise, float4.
//  * quantize_q8_1   (gemm_q4k.cu:327-358): one thread per 32 values, same operation
//                    order as the reference so the bytes match exactly.
#include "mnemo_common.hpp"
#include "mnemo_internal.hpp"

namespace mnemo {

__global__ void __launch_bounds__(256) matvec_f32_kernel(const float *__restrict__ w,
                                                         const float *__restrict__ x,
                                                         float *__restrict__ y, int n_rows,
                                                         int n_cols, int vec4) {
    const int lane = lane_id();
    const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    float acc = 0.0f;
    if (row < n_rows) {
        const float *wr = w + (size_t)row * n_cols;
        if (vec4) {
            typedef float fv4 __attribute__((ext_vector_type(4)));
            const fv4 *w4 = (const fv4 *)wr;
            const fv4 *x4 = (const fv4 *)x;
            for (int c = lane; c < n_cols / 4; c += 64) {
                fv4 a = __builtin_nontemporal_load(w4 + c), b = x4[c];
                acc = fmaf(a.x, b.x, acc);
                acc = fmaf(a.y, b.y, acc);
                acc = fmaf(a.z, b.z, acc);
                acc = fmaf(a.w, b.w, acc);
            }
        } else {
            for (int c = lane; c < n_cols; c += 64) acc = fmaf(wr[c], x[c], acc);
        }
    }
    acc = sum64_lane63(acc);
    if (lane == 63 && row < n_rows) y[row] = acc;
}

int launch_matvec_f32(const float *w, const float *x, float *y, int n_rows, int n_cols,
                      hipStream_t stream) {
    if (!w || !x || !y || n_rows <= 0 || n_cols <= 0) return set_error(kErrBadArg, "matvec_f32: bad arguments");
    const int vec4 = (n_cols % 4 == 0) && (((uintptr_t)w | (uintptr_t)x) % 16 == 0);
    const int wpb = 4;
    hipLaunchKernelGGL(matvec_f32_kernel, dim3((n_rows + wpb - 1) / wpb), dim3(64 * wpb), 0, stream,
                       w, x, y, n_rows, n_cols, vec4);
    return check_launch("matvec_f32");
}

// ---------------------------------------------------------------- top-k softmax
constexpr int kTopkMaxPerLane = 16;  // n_experts <= 1024
constexpr int kTopkMaxK = 16;        // the reference's register budget (kernels.cu:1002)

__device__ __forceinline__ bool better(float v, int i, float v2, int i2) {
    return (v > v2) || (v == v2 && i < i2);
}

__device__ void topk_wave(const float *scores, int n, int k, int *idx, float *wts, float *vals_out) {
    const int lane = lane_id();
    float v[kTopkMaxPerLane];
#pragma unroll
    for (int t = 0; t < kTopkMaxPerLane; t++) {
        const int j = lane + 64 * t;
        const float s = j < n ? scores[j] : -1e30f;
        v[t] = (s > -1e30f) ? s : -1e30f;  // NaN and <= -1e30 never win (kernels.cu:1035)
    }
    float top_v[kTopkMaxK];
    int top_i[kTopkMaxK];
    for (int r = 0; r < k; r++) {
        float bv = -1e30f;
        int bi = 0x7FFFFFFF;
#pragma unroll
        for (int t = 0; t < kTopkMaxPerLane; t++) {
            const int j = lane + 64 * t;
            if (v[t] > -1e30f && better(v[t], j, bv, bi)) { bv = v[t]; bi = j; }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o);
            const int oi = __shfl_xor(bi, o);
            if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
        }
        const bool valid = bv > -1e30f;
        top_v[r] = bv;
        top_i[r] = valid ? bi : -1;
        if (valid && (bi & 63) == lane) {
#pragma unroll
            for (int t = 0; t < kTopkMaxPerLane; t++)
                if (bi == lane + 64 * t) v[t] = -1e30f;
        }
    }
    if (lane == 0) {
        const float mx = top_v[0];
        float e[kTopkMaxK], sum = 0.0f;
        for (int r = 0; r < k; r++) {
            e[r] = top_i[r] >= 0 ? expf(top_v[r] - mx) : 0.0f;
            sum += e[r];
        }
        for (int r = 0; r < k; r++) {
            idx[r] = top_i[r];
            wts[r] = sum > 0.0f ? e[r] / sum : 0.0f;
            if (vals_out) vals_out[r] = top_v[r];
        }
    }
}

__global__ void __launch_bounds__(64) topk_softmax_kernel(const float *__restrict__ scores,
                                                          int *__restrict__ idx,
                                                          float *__restrict__ wts, int n, int k) {
    topk_wave(scores, n, k, idx, wts, nullptr);
}

int launch_topk_softmax(const float *scores, int *idx, float *wts, int n, int k, hipStream_t stream) {
    if (!scores || !idx || !wts || n <= 0 || k <= 0 || k > kTopkMaxK || n > 64 * kTopkMaxPerLane)
        return set_error(kErrBadArg, "topk_softmax: need 0 < k <= %d, 0 < n_experts <= %d", kTopkMaxK,
                         64 * kTopkMaxPerLane);
    hipLaunchKernelGGL(topk_softmax_kernel, dim3(1), dim3(64), 0, stream, scores, idx, wts, n, k);
    return check_launch("topk_softmax");
}

// ---------------------------------------------------------------- elementwise glue
__global__ void swiglu_kernel(const float *__restrict__ g, const float *__restrict__ u,
                              float *__restrict__ out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float gi = g[i];
        out[i] = gi / (1.0f + expf(-gi)) * u[i];
    }
}

__global__ void scaled_add_kernel(float *__restrict__ out, const float *__restrict__ x, float s, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] += s * x[i];
}

int launch_swiglu(const float *g, const float *u, float *out, int n, hipStream_t stream) {
    if (!g || !u || !out || n <= 0) return set_error(kErrBadArg, "swiglu: bad arguments");
    hipLaunchKernelGGL(swiglu_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, g, u, out, n);
    return check_launch("swiglu");
}

int launch_scaled_add(float *out, const float *x, float s, int n, hipStream_t stream) {
    if (!out || !x || n <= 0) return set_error(kErrBadArg, "scaled_add: bad arguments");
    hipLaunchKernelGGL(scaled_add_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, out, x, s, n);
    return check_launch("scaled_add");
}

// ---------------------------------------------------------------- Q8_1 quantizer
// dst: [N][K/128] blocks of {half2 ds4[4]; int8 qs[128]}.  One thread per (column,
// 32-value sub-block); the sum runs sequentially in value order, as the reference's.
__global__ void __launch_bounds__(256) quantize_q8_1_kernel(const float *__restrict__ src,
                                                            uint8_t *__restrict__ dst, int K, int N) {
    const int nsub = K / 32;
    const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (long)nsub * N) return;
    const int col = (int)(t / nsub), s32 = (int)(t % nsub);
    const float4 *xb4 = (const float4 *)(src + (size_t)col * K + (size_t)s32 * 32);
    float xv[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        float4 v = xb4[i];
        xv[4 * i] = v.x; xv[4 * i + 1] = v.y; xv[4 * i + 2] = v.z; xv[4 * i + 3] = v.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(xv[i]));
    const float d = amax / 127.0f;
    const float id = (amax > 0.0f) ? 127.0f / amax : 0.0f;
    float sum = 0.0f;
    uint32_t q[8];
#pragma unroll
    for (int i = 0; i < 8; i++) q[i] = 0;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        float r = rintf(xv[i] * id);
        r = fminf(fmaxf(r, -127.0f), 127.0f);
        q[i >> 2] |= ((uint32_t)(int)r & 0xFFu) << (8 * (i & 3));
        sum += xv[i];
    }
    uint8_t *blk = dst + ((size_t)col * (K / 128) + s32 / 4) * kQ81Bytes;
    const int sub = s32 & 3;
    // Round d*sum to fp32 first, then to f16 (two roundings, as the reference's
    // __float2half(d * sum)); the barrier stops the f32 multiply and the f16 conversion
    // from being fused into one v_fma_mix with a single rounding.
    float dsum = d * sum;
    asm volatile("" : "+v"(dsum));
    const uint32_t ds = (uint32_t)f2h_bits(d) | ((uint32_t)f2h_bits(dsum) << 16);
    *(uint32_t *)(blk + 4 * sub) = ds;
    uint4 *qd = (uint4 *)(blk + 16 + 32 * sub);
    qd[0] = make_uint4(q[0], q[1], q[2], q[3]);
    qd[1] = make_uint4(q[4], q[5], q[6], q[7]);
}

int launch_quantize_q8_1(const float *src, void *dst, int K, int N, hipStream_t stream) {
    if (!src || !dst || K <= 0 || N <= 0 || K % 128 != 0 || (((uintptr_t)src | (uintptr_t)dst) % 16) != 0)
        return set_error(kErrBadArg, "quantize_mmq_q8_1: need K %% 128 == 0 and a 16-byte aligned source");
    const long threads = (long)(K / 32) * N;
    hipLaunchKernelGGL(quantize_q8_1_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream,
                       src, (uint8_t *)dst, K, N);
    return check_launch("quantize_mmq_q8_1");
}

}  // namespace mnemo
