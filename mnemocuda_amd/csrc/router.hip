// router.hip -- fp32 router matvec, top-k softmax, expert glue and the Q8_1 quantizer.
//
//  * matvec_f32      (MnemoCUDA kernels.cu:859-880): one workgroup per router row, all
//                    16-byte loads issued up front, fp32 FMA, fixed-order reduction.
//  * topk_softmax    (kernels.cu:993-1057): one wave; k rounds of a wave-wide arg-max
//                    ordered by (value desc, index asc), then softmax over the winners.
//                    Winners are written in that order (the reference's order is its
//                    slot order, so only the (index, weight) pairs are comparable).
//  * swiglu / scaled_add (kernels.cu:677-688, 980-988): elementwise, float4.
//  * quantize_q8_1   (gemm_q4k.cu:327-358): one thread per 32 values, same operation
//                    order as the reference so the bytes match exactly.
#include "mnemo_common.hpp"
#include "mnemo_internal.hpp"
#include "x_image.hpp"

namespace mnemo {

// One workgroup of kRowThreads per row: every thread's loads of W and x are issued before
// any arithmetic (a loop over float4s with an FMA chain would wait for each load in turn;
// one wave per row took 8.7 us for the 128 x 4096 router).
constexpr int kRowThreads = 1024;
constexpr int kRowMaxV4 = 4;  // float4 per thread: n_cols <= 16384 on the vector path

template <int T = kRowThreads, int V4 = kRowMaxV4>
__device__ __forceinline__ float row_dot(const float *__restrict__ wr, const float *__restrict__ x, int n_cols,
                                         bool vec4) {
    typedef float fv4 __attribute__((ext_vector_type(4)));
    const int tid = threadIdx.x;
    float acc = 0.0f;
    if (vec4) {
        const fv4 *w4 = (const fv4 *)wr;
        const fv4 *x4 = (const fv4 *)x;
        const int n4 = n_cols / 4;
        fv4 a[V4], b[V4];
#pragma unroll
        for (int i = 0; i < V4; i++) {
            const int c = min(tid + i * T, n4 - 1);  // clamped: branch-free loads
            a[i] = __builtin_nontemporal_load(w4 + c);
            b[i] = x4[c];
        }
#pragma unroll
        for (int i = 0; i < V4; i++) {
            float t = fmaf(a[i].x, b[i].x, acc);
            t = fmaf(a[i].y, b[i].y, t);
            t = fmaf(a[i].z, b[i].z, t);
            t = fmaf(a[i].w, b[i].w, t);
            acc = tid + i * T < n4 ? t : acc;
        }
    } else {
        for (int c = tid; c < n_cols; c += T) acc = fmaf(wr[c], x[c], acc);
    }
    return acc;
}

// Workgroup sum in a fixed order (wave sums, then wave 0, 1, ..): deterministic.
template <int T = kRowThreads>
__device__ __forceinline__ float block_sum(float v, float *part) {
    v = sum64_lane63(v);
    if (lane_id() == 63) part[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.0f;
    if (threadIdx.x == 0)
        for (int i = 0; i < T / 64; i++) s += part[i];
    return s;
}

__global__ void __launch_bounds__(kRowThreads) matvec_f32_kernel(const float *__restrict__ w,
                                                                 const float *__restrict__ x,
                                                                 float *__restrict__ y, int n_cols, int vec4) {
    __shared__ float part[kRowThreads / 64];
    const int row = blockIdx.x;
    const float s = block_sum(row_dot(w + (size_t)row * n_cols, x, n_cols, vec4), part);
    if (threadIdx.x == 0) y[row] = s;
}

int launch_matvec_f32(const float *w, const float *x, float *y, int n_rows, int n_cols,
                      hipStream_t stream) {
    if (!w || !x || !y || n_rows <= 0 || n_cols <= 0) return set_error(kErrBadArg, "matvec_f32: bad arguments");
    const int vec4 = (n_cols % 4 == 0) && (n_cols <= 4 * kRowMaxV4 * kRowThreads) &&
                     (((uintptr_t)w | (uintptr_t)x) % 16 == 0);
    hipLaunchKernelGGL(matvec_f32_kernel, dim3(n_rows), dim3(kRowThreads), 0, stream, w, x, y, n_cols, vec4);
    return check_launch("matvec_f32");
}

// ---------------------------------------------------------------- top-k softmax
constexpr int kTopkMaxPerLane = 16;  // n_experts <= 1024
constexpr int kTopkMaxK = 16;        // the reference's register budget (kernels.cu:1002)


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

// ---------------------------------------------------------------- router + top-k, one launch
// The decode MoE block's router (kernels.cu:859-880) and top-k softmax (kernels.cu:993-1057)
// in one launch: workgroup r computes logit r; the last workgroup to count in (an arrival
// counter) selects the top k by rank -- logit i's rank is the number of logits ordered
// before it by (value desc, index asc), so the k winners come out sorted and ties go to the
// lower index, as topk_wave orders them -- and writes the softmax over the winners.
// Logits <= -1e30 and NaN never win.
//
// Arrival without fences (an agent-scope release/acquire pair writes back and invalidates
// the XCDs' L2s, ~2.5 us a launch): the counter is 64 bits, the launch number in the high
// half and the arrivals of this launch in the low half.  Each workgroup counts in with a
// relaxed fetch-add as it starts, which hands it the launch number g, and stores its logit
// as one 64-bit atomic slot {g + 1, logit bits} when it has it.  The workgroup that sees
// n - 1 earlier arrivals ranks the logits: it moves the counter on to {g + 1, 0} (every
// workgroup of the launch has counted in, and the next launch on the stream starts after
// this one ends) and reads each slot until it carries the tag g + 1.  Every workgroup that
// counted in is running and stores its slot, so the wait ends, without any ordering
// between the two locations.  A zero-filled
// counter and slots are a valid start (tag 0 never matches g + 1 before 2^32 launches).
// With nw, x is first RMS-normalised (x * rsqrt(mean(x^2) + eps) * nw, the reference's
// rms_norm_kernel, kernels.cu:692-722) inside every workgroup: each holds all of x.
template <int T, int V4>
__device__ __forceinline__ float row_dot_norm(const float *__restrict__ wr, const float *__restrict__ x,
                                              const float *__restrict__ nw, int n_cols, float eps, float *part,
                                              float *img_scale) {
    typedef float fv4 __attribute__((ext_vector_type(4)));
    const int tid = threadIdx.x;
    const fv4 *w4 = (const fv4 *)wr, *x4 = (const fv4 *)x, *n4w = (const fv4 *)nw;
    const int n4 = n_cols / 4;
    fv4 a[V4], b[V4], c[V4];
#pragma unroll
    for (int i = 0; i < V4; i++) {
        const int j = min(tid + i * T, n4 - 1);
        a[i] = __builtin_nontemporal_load(w4 + j);
        b[i] = x4[j];
        c[i] = n4w[j];
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < V4; i++)
        if (tid + i * T < n4) ss += b[i].x * b[i].x + b[i].y * b[i].y + b[i].z * b[i].z + b[i].w * b[i].w;
    ss = sum64_lane63(ss);
    if (lane_id() == 63) part[tid >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < T / 64; i++) tot += part[i];
    __syncthreads();  // part[] is reused by block_sum
    const float scale = __builtin_amdgcn_rsqf(tot / (float)n_cols + eps);  // rsqrtf, as the reference (kernels.cu:718)
    if (img_scale && blockIdx.x == 0 && tid == 0) *img_scale = scale;
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < V4; i++) {
        float t = fmaf(a[i].x, b[i].x * scale * c[i].x, acc);
        t = fmaf(a[i].y, b[i].y * scale * c[i].y, t);
        t = fmaf(a[i].z, b[i].z * scale * c[i].z, t);
        t = fmaf(a[i].w, b[i].w * scale * c[i].w, t);
        acc = tid + i * T < n4 ? t : acc;
    }
    return acc;
}

// upper bound on one slot's wait (s_sleep rounds of ~64 cycles): the slot stores were all
// issued before the last arrival, so a wait ends in well under a microsecond; the bound only
// guarantees that no wave spins for ever
constexpr int kRouterSlotWait = 1 << 22;

// One workgroup of kRouterThreads per row (fewer waves than kRowThreads: the row's loads are
// as many, and the barriers before the logit is ready shorter).
constexpr int kRouterThreads = 512;

template <int T, int V4>
__global__ void __launch_bounds__(T) router_topk_kernel(const float *__restrict__ w, const float *__restrict__ x,
                                                        const float *__restrict__ nw, float eps,
                                                        unsigned long long *__restrict__ slots, int n, int n_cols,
                                                        int k, unsigned long long *__restrict__ cnt,
                                                        int *__restrict__ idx, float *__restrict__ wts, int vec4,
                                                        uint8_t *img, float *img_scale) {
    __shared__ float part[T / 64];
    __shared__ unsigned int is_last, tag, stale;
    __shared__ float z[64 * kTopkMaxPerLane];
    // rank keys: {order-preserving bits of the logit, ~index} -- a larger key is a better
    // logit, equal logits the lower index (as `better`); 0 for a logit that never wins
    __shared__ __align__(16) unsigned long long zk[64 * kTopkMaxPerLane];
    static_assert((64 * kTopkMaxPerLane) % 16 == 0, "whole 16-key blocks");
    __shared__ float sel_v[kTopkMaxK];
    __shared__ int sel_i[kTopkMaxK];
    const int tid = threadIdx.x;
    const int row = blockIdx.x;
    // count in before the row's dot product, so that the atomic's round trip overlaps the
    // row's loads
    unsigned long long old = 0;
    if (tid == 0) stale = 0;  // ordered before its uses by the barrier after the count-in
    if (tid == 0) old = __hip_atomic_fetch_add(cnt, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const float v = block_sum<T>(nw ? row_dot_norm<T, V4>(w + (size_t)row * n_cols, x, nw, n_cols, eps, part, img_scale)
                                    : row_dot<T, V4>(w + (size_t)row * n_cols, x, n_cols, vec4),
                                 part);
    if (tid == 0) {
        const unsigned int g1 = (unsigned int)(old >> 32) + 1u;
        __hip_atomic_store(slots + row, ((unsigned long long)g1 << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        is_last = (unsigned int)old == (unsigned int)(n - 1);
        tag = g1;
        if (is_last)  // {g, n - 1} + 1 + (2^32 - n) = {g + 1, 0}
            __hip_atomic_fetch_add(cnt, (1ull << 32) - (unsigned long long)n, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
    if (img && nw && row == 0) {
        // after its logit is out: the image of x * g for the gate/up launch that follows, and
        // (in row_dot_norm) 1 / rms, which multiplies that launch's finished sums; the same
        // float4 per thread as row_dot_norm's, reloaded from the caches
        XRegs<V4> R, R2;
        const int n4 = n_cols / 4;
#pragma unroll
        for (int i = 0; i < V4; i++) {
            const int j = min(tid + i * T, n4 - 1);
            R.v[i] = ((const float4 *)x)[j];
            R2.v[i] = ((const float4 *)nw)[j];
        }
        const int kp = (n_cols + 255) & ~255;
        build_x<V4, 2, T>(R, R2, n_cols, kp, XLds(img, kp), tid);
    }
    __syncthreads();
    if (!is_last) return;
    const unsigned int g1 = tag;
    const int n16 = (n + 15) & ~15;
    for (int i = tid; i < n16; i += T) {
        unsigned long long key = 0;
        if (i < n) {
            unsigned long long sv = __hip_atomic_load(slots + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            for (int t = 0; (unsigned int)(sv >> 32) != g1 && t < kRouterSlotWait; t++) {
                __builtin_amdgcn_s_sleep(1);
                sv = __hip_atomic_load(slots + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            // a slot that never carried this call's tag (a broken ordering, never seen) marks
            // the whole ranking stale: the weights come out NaN, so the error shows downstream
            if ((unsigned int)(sv >> 32) != g1) stale = 1;
            const float l = __uint_as_float((unsigned int)sv);
            const bool ok = l > -1e30f;  // NaN and <= -1e30 never win
            z[i] = ok ? l : -1e30f;
            const uint32_t bits = __float_as_uint(l + 0.0f);  // -0 as +0: they compare equal
            const uint32_t ord = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
            key = ok ? ((unsigned long long)ord << 32) | (uint32_t)~(uint32_t)i : 0ull;
        }
        zk[i] = key;
    }
    if (tid < k) sel_i[tid] = -1;
    __syncthreads();
    // G threads per candidate (a power of two <= 64) count the keys above its own, each over
    // its share of the blocks of 16 keys; the counts meet in G-lane sums
    int G = 1;
    while (G < 64 && G * 2 * n <= T && 16 * G < n) G *= 2;
    const int sub = tid & (G - 1);
    for (int i = tid / G; i < n; i += T / G) {
        const unsigned long long ki = zk[i];
        int rank = 0;
        for (int j0 = 16 * sub; j0 < n; j0 += 16 * G) {
            unsigned long long kb[16];
#pragma unroll
            for (int q = 0; q < 8; q++) *(ulonglong2 *)&kb[2 * q] = *(const ulonglong2 *)&zk[j0 + 2 * q];
#pragma unroll
            for (int u = 0; u < 16; u++) rank += kb[u] > ki;
        }
        // the group's partial counts: DPP within 8 lanes (quad exchanges, then the half-row
        // mirror pairs the two quads), lane permutes beyond
        if (G >= 2) rank += __builtin_amdgcn_update_dpp(0, rank, kDppXor1, 0xF, 0xF, false);
        if (G >= 4) rank += __builtin_amdgcn_update_dpp(0, rank, kDppXor2, 0xF, 0xF, false);
        if (G >= 8) rank += __builtin_amdgcn_update_dpp(0, rank, kDppRowHalfMirror, 0xF, 0xF, false);
        for (int o = 8; o < G; o <<= 1) rank += __shfl_xor(rank, o);
        if (sub == 0 && ki != 0 && rank < k) {
            sel_v[rank] = z[i];
            sel_i[rank] = i;
        }
    }
    __syncthreads();
    if (tid < 64) {
        // softmax over the winners: lane r takes winner r; the sum runs in rank order, as a
        // sequential loop over the winners forms it
        static_assert(kTopkMaxK <= 64, "one winner per lane");
        const int r = tid;
        const float mx = sel_v[0];
        const float e = r < k && sel_i[r] >= 0 ? expf(sel_v[r] - mx) : 0.0f;
        float sum = 0.0f;
        for (int q = 0; q < k; q++)
            sum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e), q));
        if (r < k) {
            idx[r] = sel_i[r];
            wts[r] = stale ? __builtin_nanf("") : (sum > 0.0f ? e / sum : 0.0f);
        }
    }
}

int launch_router_topk(const float *w, const float *x, const float *nw, float eps, unsigned long long *slots, int n,
                       int n_cols, int k, unsigned long long *cnt, int *idx, float *wts, uint8_t *img,
                       float *img_scale, hipStream_t stream) {
    constexpr int T = kRouterThreads, kMaxV4 = 8;
    if (!w || !x || !slots || !cnt || !idx || !wts || n <= 0 || n_cols <= 0 || k <= 0 || k > kTopkMaxK ||
        k > n || n > 64 * kTopkMaxPerLane)
        return set_error(kErrBadArg, "router_topk: need 0 < k <= min(%d, n_experts), n_experts <= %d", kTopkMaxK,
                         64 * kTopkMaxPerLane);
    const int vec4 = (n_cols % 4 == 0) && (n_cols <= 4 * kMaxV4 * T) &&
                     (((uintptr_t)w | (uintptr_t)x | (uintptr_t)nw) % 16 == 0);
    if (nw && !vec4)
        return set_error(kErrBadArg, "router_topk: the fused RMS norm needs n_cols %% 4 == 0, <= %d and aligned vectors",
                         4 * kMaxV4 * T);
    // float4s per thread: the fewest that cover the row
    if (n_cols <= 4 * 2 * T)
        hipLaunchKernelGGL((router_topk_kernel<T, 2>), dim3(n), dim3(T), 0, stream, w, x, nw, eps, slots, n, n_cols, k,
                           cnt, idx, wts, vec4, img, img_scale);
    else if (n_cols <= 4 * 4 * T)
        hipLaunchKernelGGL((router_topk_kernel<T, 4>), dim3(n), dim3(T), 0, stream, w, x, nw, eps, slots, n, n_cols, k,
                           cnt, idx, wts, vec4, img, img_scale);
    else
        hipLaunchKernelGGL((router_topk_kernel<T, kMaxV4>), dim3(n), dim3(T), 0, stream, w, x, nw, eps, slots, n,
                           n_cols, k, cnt, idx, wts, vec4, img, img_scale);
    return check_launch("router_topk");
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
