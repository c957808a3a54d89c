// sample.hip -- next-token selection from the lm_head logits (MnemoCUDA kernels.cu:2020-2174,
// wrapper kernels.cu:2208-2215), one workgroup of 1024 threads.
//
// Semantics kept from the reference (they decide which token is drawn for a given seed):
//  * temperature <= 0: argmax (this build breaks exact ties toward the lower index).
//  * temperature > 0: p_i = exp((z_i - max z) / T); the nucleus is drawn from 2048
//    candidates: for each residue class c = i mod 256, the 8 largest p of the class (equal
//    p: the lower index first, which is what the reference's in-order scan that only
//    replaces its minimum by a strictly larger value keeps).  Candidates are taken in
//    decreasing p until their running sum reaches top_p * total (total = sum of all p),
//    the kept ones are renormalised and one is drawn with u from xoroshiro128+ (s0 =
//    rng_state, s1 = rng_state ^ 0xDEADBEEFCAFEBABE, three warm-up steps, u = (s0 + s1) >> 11
//    as a float times 2^-53).
// What differs: the reference sums in one order on 256 threads and runs a selection sort and
// the running sums on one thread (up to 2048 x nucleus comparisons, then three sequential
// passes).  Here four threads share a class, the candidates are sorted by a bitonic network
// and the running sums are a parallel scan: fp32 sums in another order, which can change
// the drawn token only when the draw or top_p * total lies within rounding (~1e-6 of the
// mass) of a cumulative boundary; equal p are ordered by token id.
#include "mnemo_common.hpp"
#include "mnemo_internal.hpp"

namespace mnemo {

constexpr int kSampleThreads = 1024;
constexpr int kClasses = 256, kPerClass = 8, kSub = kSampleThreads / kClasses;  // 4 threads per class
constexpr int kCands = kClasses * kPerClass;                                    // 2048

__device__ __forceinline__ uint64_t xoro_next(uint64_t &s0, uint64_t &s1) {
    const uint64_t t = s0 ^ (s0 << 23);
    s0 = s1;
    s1 = t ^ s1 ^ (t >> 17) ^ (s1 >> 26);
    return s0 + s1;
}

__device__ __forceinline__ bool before(float pa, int ia, float pb, int ib) {
    return pa > pb || (pa == pb && ia < ib);
}

__global__ void __launch_bounds__(kSampleThreads) sample_token_kernel(const float *__restrict__ logits, int V,
                                                                      float temperature, float top_p,
                                                                      unsigned long long seed, int *__restrict__ out) {
    __shared__ float red_f[kSampleThreads];
    __shared__ int red_i[kSampleThreads];
    __shared__ float cp[kCands];
    __shared__ int ci[kCands];
    __shared__ float mp[kSampleThreads * kPerClass];  // every thread's list before the class merge
    __shared__ int mi[kSampleThreads * kPerClass];
    const int tid = threadIdx.x;

    float m = -1e30f;
    for (int i0 = tid; i0 < V; i0 += kSampleThreads * 8) {
        float zb[8];
#pragma unroll
        for (int u = 0; u < 8; u++) zb[u] = logits[min(i0 + u * kSampleThreads, V - 1)];  // clamped: a repeat
#pragma unroll
        for (int u = 0; u < 8; u++) m = fmaxf(m, zb[u]);
    }
    red_f[tid] = m;
    __syncthreads();
    for (int s = kSampleThreads / 2; s > 0; s >>= 1) {
        if (tid < s) red_f[tid] = fmaxf(red_f[tid], red_f[tid + s]);
        __syncthreads();
    }
    const float gmax = red_f[0];
    __syncthreads();

    if (temperature <= 0.0f) {  // argmax, ties to the lower index
        float bv = -1e30f;
        int bi = 0x7FFFFFFF;
        for (int i = tid; i < V; i += kSampleThreads) {
            const float v = logits[i];
            if (v > bv) { bv = v; bi = i; }
        }
        red_f[tid] = bv;
        red_i[tid] = bi;
        __syncthreads();
        for (int s = kSampleThreads / 2; s > 0; s >>= 1) {
            if (tid < s && before(red_f[tid + s], red_i[tid + s], red_f[tid], red_i[tid])) {
                red_f[tid] = red_f[tid + s];
                red_i[tid] = red_i[tid + s];
            }
            __syncthreads();
        }
        if (tid == 0) *out = red_i[0] == 0x7FFFFFFF ? 0 : red_i[0];
        return;
    }

    // thread (sub = tid / 256, class c = tid % 256) scans indices c + 256 * (sub + 4 t) in
    // increasing order (adjacent lanes read adjacent logits), keeping its 8 largest p (ties:
    // the earliest) and its sum
    const int c = tid % kClasses, sub = tid / kClasses;
    float sum = 0.0f;
    float hv[kPerClass];
    int hi[kPerClass];
#pragma unroll
    for (int k = 0; k < kPerClass; k++) {
        hv[k] = -1.0f;
        hi[k] = -1;
    }
    float hmin = -1.0f;  // the current minimum of hv
    // logits are loaded kBatch at a time (independent loads in flight), then scanned in order
    constexpr int kStride = kClasses * kSub, kBatch = 16;
    for (int i0 = c + kClasses * sub; i0 < V; i0 += kStride * kBatch) {
        float zb[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; u++) zb[u] = logits[min(i0 + u * kStride, V - 1)];
#pragma unroll
        for (int u = 0; u < kBatch; u++) {
        const int i = i0 + u * kStride;
        if (i >= V) break;
        const float p = expf((zb[u] - gmax) / temperature);
        sum += p;
        if (p > hmin) {
            int at = 0;  // first position holding the minimum
#pragma unroll
            for (int k = kPerClass - 1; k >= 0; k--) at = hv[k] == hmin ? k : at;
#pragma unroll
            for (int k = 0; k < kPerClass; k++)
                if (k == at) {
                    hv[k] = p;
                    hi[k] = i;
                }
            hmin = hv[0];
#pragma unroll
            for (int k = 1; k < kPerClass; k++) hmin = fminf(hmin, hv[k]);
        }
        }
    }
#pragma unroll
    for (int k = 0; k < kPerClass; k++) {
        mp[tid * kPerClass + k] = hv[k];
        mi[tid * kPerClass + k] = hi[k];
    }
    red_f[tid] = sum;
    __syncthreads();
    // merge the class's 4 lists (threads c, c + 256, c + 512, c + 768): the first 8 of 32 by
    // (p desc, index asc)
    if (sub == 0) {
        for (int k = 0; k < kPerClass; k++) {
            int best = -1;
            float bp = -2.0f;
            int bi = 0x7FFFFFFF;
            for (int j = 0; j < kSub * kPerClass; j++) {
                const int at = ((j / kPerClass) * kClasses + c) * kPerClass + j % kPerClass;
                const float pj = mp[at];
                const int ij = mi[at];
                if (ij >= 0 && before(pj, ij, bp, bi)) {
                    bp = pj;
                    bi = ij;
                    best = at;
                }
            }
            cp[c * kPerClass + k] = best >= 0 ? bp : -1.0f;
            ci[c * kPerClass + k] = best >= 0 ? bi : 0x7FFFFFFF;
            if (best >= 0) mi[best] = -1;
        }
    }
    for (int s = kSampleThreads / 2; s > 0; s >>= 1) {
        if (tid < s) red_f[tid] += red_f[tid + s];
        __syncthreads();
    }
    const float total = red_f[0];

    // bitonic sort of the candidates by (p desc, id asc)
    for (int k = 2; k <= kCands; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int t = tid; t < kCands / 2; t += kSampleThreads) {
                const int a = ((t & ~(j - 1)) << 1) | (t & (j - 1)), b = a + j;  // j is a power of two
                const bool up = (a & k) == 0;
                const float pa = cp[a], pb = cp[b];
                const int ia = ci[a], ib = ci[b];
                if (before(pa, ia, pb, ib) != up) {
                    cp[a] = pb;
                    cp[b] = pa;
                    ci[a] = ib;
                    ci[b] = ia;
                }
            }
            __syncthreads();
        }
    }
    // inclusive running sums of the positive p (Hillis-Steele, two elements per thread)
    float *cs = mp;
    for (int t = tid; t < kCands; t += kSampleThreads) cs[t] = fmaxf(cp[t], 0.0f);
    __syncthreads();
    for (int off = 1; off < kCands; off <<= 1) {
        float v[2];
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const int t = tid + q * kSampleThreads;
            v[q] = cs[t] + (t >= off ? cs[t - off] : 0.0f);
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < 2; q++) cs[tid + q * kSampleThreads] = v[q];
        __syncthreads();
    }
    // nucleus size n: 1 + the first position whose running sum reaches top_p * total, or
    // the number of positive candidates
    uint64_t s0 = seed, s1 = seed ^ 0xDEADBEEFCAFEBABEull;
    for (int w = 0; w < 3; w++) xoro_next(s0, s1);
    const float r = (float)(xoro_next(s0, s1) >> 11) * (1.0f / 9007199254740992.0f);
    const float mass = top_p * total;
    if (tid == 0) {
        red_i[0] = kCands;
        red_i[1] = 0x7FFFFFFF;
    }
    __syncthreads();
    for (int t = tid; t < kCands; t += kSampleThreads)
        if (cp[t] <= 0.0f || cs[t] >= mass) atomicMin(&red_i[0], cp[t] <= 0.0f ? t : t + 1);
    __syncthreads();
    const int n = red_i[0];
    const float target = r * (n > 0 ? cs[n - 1] : 0.0f);
    for (int t = tid; t < n; t += kSampleThreads)
        if (cs[t] >= target) atomicMin(&red_i[1], t);
    __syncthreads();
    if (tid == 0) {
        const int pick = red_i[1] == 0x7FFFFFFF ? 0 : red_i[1];
        const int id = ci[pick];
        *out = (id < 0 || id == 0x7FFFFFFF) ? 0 : id;
    }
}

int launch_sample_token(const float *logits, int V, float temperature, float top_p, unsigned long long seed,
                        int *out, hipStream_t stream) {
    if (!logits || !out || V <= 0) return set_error(kErrBadArg, "sample_token: bad arguments");
    hipLaunchKernelGGL(sample_token_kernel, dim3(1), dim3(kSampleThreads), 0, stream, logits, V, temperature, top_p,
                       seed, out);
    return check_launch("sample_token");
}

}  // namespace mnemo
