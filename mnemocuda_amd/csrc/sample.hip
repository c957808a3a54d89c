// sample.hip -- next-token selection from the lm_head logits (MnemoCUDA kernels.cu:2020-2174,
// wrapper kernels.cu:2208-2215), one workgroup of 256 threads.
//
// Semantics kept from the reference (they decide which token is drawn for a given seed):
//  * temperature <= 0: argmax (this build breaks exact ties toward the lower index).
//  * temperature > 0: p_i = exp((z_i - max z) / T); the nucleus is drawn from 2048
//    candidates: for each residue class c = i mod 256, the 8 largest p of the class,
//    kept by a scan in index order that replaces its current minimum only by a strictly
//    larger value; total = sum of all p, summed per class in index order and then over
//    the classes by the pairwise halving tree 128, 64, .., 1.  Candidates are taken in
//    decreasing p until their running sum reaches top_p * total, the kept ones are
//    renormalised and one is drawn with u from xoroshiro128+ (seed s0 = rng_state,
//    s1 = rng_state ^ 0xDEADBEEFCAFEBABE, three warm-up steps, u = (s0 + s1) >> 11 as a
//    float times 2^-53).
// What differs: the reference orders the candidates by a selection sort on one thread
// (up to 2048 x nucleus comparisons); here a bitonic sort by (p desc, candidate slot asc)
// does it in parallel.  For distinct p the order is the same; equal p may be taken in a
// different order.
#include "mnemo_common.hpp"
#include "mnemo_internal.hpp"

namespace mnemo {

constexpr int kSampleThreads = 256;  // = the number of candidate classes
constexpr int kPerClass = 8;
constexpr int kCands = kSampleThreads * kPerClass;

__device__ __forceinline__ uint64_t xoro_next(uint64_t &s0, uint64_t &s1) {
    const uint64_t t = s0 ^ (s0 << 23);
    s0 = s1;
    s1 = t ^ s1 ^ (t >> 17) ^ (s1 >> 26);
    return s0 + s1;
}

__global__ void __launch_bounds__(kSampleThreads) sample_token_kernel(const float *__restrict__ logits, int V,
                                                                      float temperature, float top_p,
                                                                      unsigned long long seed, int *__restrict__ out) {
    __shared__ float red_f[kSampleThreads];
    __shared__ int red_i[kSampleThreads];
    __shared__ float cp[kCands];
    __shared__ int ci[kCands];
    const int tid = threadIdx.x;

    float m = -1e30f;
    for (int i = tid; i < V; i += kSampleThreads) m = fmaxf(m, logits[i]);
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
            if (v > bv) { bv = v; bi = i; }  // first maximum of this class
        }
        red_f[tid] = bv;
        red_i[tid] = bi;
        __syncthreads();
        for (int s = kSampleThreads / 2; s > 0; s >>= 1) {
            if (tid < s) {
                const float ov = red_f[tid + s];
                const int oi = red_i[tid + s];
                if (ov > red_f[tid] || (ov == red_f[tid] && oi < red_i[tid])) {
                    red_f[tid] = ov;
                    red_i[tid] = oi;
                }
            }
            __syncthreads();
        }
        if (tid == 0) *out = red_i[0] == 0x7FFFFFFF ? 0 : red_i[0];
        return;
    }

    // per class: the sum of p in index order and the 8 largest p
    float sum = 0.0f;
    float hv[kPerClass];
    int hi[kPerClass];
#pragma unroll
    for (int k = 0; k < kPerClass; k++) {
        hv[k] = -1.0f;
        hi[k] = -1;
    }
    for (int i = tid; i < V; i += kSampleThreads) {
        const float p = expf((logits[i] - gmax) / temperature);
        sum += p;
        int mi = 0;
#pragma unroll
        for (int k = 1; k < kPerClass; k++) mi = hv[k] < hv[mi] ? k : mi;
        float mv = hv[0];
#pragma unroll
        for (int k = 1; k < kPerClass; k++) mv = k == mi ? hv[k] : mv;
        if (p > mv) {
#pragma unroll
            for (int k = 0; k < kPerClass; k++)
                if (k == mi) {
                    hv[k] = p;
                    hi[k] = i;
                }
        }
    }
    red_f[tid] = sum;
#pragma unroll
    for (int k = 0; k < kPerClass; k++) {
        cp[tid * kPerClass + k] = hv[k];
        ci[tid * kPerClass + k] = tid * kPerClass + k;  // slot: class * 8 + heap position
    }
    __syncthreads();
    for (int s = kSampleThreads / 2; s > 0; s >>= 1) {
        if (tid < s) red_f[tid] += red_f[tid + s];
        __syncthreads();
    }
    const float total = red_f[0];

    // bitonic sort of (p, slot) by p desc, slot asc
    for (int k = 2; k <= kCands; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int t = tid; t < kCands / 2; t += kSampleThreads) {
                const int a = ((t / j) * 2 * j) + (t % j), b = a + j;
                const bool up = (a & k) == 0;  // this run sorts "first before second"
                const float pa = cp[a], pb = cp[b];
                const int sa = ci[a], sb = ci[b];
                const bool a_first = pa > pb || (pa == pb && sa < sb);
                if (a_first != up) {
                    cp[a] = pb;
                    cp[b] = pa;
                    ci[a] = sb;
                    ci[b] = sa;
                }
            }
            __syncthreads();
        }
    }
    if (tid == 0) {
        uint64_t s0 = seed, s1 = seed ^ 0xDEADBEEFCAFEBABEull;
        for (int w = 0; w < 3; w++) xoro_next(s0, s1);
        const float r = (float)(xoro_next(s0, s1) >> 11) * (1.0f / 9007199254740992.0f);
        const float mass = top_p * total;
        float cumul = 0.0f;
        int n = 0;
        for (int i = 0; i < kCands; i++) {
            const float p = cp[i];
            if (p <= 0.0f) break;
            cumul += p;
            n = i + 1;
            if (cumul >= mass) break;
        }
        float nsum = 0.0f;
        for (int i = 0; i < n; i++) nsum += cp[i];
        const float target = r * nsum;
        float acc = 0.0f;
        int pick = 0;
        for (int i = 0; i < n; i++) {
            acc += cp[i];
            if (acc >= target) {
                pick = i;
                break;
            }
        }
        red_i[0] = ci[pick];  // candidate slot = class * 8 + heap position
    }
    __syncthreads();
    const int slot = red_i[0];  // the class's thread still holds the token ids
    if (tid == slot / kPerClass) {
        int id = 0;
#pragma unroll
        for (int k = 0; k < kPerClass; k++) id = k == slot % kPerClass ? hi[k] : id;
        *out = id < 0 ? 0 : id;
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
