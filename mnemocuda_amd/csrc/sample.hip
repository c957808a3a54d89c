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

// Top-p draw from the 2048 candidates (cp[] = p, ci[] = token id; p < 0 marks an empty slot)
// with total = the sum of all p: bitonic sort by (p desc, id asc), running sums, nucleus,
// draw.  All kSampleThreads threads call this; cs (2048 floats) and red (2 ints) are LDS
// scratch.
__device__ void select_candidates(float *cp, int *ci, float *cs, int *red_i, float total, float top_p,
                                  unsigned long long seed, int *__restrict__ out) {
    const int tid = threadIdx.x;
    __syncthreads();
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

    select_candidates(cp, ci, mp, red_i, total, top_p, seed, out);
}

// ------------------------------------------------------------------ workspace form
// The same selection over two launches that spread the scan of the vocabulary:
//  1. sample_classes_kernel, 64 workgroups: workgroup w takes the residue classes 4w .. 4w+3
//     (i mod 256) over the whole vocabulary, each class on 64 threads; it writes its 32
//     class winners -- the 8 largest logits of each class, equal logits by the lower index
//     (the order of p = exp((z - max) / T), which is increasing in z) -- with their ids, its
//     largest logit m_w and S_w = sum exp((z - m_w) / T) over its classes;
//  2. sample_finish_kernel, one workgroup: M = max m_w, total = sum_w S_w exp((m_w - M) / T),
//     p of the 2048 winners from their logits as the one-launch form computes them, then the
//     same sort, nucleus and draw (temperature <= 0: the first winner in (z desc, id asc)
//     order, the argmax).
// Differences to the one-launch form: the total is summed per class group first (fp32 sums
// in another order); a class's 8th and 9th largest p can only be exchanged when their
// logits differ but round to the same p.
constexpr int kClsGroups = 64;                 // workgroups of the first launch
constexpr int kClsPerGroup = kClasses / kClsGroups;  // 4
constexpr int kClsThreads = 256;               // 64 threads per class
constexpr int kClsPerThread = 16;              // logits per thread: vocab <= 16 * 64 * 256 = 262144
struct SampleWs {
    float m[kClsGroups], s[kClsGroups];
    float z[kCands];
    int id[kCands];
};

size_t sample_workspace_bytes() { return sizeof(SampleWs); }

__global__ void __launch_bounds__(kClsThreads) sample_classes_kernel(const float *__restrict__ logits, int V,
                                                                     float temperature, SampleWs *__restrict__ ws) {
    __shared__ float lz[kClsThreads * kPerClass];
    __shared__ int li[kClsThreads * kPerClass];
    __shared__ float red[kClsThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int cl = tid & (kClsPerGroup - 1);                   // class within the group
    const int c = (int)blockIdx.x * kClsPerGroup + cl, j0 = tid / kClsPerGroup;  // 64 threads per class
    float z[kClsPerThread];
    float m = -INFINITY;
#pragma unroll
    for (int u = 0; u < kClsPerThread; u++) {
        const int i = c + kClasses * (j0 + 64 * u);
        z[u] = i < V ? logits[i] : -INFINITY;
        m = fmaxf(m, z[u]);
    }
    // the group's largest logit
    m = wave_max_all(m);
    if (lane == 0) red[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // this thread's 8 largest (z desc, index asc: its indices increase with u) and its sum
    float hv[kPerClass];
    int hi[kPerClass];
#pragma unroll
    for (int k = 0; k < kPerClass; k++) {
        hv[k] = -INFINITY;
        hi[k] = 0x7FFFFFFF;
    }
    float sum = 0.0f;
#pragma unroll
    for (int u = 0; u < kClsPerThread; u++) {
        const int i = c + kClasses * (j0 + 64 * u);
        if (i < V) {
            sum += expf((z[u] - m) / temperature);
            // insert (z[u], i) keeping hv sorted descending; a later equal z goes after
            float v = z[u];
            int id = i;
#pragma unroll
            for (int k = 0; k < kPerClass; k++) {
                const bool take = v > hv[k];
                const float tv = hv[k];
                const int ti = hi[k];
                hv[k] = take ? v : hv[k];
                hi[k] = take ? id : hi[k];
                v = take ? tv : v;
                id = take ? ti : id;
            }
        }
    }
#pragma unroll
    for (int k = 0; k < kPerClass; k++) {
        lz[tid * kPerClass + k] = hv[k];
        li[tid * kPerClass + k] = hi[k];
    }
    sum = sum64_lane63(sum);
    __syncthreads();
    if (lane == 63) red[tid >> 6] = sum;
    __syncthreads();
    if (tid == 0) {
        ws->m[blockIdx.x] = m;
        ws->s[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
    }
    // wave w merges class w's 64 lists (512 entries, 8 per lane) by 8 rounds of wave argmax
    const int w = tid >> 6;
    const int cw = (int)blockIdx.x * kClsPerGroup + w;
    float bz[kPerClass];
    int bi[kPerClass];
#pragma unroll
    for (int k = 0; k < kPerClass; k++) {
        const int t = kClsPerGroup * lane + w;  // thread of class w in slot `lane`
        bz[k] = lz[t * kPerClass + k];
        bi[k] = li[t * kPerClass + k];
    }
    int head = 0;  // the lane's list is sorted: its best remaining entry is bz[head]
    for (int r = 0; r < kPerClass; r++) {
        float v = -INFINITY;
        int id = 0x7FFFFFFF;
#pragma unroll
        for (int k = 0; k < kPerClass; k++)
            if (k == head) {
                v = bz[k];
                id = bi[k];
            }
        float bv = v;
        int bid = id;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o);
            const int oi = __shfl_xor(bid, o);
            if (ov > bv || (ov == bv && oi < bid)) {
                bv = ov;
                bid = oi;
            }
        }
        if (id == bid && v == bv && bid != 0x7FFFFFFF) head++;  // the owner drops its head
        if (lane == 0) {
            ws->z[cw * kPerClass + r] = bv;
            ws->id[cw * kPerClass + r] = bid;
        }
    }
}

__global__ void __launch_bounds__(kSampleThreads) sample_finish_kernel(const SampleWs *__restrict__ ws,
                                                                       float temperature, float top_p,
                                                                       unsigned long long seed, int *__restrict__ out) {
    __shared__ float cp[kCands];
    __shared__ int ci[kCands];
    __shared__ float cs[kCands];
    __shared__ int red_i[2];
    __shared__ float tot;
    __shared__ float Ms;
    const int tid = threadIdx.x;
    if (tid < 64) {
        // one group per lane: the common max and the rescaled total as wave reductions
        // (one round trip to the workspace, a fixed summation order)
        static_assert(kClsGroups == 64, "one class group per lane");
        const float mg = ws->m[tid], sg = ws->s[tid];
        const float M = wave_max_all(mg);
        const float t = wave_sum_all(mg > -INFINITY ? sg * expf((mg - M) / temperature) : 0.0f);
        if (tid == 0) {
            Ms = M;
            tot = t;
        }
    }
    __syncthreads();
    const float M = Ms;
    if (temperature <= 0.0f) {  // argmax: the best class winner (ties to the lower id)
        if (tid < kClasses) {  // thread c holds class c's first winner
            float bv = ws->z[tid * kPerClass];
            int bi = ws->id[tid * kPerClass];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const float ov = __shfl_xor(bv, o);
                const int oi = __shfl_xor(bi, o);
                if (ov > bv || (ov == bv && oi < bi)) {
                    bv = ov;
                    bi = oi;
                }
            }
            if ((tid & 63) == 0) {
                cp[tid >> 6] = bv;
                ci[tid >> 6] = bi;
            }
        }
        __syncthreads();
        if (tid == 0) {
            float bv = cp[0];
            int bi = ci[0];
            for (int w = 1; w < kClasses / 64; w++)
                if (cp[w] > bv || (cp[w] == bv && ci[w] < bi)) {
                    bv = cp[w];
                    bi = ci[w];
                }
            *out = bi == 0x7FFFFFFF ? 0 : bi;
        }
        return;
    }
    for (int t = tid; t < kCands; t += kSampleThreads) {
        const int id = ws->id[t];
        cp[t] = id == 0x7FFFFFFF ? -1.0f : expf((ws->z[t] - M) / temperature);
        ci[t] = id;
    }
    __syncthreads();
    select_candidates(cp, ci, cs, red_i, tot, top_p, seed, out);
}

int launch_sample_token_ws(const float *logits, int V, float temperature, float top_p, unsigned long long seed,
                           void *ws, size_t ws_bytes, int *out, hipStream_t stream) {
    if (!logits || !out || !ws || V <= 0) return set_error(kErrBadArg, "sample_token_ws: bad arguments");
    if (V > kClasses * 64 * kClsPerThread)
        return set_error(kErrBadArg, "sample_token_ws: vocabulary above %d", kClasses * 64 * kClsPerThread);
    if (ws_bytes < sizeof(SampleWs) || ((uintptr_t)ws & 15))
        return set_error(kErrBadArg, "sample_token_ws: workspace of %zu bytes (need %zu, 16-byte aligned)", ws_bytes,
                         sizeof(SampleWs));
    SampleWs *w = (SampleWs *)ws;
    hipLaunchKernelGGL(sample_classes_kernel, dim3(kClsGroups), dim3(kClsThreads), 0, stream, logits, V,
                       temperature > 0.0f ? temperature : 1.0f, w);
    hipLaunchKernelGGL(sample_finish_kernel, dim3(1), dim3(kSampleThreads), 0, stream, w, temperature, top_p, seed,
                       out);
    return check_launch("sample_token_ws");
}

int launch_sample_token(const float *logits, int V, float temperature, float top_p, unsigned long long seed,
                        int *out, hipStream_t stream) {
    if (!logits || !out || V <= 0) return set_error(kErrBadArg, "sample_token: bad arguments");
    hipLaunchKernelGGL(sample_token_kernel, dim3(1), dim3(kSampleThreads), 0, stream, logits, V, temperature, top_p,
                       seed, out);
    return check_launch("sample_token");
}

}  // namespace mnemo
