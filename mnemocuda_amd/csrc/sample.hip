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

// ------------------------------------------------------------------ top-p selection
// The 2048 candidates are sorted by (p desc, id asc) on 256 threads, 8 per thread: thread t
// holds sorted positions 8t .. 8t+7 in registers.  A candidate's order is that of one 64-bit
// key, {p bits, ~id} (p >= 0 orders like its bits); an empty slot (p < 0, NaN) is key 0 and
// sorts last.  Bitonic network: strides below 8 inside a thread, 8 .. 256 between the lanes
// of a wave (DPP up to 64, permutes at 128 and 256), 512 and 1024 through LDS.  Then the running sums (inclusive, in
// sorted order: sequential within a thread, a scan over the threads), the nucleus and the
// draw.
constexpr int kSelThreads = kCands / 8;  // 256
constexpr int kSelWaves = kSelThreads / 64;

__device__ __forceinline__ uint64_t cand_key(float p, int id) {
    if (!(p >= 0.0f)) return 0ull;
    return ((uint64_t)__float_as_uint(fabsf(p)) << 32) | (uint32_t)~(uint32_t)id;
}

// keep the better (larger key) of a and b in a when `better_here`, the other one otherwise
__device__ __forceinline__ uint64_t keep(uint64_t a, uint64_t b, bool better_here) {
    return (a > b) == better_here ? a : b;  // one compare, one select (keys are distinct or equal)
}

// v of lane ^ M: DPP within rows of 16 lanes (quad permutes; row rotations, where lane i
// reads lane (i - n) mod 16), a cross-lane permute beyond
template <int M>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
    if constexpr (M == 1) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppXor1, 0xF, 0xF, false);
    else if constexpr (M == 2) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppXor2, 0xF, 0xF, false);
    else if constexpr (M == 4) {
        const uint32_t dn = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x124, 0xF, 0xF, false);  // i - 4
        const uint32_t up = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x12C, 0xF, 0xF, false);  // i + 4
        return (lane_id() & 4) ? dn : up;
    } else if constexpr (M == 8) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false);
    else return (uint32_t)__shfl_xor((int)v, M);
}

// a bitonic pass between lanes t and t ^ M (strides 8M): every key's partner first, then
// the choices (one wait for the exchanged values, not one per key)
template <int M>
__device__ __forceinline__ void lane_pass(uint64_t (&k)[8], bool better_here) {
    uint64_t o[8];
#pragma unroll
    for (int r = 0; r < 8; r++)
        o[r] = ((uint64_t)xor_lane<M>((uint32_t)(k[r] >> 32)) << 32) | xor_lane<M>((uint32_t)k[r]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < 8; r++) k[r] = keep(k[r], o[r], better_here);
}

// a bitonic pass of stride J < 8: pairs inside the thread's 8 keys (sorted positions 8t + r)
template <int J>
__device__ __forceinline__ void reg_pass(uint64_t (&k)[8], int t, int kk) {
#pragma unroll
    for (int r = 0; r < 8; r++) {
        if (r & J) continue;
        const bool up = ((8 * t + r) & kk) == 0;
        const uint64_t a = k[r], b = k[r | J];
        k[r] = keep(a, b, up);
        k[r | J] = keep(a, b, !up);
    }
}

struct SelLds {
    uint64_t xch[kCands];
    float wsum[kSelWaves];
    int wmin[2][kSelWaves];
    float cs_last;
};

// Every thread of the NT-thread workgroup calls this (it holds barriers); threads
// t < kSelThreads hold candidates 8t .. 8t+7 in k (any order).  total = the sum of all p.
template <int NT>
__device__ void select_sorted(uint64_t (&k)[8], float total, float top_p, unsigned long long seed, SelLds &L,
                              int *__restrict__ out) {
    static_assert(NT % 64 == 0 && NT >= kSelThreads, "the selection needs 256 threads");
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const bool act = t < kSelThreads;
    // bitonic sort, best first: at level kk the pair (e, e ^ j), e < e ^ j, puts the better
    // key at e when (e & kk) == 0
    for (int kk = 2; kk <= kCands; kk <<= 1) {
        for (int j = kk >> 1; j >= 8; j >>= 1) {
            const int m = j >> 3;  // partner thread t ^ m
            const bool up = ((8 * t) & kk) == 0, lower = (t & m) == 0;
            if (j < 512) {  // partner in the same wave (m is uniform)
                const bool b = up == lower;
                switch (m) {
                case 1: lane_pass<1>(k, b); break;
                case 2: lane_pass<2>(k, b); break;
                case 4: lane_pass<4>(k, b); break;
                case 8: lane_pass<8>(k, b); break;
                case 16: lane_pass<16>(k, b); break;
                default: lane_pass<32>(k, b); break;
                }
            } else {
                if (act)
#pragma unroll
                    for (int r = 0; r < 8; r++) L.xch[8 * t + r] = k[r];
                __syncthreads();
                if (act)
#pragma unroll
                    for (int r = 0; r < 8; r++) k[r] = keep(k[r], L.xch[8 * (t ^ m) + r], up == lower);
                __syncthreads();
            }
        }
        // strides 4, 2, 1 inside the thread
        if (kk > 4) reg_pass<4>(k, t, kk);
        if (kk > 2) reg_pass<2>(k, t, kk);
        reg_pass<1>(k, t, kk);
    }
    // inclusive running sums of the positive p in sorted order
    float p[8], c[8];
#pragma unroll
    for (int r = 0; r < 8; r++) p[r] = act ? __uint_as_float((uint32_t)(k[r] >> 32)) : 0.0f;
    c[0] = p[0];
#pragma unroll
    for (int r = 1; r < 8; r++) c[r] = c[r - 1] + p[r];
    float s = c[7];  // inclusive scan of the thread totals over the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float v = __shfl_up(s, o);
        if (lane >= o) s += v;
    }
    float excl = __shfl_up(s, 1);
    if (lane == 0) excl = 0.0f;
    if (act && lane == 63) L.wsum[w] = s;
    __syncthreads();
    float off = 0.0f;
    for (int i = 0; i < w && i < kSelWaves; i++) off += L.wsum[i];
    const float pre = off + excl;
#pragma unroll
    for (int r = 0; r < 8; r++) c[r] = pre + c[r];
    // nucleus size n: 1 + the first position whose running sum reaches top_p * total, the
    // position of the first candidate with p <= 0, or all of them
    const float mass = top_p * total;
    int nc = kCands;
#pragma unroll
    for (int r = 7; r >= 0; r--)
        if (act && (p[r] <= 0.0f || c[r] >= mass)) nc = p[r] <= 0.0f ? 8 * t + r : 8 * t + r + 1;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) nc = min(nc, __shfl_xor(nc, o));
    if (act && lane == 0) L.wmin[0][w] = nc;
    __syncthreads();
    int n = kCands;
    for (int i = 0; i < kSelWaves; i++) n = min(n, L.wmin[0][i]);
    if (act && n > 0 && t == (n - 1) >> 3) {
        float v = c[0];
#pragma unroll
        for (int r = 1; r < 8; r++) v = r == ((n - 1) & 7) ? c[r] : v;
        L.cs_last = v;
    }
    __syncthreads();
    uint64_t s0 = seed, s1 = seed ^ 0xDEADBEEFCAFEBABEull;
    for (int i = 0; i < 3; i++) xoro_next(s0, s1);
    const float u = (float)(xoro_next(s0, s1) >> 11) * (1.0f / 9007199254740992.0f);
    const float target = u * (n > 0 ? L.cs_last : 0.0f);
    // the draw: the first position below n whose running sum reaches the target
    int pk = 0x7FFFFFFF;
#pragma unroll
    for (int r = 7; r >= 0; r--)
        if (act && 8 * t + r < n && c[r] >= target) pk = 8 * t + r;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) pk = min(pk, __shfl_xor(pk, o));
    if (act && lane == 0) L.wmin[1][w] = pk;
    __syncthreads();
    int pick = 0x7FFFFFFF;
    for (int i = 0; i < kSelWaves; i++) pick = min(pick, L.wmin[1][i]);
    if (pick == 0x7FFFFFFF) pick = 0;
    if (act && t == pick >> 3) {
        uint64_t kv = k[0];
#pragma unroll
        for (int r = 1; r < 8; r++) kv = r == (pick & 7) ? k[r] : kv;
        const int id = kv ? (int)~(uint32_t)kv : -1;
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

    __shared__ SelLds sel;
    uint64_t key[8];
#pragma unroll
    for (int r = 0; r < 8; r++) key[r] = tid < kSelThreads ? cand_key(cp[8 * tid + r], ci[8 * tid + r]) : 0ull;
    select_sorted<kSampleThreads>(key, total, top_p, seed, sel, out);
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

__global__ void __launch_bounds__(kSelThreads) sample_finish_kernel(const SampleWs *__restrict__ ws,
                                                                    float temperature, float top_p,
                                                                    unsigned long long seed, int *__restrict__ out) {
    __shared__ SelLds sel;
    __shared__ float wv[kSelWaves];
    __shared__ int wi[kSelWaves];
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
        static_assert(kClasses == kSelThreads, "thread c holds class c's first winner");
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
            wv[tid >> 6] = bv;
            wi[tid >> 6] = bi;
        }
        __syncthreads();
        if (tid == 0) {
            bv = wv[0];
            bi = wi[0];
            for (int w = 1; w < kSelWaves; w++)
                if (wv[w] > bv || (wv[w] == bv && wi[w] < bi)) {
                    bv = wv[w];
                    bi = wi[w];
                }
            *out = bi == 0x7FFFFFFF ? 0 : bi;
        }
        return;
    }
    // thread t: class t's 8 winners, p as the one-launch form computes it
    uint64_t key[8];
#pragma unroll
    for (int r = 0; r < 8; r++) {
        const int id = ws->id[8 * tid + r];
        key[r] = cand_key(id == 0x7FFFFFFF ? -1.0f : expf((ws->z[8 * tid + r] - M) / temperature), id);
    }
    select_sorted<kSelThreads>(key, tot, top_p, seed, sel, out);
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
    hipLaunchKernelGGL(sample_finish_kernel, dim3(1), dim3(kSelThreads), 0, stream, w, temperature, top_p, seed, out);
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
