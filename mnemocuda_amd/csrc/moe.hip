// moe.hip -- grouped-expert prefill: route T tokens x k experts into expert-sorted rows,
// run every active expert's gate+up (SwiGLU fused) and down projections as grouped
// Q4_K/Q6_K x Q8_1 GEMMs, then scatter-add the router-weighted rows back per token.
//
// The reference has no batched MoE path: its prefill runs the decode chain token by
// token (src/forward.c:1783-1830), i.e. per token and selected expert
//   gate = W_g x, up = W_u x (Q4_K, src/forward.c:876-882)
//   act = silu(gate) * up (src/kernels.cu:1310-1313)
//   out += w_slot * W_d act (Q4_K or Q6_K down, src/forward.c:884-893)
// This file computes the same composition with the activations quantized to Q8_1 blocks
// (x once per token, act once per token-expert pair), the semantics the GEMMs implement;
// the quantized rows are staged directly in the GEMM's f16 operand form.
//
// Workspace layout (each part 256-byte aligned), sizes for T tokens, k slots, E experts:
//   xs      T staged rows of x (StagedAct: q8 [T][hidden] f16, rho and ds [T][hidden/32],
//           dlast [T])
//   counts  E ints, offsets E ints
//   rank    T*k ints   (rank of a pair within its expert; -1 for dropped slots)
//   inv     T*k ints   (pair -> expert-sorted row, -1 for dropped slots)
//   perm    T*k ints   (expert-sorted row -> token)
//   tiles   1 + E + ceil(T*k/kGroupTile) ints (count, then (expert << 16) | token tile)
//   act     T*k rows of eff fp32 (SwiGLU output)
//   acts    T*k staged rows of Q8_1(act) (StagedAct)
//   down    T*k rows of hidden fp32
#include <algorithm>
#include <cstring>
#include <mutex>

#include "mnemo_common.hpp"
#include "mnemo_internal.hpp"
#include "x_image.hpp"

namespace mnemo {

int launch_stage_f32(const float *x, int K, int N, StagedAct sa, hipStream_t s);
int launch_gemm_grouped(int type, int swiglu, const void *experts, size_t expert_stride, size_t w_off,
                        size_t w_off2, StagedAct act, const int *counts, const int *offsets, const int *perm,
                        const int *tiles, int max_tiles, float *out, int out_ld, int M, int K, hipStream_t stream);

int launch_matvec_f32(const float *w, const float *x, float *y, int n_rows, int n_cols, hipStream_t s);
int launch_topk_softmax(const float *scores, int *idx, float *wts, int n, int k, hipStream_t s);
int launch_router_topk(const float *w, const float *x, const float *nw, float eps, unsigned long long *slots, int n,
                       int n_cols, int k, unsigned long long *cnt, int *idx, float *wts, uint8_t *img,
                       float *img_scale, hipStream_t stream);

constexpr int kRouteThreads = 1024;
constexpr int kRouteWaves = kRouteThreads / 64;
constexpr int kMaxMoeExperts = 512;
constexpr int kMoeTileRows = kGroupTile;  // token rows per grouped GEMM tile

struct MoeLayout {
    size_t xs, xr, xds, xdl, counts, offsets, rank, inv, perm, tiles, act, acts, actr, actds, actdl, down, total;
    int max_tiles;
};

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

static MoeLayout moe_layout(int T, int hidden, int eff, int E, int k) {
    MoeLayout L{};
    const size_t pairs = (size_t)T * k;
    L.max_tiles = E + (int)((pairs + kMoeTileRows - 1) / kMoeTileRows);
    size_t o = 0;
    auto take = [&](size_t bytes) {
        size_t at = o;
        o = align256(o + bytes);
        return at;
    };
    L.xs = take((size_t)T * hidden * 2);
    L.xr = take((size_t)T * (hidden / 32) * 4);
    L.xds = take((size_t)T * (hidden / 32) * 2);
    L.xdl = take((size_t)T * 4);
    L.counts = take((size_t)E * 4);
    L.offsets = take((size_t)E * 4);
    L.rank = take(pairs * 4);
    L.inv = take(pairs * 4);
    L.perm = take(pairs * 4);
    L.tiles = take((size_t)(1 + L.max_tiles) * 4);
    L.act = take(pairs * eff * 4);
    L.acts = take(pairs * eff * 2);
    L.actr = take(pairs * (eff / 32) * 4);
    L.actds = take(pairs * (eff / 32) * 2);
    L.actdl = take(pairs * 4);
    L.down = take(pairs * hidden * 4);
    L.total = o;
    return L;
}

// Wave-wide "match any": mask of the lanes whose value equals this lane's (v < 2^bits).
__device__ inline uint64_t match_mask(int v, int bits) {
    uint64_t m = ~0ull;
    for (int b = 0; b < bits; b++) {
        const bool bit = (v >> b) & 1;
        const uint64_t bal = __ballot(bit);
        m &= bit ? bal : ~bal;
    }
    return m;
}

// One block of 1024 threads.  Pass 1: wave w walks its own contiguous range of the pairs
// (pair order = token major, slot minor) in steps of 64 and gives each pair its rank among
// the earlier pairs of the same expert in that range (a wave-wide match, a per-wave count
// per expert in LDS); the per-wave counts are then scanned across waves, so a pair's rank
// among all earlier pairs of its expert is its wave's prefix plus its rank in the range:
// the expert-sorted order is deterministic, token ascending within an expert.  Pass 2 scans
// the counts, places the pairs and writes the tile list.
__global__ void __launch_bounds__(kRouteThreads) moe_route_kernel(const int *__restrict__ topk_idx, int pairs, int E,
                                                                  int bits, int *__restrict__ counts,
                                                                  int *__restrict__ offsets, int *__restrict__ rank,
                                                                  int *__restrict__ inv, int *__restrict__ perm,
                                                                  int *__restrict__ tiles, int k) {
    __shared__ int running[kMaxMoeExperts];
    __shared__ int wave_cnt[kRouteWaves][kMaxMoeExperts];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < kRouteWaves * E; i += kRouteThreads) wave_cnt[i / E][i % E] = 0;
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const int per = ((pairs + kRouteWaves - 1) / kRouteWaves + 63) & ~63;  // pairs per wave range
    __syncthreads();
    {
        const int w0 = wave * per, w1 = min(w0 + per, pairs);
        for (int c = w0; c < w1; c += 64) {  // wave-uniform
            const int p = c + lane;
            int e = p < w1 ? topk_idx[p] : -1;
            if (e >= E) e = -1;  // out-of-range expert ids are dropped like empty slots
            const int key = e < 0 ? E : e;  // E = "dropped" bucket, matched like any value
            const uint64_t m = match_mask(key, bits);
            const int r_in = __popcll(m & lt);
            if (e >= 0) rank[p] = wave_cnt[wave][e] + r_in;
            else if (p < w1) rank[p] = -1;
            // the group's first lane adds the group; the next step's reads come after it
            // (one wave's LDS operations complete in order)
            if (e >= 0 && r_in == 0) wave_cnt[wave][e] += __popcll(m);
        }
    }
    __syncthreads();
    for (int ex = tid; ex < E; ex += kRouteThreads) {  // exclusive prefix over the waves
        int acc = 0;
        for (int w = 0; w < kRouteWaves; w++) {
            const int t = wave_cnt[w][ex];
            wave_cnt[w][ex] = acc;
            acc += t;
        }
        running[ex] = acc;
    }
    __syncthreads();
    // exclusive scans of the counts and of the tiles per expert: thread ex holds expert ex
    // (E <= 512), a wave-wide scan (DPP shuffles), then the wave totals in wave order
    __shared__ int wsum[2][kRouteWaves];
    __shared__ int s_off[kMaxMoeExperts];
    const int c = tid < E ? running[tid] : 0;
    const int nt = (c + kMoeTileRows - 1) / kMoeTileRows;
    int ic = c, it = nt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int a = __shfl_up(ic, o), b = __shfl_up(it, o);
        if (lane >= o) {
            ic += a;
            it += b;
        }
    }
    if (lane == 63) {
        wsum[0][wave] = ic;
        wsum[1][wave] = it;
    }
    __syncthreads();
    int bc = 0, bt = 0;
    for (int w = 0; w < wave; w++) {
        bc += wsum[0][w];
        bt += wsum[1][w];
    }
    if (tid < E) {
        const int oc = bc + ic - c, ot = bt + it - nt;
        counts[tid] = c;
        offsets[tid] = oc;
        s_off[tid] = oc;
        for (int j = 0; j < nt; j++) tiles[1 + ot + j] = (tid << 16) | j;  // expert order
        if (tid == E - 1) tiles[0] = ot + nt;
    }
    __syncthreads();
    // place the pairs (loads of four pairs per thread in flight at a time)
    for (int p0 = 0; p0 < pairs; p0 += 4 * kRouteThreads) {
        int r[4], e[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int p = min(p0 + tid + i * kRouteThreads, pairs - 1);
            r[i] = rank[p];
            e[i] = topk_idx[p];
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int p = p0 + tid + i * kRouteThreads;
            if (p >= pairs) break;
            if (r[i] < 0) {
                inv[p] = -1;
                continue;
            }
            const int rr = r[i] + wave_cnt[p / per][e[i]];
            rank[p] = rr;
            const int q = s_off[e[i]] + rr;
            inv[p] = q;
            perm[q] = p / k;
        }
    }
}

// out[t][i] += sum over slots (in slot order) of w[t][slot] * down[inv[t][slot]][i]
__global__ void __launch_bounds__(256) moe_combine_kernel(const float *__restrict__ down, const int *__restrict__ inv,
                                                          const float *__restrict__ topk_w, float *__restrict__ out,
                                                          int T, int hidden, int k) {
    const long n4 = (long)T * hidden / 4;
    const int h4 = hidden / 4;
    for (long v = (long)blockIdx.x * blockDim.x + threadIdx.x; v < n4; v += (long)gridDim.x * blockDim.x) {
        const int t = (int)(v / h4), i4 = (int)(v % h4);
        float4 acc = ((float4 *)out)[v];
        for (int s = 0; s < k; s++) {
            const int q = inv[t * k + s];
            if (q < 0) continue;
            const float w = topk_w[t * k + s];
            const float4 d = ((const float4 *)(down + (size_t)q * hidden))[i4];
            acc.x += w * d.x;
            acc.y += w * d.y;
            acc.z += w * d.z;
            acc.w += w * d.w;
        }
        ((float4 *)out)[v] = acc;
    }
}

size_t moe_prefill_workspace_bytes(int T, int hidden, int eff, int E, int k) {
    if (T <= 0 || hidden <= 0 || eff <= 0 || E <= 0 || k <= 0) return 0;
    return moe_layout(T, hidden, eff, E, k).total;
}

int launch_moe_prefill(const void *experts, size_t expert_stride, size_t gate_off, size_t up_off, size_t down_off,
                       int down_type, const float *x, const int *topk_idx, const float *topk_w, int T, int hidden,
                       int eff, int E, int k, void *ws, size_t ws_bytes, float *out, hipStream_t s) {
    if (!experts || !x || !topk_idx || !topk_w || !ws || !out || T <= 0 || k <= 0 || k > 64 || E <= 0)
        return set_error(kErrBadArg, "moe_prefill: null pointer or non-positive size");
    if (E > kMaxMoeExperts) return set_error(kErrBadArg, "moe_prefill: at most %d experts", kMaxMoeExperts);
    if (hidden % 256 != 0 || eff % 256 != 0)
        return set_error(kErrBadArg, "moe_prefill: hidden and eff must be multiples of 256");
    // a tile-list entry is (expert << 16) | tile: an expert's tiles must stay below 65536
    if ((long)T * k > 65536L * kMoeTileRows)
        return set_error(kErrBadArg, "moe_prefill: more than %ld token-expert pairs", 65536L * kMoeTileRows);
    if (down_type != kTypeQ4K && down_type != kTypeQ6K)
        return set_error(kErrUnsupportedType, "moe_prefill: unsupported down type %d", down_type);
    if ((((uintptr_t)ws | (uintptr_t)x | (uintptr_t)out) & 15) != 0)
        return set_error(kErrBadArg, "moe_prefill: workspace, x and out must be 16-byte aligned");
    // the grouped kernels copy weight blocks into LDS with 16-byte DMA from 4-byte aligned
    // addresses (Q6_K rows start 2 bytes past one when the row length is odd in blocks, which
    // the copies absorb)
    if ((((uintptr_t)experts | expert_stride | gate_off | up_off | down_off) & 3) != 0)
        return set_error(kErrBadArg, "moe_prefill: the expert table, its stride and offsets must be 4-byte aligned");
    const MoeLayout L = moe_layout(T, hidden, eff, E, k);
    if (ws_bytes < L.total)
        return set_error(kErrBadArg, "moe_prefill: workspace of %zu bytes, need %zu", ws_bytes, L.total);
    uint8_t *w8 = (uint8_t *)ws;
    int *counts = (int *)(w8 + L.counts), *offsets = (int *)(w8 + L.offsets);
    int *rank = (int *)(w8 + L.rank), *inv = (int *)(w8 + L.inv), *perm = (int *)(w8 + L.perm);
    int *tiles = (int *)(w8 + L.tiles);
    float *act = (float *)(w8 + L.act), *down = (float *)(w8 + L.down);
    const int pairs = T * k;
    int bits = 1;
    while ((1 << bits) <= E) bits++;

    const StagedAct xs{(_Float16 *)(w8 + L.xs), (float *)(w8 + L.xr), (uint16_t *)(w8 + L.xds),
                       (float *)(w8 + L.xdl)};
    const StagedAct acts{(_Float16 *)(w8 + L.acts), (float *)(w8 + L.actr), (uint16_t *)(w8 + L.actds),
                         (float *)(w8 + L.actdl)};
    int rc = launch_stage_f32(x, hidden, T, xs, s);
    if (rc) return rc;
    hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(kRouteThreads), 0, s, topk_idx, pairs, E, bits, counts,
                       offsets, rank, inv, perm, tiles, k);
    if ((rc = check_launch("moe_route"))) return rc;
    // gate + up, SwiGLU fused: act[q][f]
    rc = launch_gemm_grouped(kTypeQ4K, 1, experts, expert_stride, gate_off, up_off, xs, counts, offsets, perm,
                             tiles + 1, L.max_tiles, act, eff, eff, hidden, s);
    if (rc) return rc;
    if ((rc = launch_stage_f32(act, eff, pairs, acts, s))) return rc;
    rc = launch_gemm_grouped(down_type, 0, experts, expert_stride, down_off, down_off, acts, counts, offsets,
                             nullptr, tiles + 1, L.max_tiles, down, hidden, hidden, eff, s);
    if (rc) return rc;
    const long n4 = (long)T * hidden / 4;
    hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)std::min<long>((n4 + 255) / 256, 8192)), dim3(256), 0, s,
                       down, inv, topk_w, out, T, hidden, k);
    return check_launch("moe_combine");
}

// ------------------------------------------------------------------ decode (one token)
// The reference's decode MoE block (src/forward.c:814-1077): router matvec, top-k, then per
// selected expert a host round trip to find its weights, gate+up, SwiGLU, down, scaled add.
// Here the expert ids never leave the device: the two expert GEMVs read them from the
// workspace (expert mode of the GEMV kernel), so the block is three stream-ordered
// launches (router + top-k, gate + up, down + combine) with no synchronisation,
// graph-capturable.
//
// Workspace: router arrival counter (64 bits) | tagged logit slots [E] (64 bits each) |
// idx[k] | w[k] | gate/up rows [k][2][eff] | tagged partial slots [k][hidden] (64 bits
// each, used when the down launch combines through partials) | tile counters [hidden] |
// the router's image of the normed x with 1 / rms (x_image.hpp), each 256-byte aligned.  The counter sits at offset 0 whatever the sizes, so a workspace
// shared by calls of different shapes never finds other data there.  Zero the workspace
// once when allocating it; calls keep the counter and slots valid from then on.
struct MoeDecodeLayout {
    size_t rcnt, logits, idx, w, gu, partial, cnt, img, total;
};

static MoeDecodeLayout moe_decode_layout(int hidden, int eff, int E, int k) {
    MoeDecodeLayout L{};
    size_t o = 0;
    auto take = [&](size_t bytes) {
        size_t at = o;
        o = align256(o + bytes);
        return at;
    };
    L.rcnt = take(8);
    L.logits = take((size_t)E * 8);
    L.idx = take((size_t)k * 4);
    L.w = take((size_t)k * 4);
    L.gu = take((size_t)k * 2 * eff * 4);
    L.partial = take((size_t)k * hidden * 8);
    L.cnt = take((size_t)hidden * 4);
    L.img = take(xlds_bytes((hidden + 255) & ~255) + 16);  // the image, then 1 / rms
    L.total = o;
    return L;
}

size_t moe_decode_workspace_bytes(int hidden, int eff, int E, int k) {
    if (hidden <= 0 || eff <= 0 || E <= 0 || k <= 0) return 0;
    return moe_decode_layout(hidden, eff, E, k).total;
}

int launch_moe_decode(const float *router_w, const void *experts, size_t expert_stride, size_t gate_off,
                      size_t up_off, size_t down_off, int down_type, const float *x, const float *norm_w, float eps,
                      int hidden, int eff, int E, int k, void *ws, size_t ws_bytes, float *out, int *idx_out,
                      float *w_out, hipStream_t s) {
    if (!router_w || !experts || !x || !ws || !out || hidden <= 0 || eff <= 0 || E <= 0 || k <= 0)
        return set_error(kErrBadArg, "moe_decode: null pointer or non-positive size");
    if (k > 16 || k > E || E > 1024) return set_error(kErrBadArg, "moe_decode: need k <= 16, k <= n_experts <= 1024");
    if (down_type != kTypeQ4K && down_type != kTypeQ6K)
        return set_error(kErrUnsupportedType, "moe_decode: unsupported down type %d", down_type);
    if ((((uintptr_t)ws) & 15) != 0) return set_error(kErrBadArg, "moe_decode: workspace must be 16-byte aligned");
    const MoeDecodeLayout L = moe_decode_layout(hidden, eff, E, k);
    if (ws_bytes < L.total)
        return set_error(kErrBadArg, "moe_decode: workspace of %zu bytes, need %zu", ws_bytes, L.total);
    uint8_t *w8 = (uint8_t *)ws;
    // the routing goes to the caller's arrays when given (the engine logs expert use),
    // else to the workspace
    unsigned long long *slots = (unsigned long long *)(w8 + L.logits);
    float *wts = w_out ? w_out : (float *)(w8 + L.w);
    int *idx = idx_out ? idx_out : (int *)(w8 + L.idx);
    float *gu = (float *)(w8 + L.gu);
    unsigned long long *partial = (unsigned long long *)(w8 + L.partial);
    int *cnt = (int *)(w8 + L.cnt);

    // with norm_w, x is the raw hidden state and both the router and the gate/up launch apply
    // the RMS norm themselves (the reference's separate rms_norm launch, forward.c:800-806)
    // with the norm, router workgroup 0 also writes the image of x * g and 1 / rms, which the
    // staged gate/up launch copies instead of building its own (one build instead of one per
    // workgroup, and no x or norm-weight loads in front of its weight loads)
    const size_t img_bytes = xlds_bytes((hidden + 255) & ~255);
    uint8_t *img = norm_w ? w8 + L.img : nullptr;
    float *img_scale = norm_w ? (float *)(w8 + L.img + img_bytes) : nullptr;
    int rc = launch_router_topk(router_w, x, norm_w, eps, slots, E, hidden, k,
                                (unsigned long long *)(w8 + L.rcnt), idx, wts, img, img_scale, s);
    if (rc) return rc;

    GemvArgs a;
    memset(&a, 0, sizeof a);
    a.x = x;
    a.x2 = norm_w;
    a.ximg = img;
    a.xscale = img_scale;
    a.eps = eps;
    a.n_cols = hidden;
    a.ex.table = (const uint8_t *)experts;
    a.ex.stride = expert_stride;
    a.ex.off[0] = gate_off;
    a.ex.off[1] = up_off;
    a.ex.idx = idx;
    a.ex.wt = wts;
    a.ex.y = gu;
    a.ex.tile_cnt = cnt;
    a.ex.ntiles = hidden;
    a.ex.slots = k;
    a.ex.nm = 2;
    a.ex.rows = eff;
    // gate and up rows in one pass give silu(gate) * up directly (rows of up to 4096 values)
    const int act = ((hidden + 255) & ~255) <= 4096;
    a.ex.act = act;
    a.ex.type = kTypeQ4K;  // gate/up are Q4_K in Q4_K_M experts (src/forward.c:866-872)
    a.ex.n_experts = E;
    if ((rc = launch_gemv_experts(a, s))) return rc;

    memset(&a, 0, sizeof a);
    a.n_cols = eff;
    a.ex.table = (const uint8_t *)experts;
    a.ex.stride = expert_stride;
    a.ex.off[0] = down_off;
    a.ex.idx = idx;
    a.ex.wt = wts;
    a.ex.xs = gu;
    a.ex.part = partial;
    a.ex.gen = (const unsigned long long *)(w8 + L.rcnt);
    a.ex.out = out;
    a.ex.tile_cnt = cnt;
    a.ex.slots = k;
    a.ex.nm = 1;
    a.ex.act = act;
    a.ex.rows = hidden;
    a.ex.type = down_type;
    a.ex.n_experts = E;
    if ((rc = launch_gemv_experts(a, s))) return rc;
    return kOk;
}

// ------------------------------------------------------------------ decode without allocation
// The decode MoE block for callers that cannot allocate or pass a workspace (code under
// graph capture, serving loops): the workspace is the file-scope device array below, one
// copy per GPU, held until the process ends.  Every call on a GPU uses that GPU's copy, so
// calls that overlap on one GPU (other streams, other threads) race.  The array is zeroed
// when a GPU's copy is first set up; from then on every call keeps the router's counter
// (at offset 0 for every shape) and logit slots valid, and the gate/up launch clears the
// tile counters itself.  Sizes: moe_decode_layout(hidden, eff, n_experts, k) must fit kDecodeScratchBytes
// (hidden 8192, eff 4096, 1024 experts, k 16 fit).
constexpr size_t kDecodeScratchBytes = (size_t)1664 * 1024;
static __device__ __align__(256) uint8_t scratch[kDecodeScratchBytes];

constexpr int kMaxScratchDevices = 64;
static void *g_scratch_ptr[kMaxScratchDevices];
static std::mutex g_scratch_mu;

__global__ void zero_words_kernel(uint32_t *__restrict__ p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

// The device address of this GPU's scratch (hipGetSymbolAddress: the array's name is a
// host-side stand-in that kernels cannot use).  `s`: the stream that zeroes a first-time
// copy with a fill kernel (stream-ordered and capture-safe), or null to zero it
// synchronously (set-up from cuda_kernels_init, outside any capture).
static int decode_scratch(hipStream_t s, bool sync, void **out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices)
        return set_error(kErrLaunch, "moe_decode scratch: no usable HIP device");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return set_error(kErrLaunch, "moe_decode scratch: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
        const int words = (int)(kDecodeScratchBytes / 4);
        if (sync) {
            if (hipMemset(p, 0, kDecodeScratchBytes) != hipSuccess || hipDeviceSynchronize() != hipSuccess)
                return set_error(kErrLaunch, "moe_decode scratch: zeroing failed");
        } else {
            // a first call under graph capture would record the zeroing into the graph (run
            // again on every replay): set-up belongs to cuda_kernels_init
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
                (void)hipGetLastError();
                return set_error(kErrBadArg,
                                 "moe_decode scratch: first use on this GPU under graph capture; call "
                                 "cuda_kernels_init first");
            }
            hipLaunchKernelGGL(zero_words_kernel, dim3(256), dim3(256), 0, s, (uint32_t *)p, words);
            if (int rc = check_launch("moe_decode scratch zero")) return rc;
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return kOk;
}

int moe_decode_scratch_init() {
    void *p;
    return decode_scratch(nullptr, true, &p);
}

int launch_moe_decode_noalloc(const float *router_w, const void *experts, size_t expert_stride, size_t gate_off,
                              size_t up_off, size_t down_off, int down_type, const float *x, const float *norm_w,
                              float eps, int hidden, int eff, int E, int k, float *out, int *idx_out, float *w_out,
                              hipStream_t s) {
    if (hidden <= 0 || eff <= 0 || E <= 0 || k <= 0)
        return set_error(kErrBadArg, "moe_decode_rmsnorm_noalloc: non-positive size");
    const size_t need = moe_decode_layout(hidden, eff, E, k).total;
    if (need > kDecodeScratchBytes)
        return set_error(kErrBadArg,
                         "moe_decode_rmsnorm_noalloc: hidden %d, eff %d, %d experts, k %d need %zu bytes of scratch, "
                         "the library holds %zu",
                         hidden, eff, E, k, need, kDecodeScratchBytes);
    void *ws = nullptr;
    if (int rc = decode_scratch(s, false, &ws)) return rc;
    return launch_moe_decode(router_w, experts, expert_stride, gate_off, up_off, down_off, down_type, x, norm_w, eps,
                             hidden, eff, E, k, ws, kDecodeScratchBytes, out, idx_out, w_out, s);
}

}  // namespace mnemo
