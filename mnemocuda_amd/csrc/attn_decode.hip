// attn_decode.hip -- decode attention for grouped-query heads on the matrix cores.
//
// Same result as the reference's attention_kernel_f16kv / _int8kv (MnemoCUDA
// kernels.cu:1550-1660, 1382-1481): out[h] = softmax_p(scale * q_h . k_p) v_p over the
// positions 0..*pos_dev of the cache [pos][n_kv_heads][head_dim].  The reference runs one
// block per query head, so each KV head is streamed gqa times and one block walks the
// whole sequence.  Here:
//  * one workgroup per (KV head, 64-position chunk): the gqa (<= 16) query heads that share
//    the KV head are the 16 rows of v_mfma_f32_16x16x32_f16, so K and V are read once per
//    chunk, and the chunks of a long sequence spread over the whole chip; the workgroup's
//    waves split the chunk by position tiles (S) and by dims (O);
//  * S = Q K^T: K fragments come straight from the cache (8 consecutive dims per lane);
//    Q is split into f16 hi + lo parts (two MFMAs) so the product keeps ~fp32 precision;
//  * softmax over the chunk in registers (16-lane row reductions), P split hi + lo;
//  * O = P V: V goes through LDS so that each lane can gather 8 consecutive positions of
//    one dim (the MFMA's K direction);
//  * each chunk writes (max, sum, O) to the workspace; a second launch merges the chunks
//    per query head (the flash-decoding combine).  Past 4 K positions (8 K with V rows) each
//    workgroup walks several chunks and merges them itself, so the partials stay at 64 or
//    128 per KV head.
// int8 caches: K and V bytes convert exactly to f16; the per-position K scale multiplies
// the score column, the V scale is folded into P.
#include <math.h>

#include <mutex>

#include "mnemo_common.hpp"
#include "mnemo_internal.hpp"

namespace mnemo {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kChunk = 64;       // positions per wave

constexpr int kHd = 128;         // head_dim of this kernel
constexpr int kRows = 16;        // query heads per KV head handled (MFMA rows)
constexpr int kPart = 2 * kRows + kRows * kHd;  // floats per (KV head, chunk) partial

size_t attn_decode_workspace_bytes(int n_kv_heads, int max_ctx) {
    const size_t chunks = ((size_t)max_ctx + kChunk - 1) / kChunk;
    return (size_t)n_kv_heads * chunks * kPart * sizeof(float);
}

// V cache layouts.  kVRows: the reference's [pos][n_kv][hd].  kVBlocked: blocks of 64
// positions, [pos / 64][n_kv][hd][pos % 64], so that 8 consecutive positions of one dim
// (an MFMA fragment of O = P V) are 16 contiguous bytes.
constexpr int kVRows = 0;
constexpr int kVBlocked = 1;

size_t kv_blocked_offset(int pos, int kvh, int d, int nkv, int hd) {
    return (((size_t)(pos / 64) * nkv + kvh) * hd + d) * 64 + pos % 64;
}

// The new token's preparation, the arithmetic of head_pass_kernel for one head of 128 in a
// wave (lane holds dims lane and lane + 64): RMS norm with w (when given), then RoPE.
__device__ __forceinline__ void prep_head(float &x0, float &x1, bool norm, float w0, float w1, float eps, float cs,
                                          float sn) {
    if (norm) {
        const float ss = fmaf(x0, x0, fmaf(x1, x1, 0.0f));
        const float scale = __builtin_amdgcn_rsqf(wave_sum_all(ss) / (float)kHd + eps);  // as head_pass_kernel
        x0 = x0 * scale * w0;
        x1 = x1 * scale * w1;
    }
    const float v0 = x0, v1 = x1;
    x0 = fmaf(v0, cs, -(v1 * sn));  // the same fmas as head_pass_kernel
    x1 = fmaf(v0, sn, v1 * cs);
}

// One head row of the new position into the cache (K rows, V rows or V blocked) and into
// an LDS copy in the cache's element type; returns the int8 scale (1 for f16).
template <int KV>
__device__ __forceinline__ float store_new_row(float x0, float x1, void *cache, float *scales, size_t base,
                                               size_t es, size_t si, uint8_t *lds) {
    const int lane = lane_id();
    // x0, x1 are rounded to fp32 first (as a float row is, then converted): without the
    // barrier the compiler folds the RoPE fma and the f16 conversion into one rounding
    asm volatile("" : "+v"(x0), "+v"(x1));
    if (KV == kKvF16) {
        const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
        _Float16 *c = (_Float16 *)cache + base;
        c[(size_t)lane * es] = h0;
        c[(size_t)(lane + kHd / 2) * es] = h1;
        ((_Float16 *)lds)[lane] = h0;
        ((_Float16 *)lds)[lane + kHd / 2] = h1;
        return 1.0f;
    } else {
        const float m = wave_max_all(fmaxf(fabsf(x0), fabsf(x1)));
        const float inv = m > 0.0f ? 127.0f / m : 0.0f;
        const int8_t q0 = (int8_t)fminf(fmaxf(rintf(x0 * inv), -127.0f), 127.0f);
        const int8_t q1 = (int8_t)fminf(fmaxf(rintf(x1 * inv), -127.0f), 127.0f);
        int8_t *c = (int8_t *)cache + base;
        c[(size_t)lane * es] = q0;
        c[(size_t)(lane + kHd / 2) * es] = q1;
        ((int8_t *)lds)[lane] = q0;
        ((int8_t *)lds)[lane + kHd / 2] = q1;
        const float sc = m > 0.0f ? m / 127.0f : 0.0f;
        if (lane == 0) scales[si] = sc;
        return sc;
    }
}

// PREP: the launch also prepares the new token (QK norm, RoPE, K/V store at *pos_dev) --
// the same values head_pass_kernel would have written, formed in registers: every chunk
// prepares its query heads itself, the chunk holding *pos_dev stores the new K / V rows
// and uses them in place of what it loaded from the cache.
//
// A chunk's workgroup has 8 waves.  All of them prepare 2 of the 16 query heads (the
// per-head norm and RoPE are serial wave work).  Waves 0-3 then own one 16-position tile
// each: its K fragments, its column of S = Q K^T and its share of the softmax; waves 4-7
// own 32 of the 128 dims each: their V fragments and their columns of O = P V.  The waves
// meet through LDS: the Q rows, the tiles' row maxima and sums, P.
constexpr int kChunkWaves = 8;
constexpr int kChunkThreads = 64 * kChunkWaves;
constexpr int kPrepHeads = kRows / kChunkWaves;
constexpr int kTiles = kChunk / 16;  // position tiles = S waves
static_assert(kChunkWaves == 2 * kTiles && kHd == 32 * (kChunkWaves - kTiles) && kRows % kChunkWaves == 0,
              "4 S waves (16 positions each), 4 O waves (32 dims each), whole query heads per wave");
// Long sequences: past 64 chunks (4 K positions; 128 with V rows) a workgroup walks the chunks g,
// g + S, g + 2S, ... of its KV head and merges them as it goes (running max, sum and O, the
// flash-decoding update), so the launch leaves S partials per KV head instead of one per
// chunk; the next chunk's K (S waves) and V (O waves) loads are issued as soon as the current
// chunk's registers are free.  S = 64 up to 192 chunks, then 128 (one layer of 4 KV heads,
// MI355X: 8 K positions 10.3 against 10.5 us, 16 K 13.5 against 15.1, 32 K 18.8 against 24.3;
// S = 256 past 384 chunks was slower, 21.6 us at 32 K).  Shorter sequences take one chunk per
// workgroup, with none of the loop's code.
constexpr int kLoopChunks = 64;
// looping: 0 never (the entry-point kernel's partials), 1 blocked V, 2 V rows (from 128 chunks
// on, S = 128: 14.6 against 15.1 us at 16 K, 21.0 against 24.0 at 32 K, but 11.0 against 10.2
// at 8 K with S = 64)
__host__ __device__ __forceinline__ int chunk_stride(int nc, int looping) {
    if (looping == 0 || nc <= (looping == 1 ? kLoopChunks : 2 * kLoopChunks)) return nc;
    return looping == 1 && nc <= 192 ? 64 : 128;
}

template <int KV, int VL, bool PREP>
struct ChunkLds {
    _Float16 qs[2][kRows][kHd + 8];  // Q hi / lo, rows padded by 16 B
    _Float16 vt[VL == kVRows ? kChunk : 1][kHd + 8];  // V tile [pos][dim]
    _Float16 ps[2][kRows][kChunk + 8];
    uint8_t knew[PREP ? 2 : 1][PREP ? 2 * kHd : 1];  // new K, V rows as stored
    float tmax[kTiles][kRows], tsum[kTiles][kRows];
    float new_sc[2];  // int8 scales of the new K / V rows
};

// LOOP: the workgroup walks chunks g, g + stride, ... (else chunk g alone, the code of
// one chunk with nothing of the loop left in it)
template <int KV, int VL, bool PREP, bool LOOP>
__device__ __forceinline__ void chunk_body(const AttnDecodeArgs &a, ChunkLds<KV, VL, PREP> &L, int pos, int seq,
                                           int nc, int stride) {
    auto &qs = L.qs;
    auto &vt = L.vt;
    auto &ps = L.ps;
    auto &knew = L.knew;
    auto &tmax = L.tmax;
    auto &tsum = L.tsum;
    auto &new_sc = L.new_sc;
    const int g = blockIdx.y, kvh = blockIdx.x, lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int G = a.gqa;
    const size_t stride_kv = (size_t)a.nkv * kHd;
    const int r = lane & 15, kg = lane >> 4;
    const int pchunk = pos / kChunk;
    // this workgroup walks the chunk holding pos: it stores the new K / V rows
    const bool mine_wg = PREP && pos < a.max_ctx && pchunk % stride == g;  // uniform
    const bool swave = wave < kTiles;        // S wave: position tile t
    const int t = wave & (kTiles - 1);
    const int nv = wave - kTiles;            // O wave: dims 32 nv .. 32 nv + 31 (n-tiles 2nv, 2nv+1)
    constexpr int EB = KV == kKvF16 ? 2 : 1;  // bytes per cache element

    // ---- PREP: the new token's raw rows, loaded before the cache so that waiting for them
    // does not wait for the cache
    float qx0[PREP ? kPrepHeads : 1], qx1[PREP ? kPrepHeads : 1];
    float k0 = 0.0f, k1 = 0.0f, v0 = 0.0f, v1 = 0.0f, qw0 = 1.0f, qw1 = 1.0f, kw0 = 1.0f, kw1 = 1.0f, fr = 0.0f;
    const bool norm = PREP && a.qw != nullptr;  // uniform
    if (PREP) {
#pragma unroll
        for (int h = 0; h < kPrepHeads; h++) {
            const float *qh = a.q + (size_t)(kvh * G + min(kPrepHeads * wave + h, G - 1)) * kHd;
            qx0[h] = qh[lane];
            qx1[h] = qh[lane + kHd / 2];
        }
        if (norm) {
            qw0 = a.qw[lane];
            qw1 = a.qw[lane + kHd / 2];
            kw0 = a.kw[lane];
            kw1 = a.kw[lane + kHd / 2];
        }
        // (loaded by every chunk: a load under the branch would wait for the cache loads)
        k0 = a.kn[(size_t)kvh * kHd + lane];
        k1 = a.kn[(size_t)kvh * kHd + lane + kHd / 2];
        v0 = a.vn[(size_t)kvh * kHd + lane];
        v1 = a.vn[(size_t)kvh * kHd + lane + kHd / 2];
        fr = a.freq[lane];
    }

    // ---- cache loads of one chunk.  S waves: the K fragments of tile t (4 steps of 32 dims;
    // lane: position p0 + 16t + r, dims 32s + 8kg .. +7) and, for int8, the positions' K and V
    // scales.  V, blocked layout (O waves): the O = P V fragments themselves, u = 2j + kk holds
    // dim 16(2nv + j) + r, positions 32kk + 8kg .. +7 of the chunk (rows past the sequence are
    // read as stored and weighted by P = 0, so the cache must hold finite values there; the
    // caller zero-fills the blocked cache once).  Rows layout (every wave): 16-element pieces
    // c = lane + 64u, u = 2 wave + i, of the tile (position c / 16, dims 8 (c % 16)), staged
    // through LDS.
    const uint8_t *kc = (const uint8_t *)a.kc, *vc = (const uint8_t *)a.vc;
    uint4 kr[4];  // f16: 8 halves; int8: 8 bytes in .x/.y
    float ksc = 1.0f, vsc = 1.0f;
    uint4 vr[4];
    auto load_k = [&](int p0) {
        const int pt = min(p0 + 16 * t + r, seq - 1);  // this lane's position in tile t (clamped)
#pragma unroll
        for (int st = 0; st < 4; st++) {
            const size_t off = ((size_t)pt * stride_kv + (size_t)kvh * kHd + 32 * st + 8 * kg) * EB;
            if (KV == kKvF16) __builtin_memcpy(&kr[st], kc + off, 16);
            else __builtin_memcpy(&kr[st], kc + off, 8);
        }
        if (KV == kKvInt8) {
            ksc = a.ksc[(size_t)pt * a.nkv + kvh];
            vsc = a.vsc[(size_t)pt * a.nkv + kvh];
        }
    };
    auto load_v = [&](int chunk) {
        const int p0 = chunk * kChunk;
        if (VL == kVBlocked) {
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int n = 2 * nv + (u >> 1), kk = u & 1;
                const size_t off =
                    ((((size_t)chunk * a.nkv + kvh) * kHd + 16 * n + r) * kChunk + 32 * kk + 8 * kg) * EB;
                if (KV == kKvF16) __builtin_memcpy(&vr[u], vc + off, 16);
                else __builtin_memcpy(&vr[u], vc + off, 8);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int c = lane + 64 * (2 * wave + i);
                const int p = min(p0 + (c >> 4), seq - 1);
                const size_t off = ((size_t)p * stride_kv + (size_t)kvh * kHd + 8 * (c & 15)) * EB;
                if (KV == kKvF16) __builtin_memcpy(&vr[i], vc + off, 16);
                else __builtin_memcpy(&vr[i], vc + off, 8);
            }
        }
    };
    if (swave) load_k(g * kChunk);
    if (VL == kVRows || !swave) load_v(g);

    // ---- Q rows (heads kvh*G .. +G-1) as f16 hi + lo
    if (PREP) {
        float sn, cs;
        sincosf((float)pos * fr, &sn, &cs);
#pragma unroll
        for (int j = 0; j < kPrepHeads; j++) {
            const int h = kPrepHeads * wave + j;
            float x0 = qx0[j], x1 = qx1[j];
            prep_head(x0, x1, norm, qw0, qw1, a.eps, cs, sn);
            if (h >= G) x0 = x1 = 0.0f;
            const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
            qs[0][h][lane] = h0;
            qs[0][h][lane + kHd / 2] = h1;
            qs[1][h][lane] = (_Float16)(x0 - (float)h0);
            qs[1][h][lane + kHd / 2] = (_Float16)(x1 - (float)h1);
        }
        if (mine_wg && wave == 0) {
            prep_head(k0, k1, norm, kw0, kw1, a.eps, cs, sn);
            const size_t si = (size_t)pos * a.nkv + kvh;
            const float nk = store_new_row<KV>(k0, k1, a.kcw, a.kscw, si * kHd, 1, si, knew[0]);
            const size_t vb = VL == kVBlocked ? (((size_t)(pos / 64) * a.nkv + kvh) * kHd) * 64 + pos % 64 : si * kHd;
            const float nvs = store_new_row<KV>(v0, v1, a.vcw, a.vscw, vb, VL == kVBlocked ? 64 : 1, si, knew[1]);
            if (lane == 0) {
                new_sc[0] = nk;
                new_sc[1] = nvs;
            }
        }
    } else for (int e = threadIdx.x; e < kRows * kHd / 4; e += kChunkThreads) {
        const int h = e / (kHd / 4), d = 4 * (e % (kHd / 4));
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (h < G) v = *(const float4 *)(a.q + (size_t)(kvh * G + h) * kHd + d);
        const float vv[4] = {v.x, v.y, v.z, v.w};
        _Float16 hi[4], lo[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            hi[j] = (_Float16)vv[j];
            lo[j] = (_Float16)(vv[j] - (float)hi[j]);
        }
        __builtin_memcpy(&qs[0][h][d], hi, 8);
        __builtin_memcpy(&qs[1][h][d], lo, 8);
    }
    __syncthreads();  // 1: Q rows, the new K / V rows and their scales

    // running state of the O waves: rows (heads) 4kg + i, dims of n-tiles 2nv, 2nv + 1
    float Mr[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY}, Lr[4] = {0.f, 0.f, 0.f, 0.f};
    f4 oacc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    for (int chunk = g;;) {
        const int p0 = chunk * kChunk;
        const int next = chunk + stride;
        const bool more = LOOP && next < nc;  // uniform
        if (PREP && mine_wg && chunk == pchunk) {
            // the loaded cache rows at pos are stale: take the new K / V rows from LDS (also
            // where a position past pos was clamped to pos)
            const int o = pos - p0;
            if (swave && 16 * t + r >= o) {
#pragma unroll
                for (int st = 0; st < 4; st++) __builtin_memcpy(&kr[st], &knew[0][(32 * st + 8 * kg) * EB], 8 * EB);
                ksc = new_sc[0];
                vsc = new_sc[1];
            }
            if (VL == kVRows) {
#pragma unroll
                for (int i = 0; i < 2; i++)
                    if (4 * (2 * wave + i) + (lane >> 4) >= o)  // position of the 16-element piece, clamped
                        __builtin_memcpy(&vr[i], &knew[1][8 * (lane & 15) * EB], 8 * EB);
            } else if (!swave && kg == ((o >> 3) & 3)) {
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int n = 2 * nv + (u >> 1), kk = u & 1;
                    if (kk != (o >> 5)) continue;
                    uint8_t *vb = (uint8_t *)&vr[u];
#pragma unroll
                    for (int j = 0; j < 8; j++)
                        if (j == (o & 7)) __builtin_memcpy(vb + j * EB, &knew[1][(16 * n + r) * EB], EB);
                }
            }
        }

        // ---- S waves: tile t of S = Q K^T (lane: heads 4kg + i, position p0 + 16t + r) and
        // its row maxima
        f4 sc = {0.f, 0.f, 0.f, 0.f};
        if (swave) {
#pragma unroll
            for (int st = 0; st < 4; st++) {
                h8 b;
                if (KV == kKvF16) {
                    __builtin_memcpy(&b, &kr[st], 16);
                } else {
                    const int8_t *kb = (const int8_t *)&kr[st];
#pragma unroll
                    for (int j = 0; j < 8; j++) b[j] = (_Float16)kb[j];
                }
                h8 ah, al;
                __builtin_memcpy(&ah, &qs[0][r][32 * st + 8 * kg], 16);
                __builtin_memcpy(&al, &qs[1][r][32 * st + 8 * kg], 16);
                sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, b, sc, 0, 0, 0);
                sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, b, sc, 0, 0, 0);
            }
            const bool ok = p0 + 16 * t + r < seq;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sc[i] = ok ? sc[i] * (a.scale * ksc) : -INFINITY;
                const float mx = max16(sc[i]);
                if (r == 0) tmax[t][4 * kg + i] = mx;
            }
        }
        __syncthreads();  // 2: the tiles' row maxima
        if (swave) {
            // P = exp(S - m) (times the V scale for int8) to LDS as hi + lo; the tile's row sums
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int h = 4 * kg + i;
                float m = tmax[0][h];
#pragma unroll
                for (int u = 1; u < kTiles; u++) m = fmaxf(m, tmax[u][h]);  // finite: position p0 < seq
                const float e = expf(sc[i] - m);  // exp(-inf) = 0 for masked positions
                const float sum = sum16(e);
                if (r == 0) tsum[t][h] = sum;
                const float pv = e * vsc;
                const _Float16 hi = (_Float16)pv;
                ps[0][h][16 * t + r] = hi;
                ps[1][h][16 * t + r] = (_Float16)(pv - (float)hi);
            }
            if (more) load_k(next * kChunk);  // this chunk's K and scales are used
        }
        if (VL == kVRows) {
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int c = lane + 64 * (2 * wave + i);
                h8 v;
                if (KV == kKvF16) {
                    __builtin_memcpy(&v, &vr[i], 16);
                } else {
                    const int8_t *vb = (const int8_t *)&vr[i];
#pragma unroll
                    for (int j = 0; j < 8; j++) v[j] = (_Float16)vb[j];
                }
                __builtin_memcpy(&vt[c >> 4][8 * (c & 15)], &v, 16);
            }
            if (more) load_v(next);  // the pieces are in LDS
        }
        __syncthreads();  // 3: P, the row sums and (rows layout) the V tile
        constexpr bool single = !LOOP;  // the workgroup's only chunk (a looping one has >= 2)
        if (single && wave == 0 && lane < kRows) {
            // its m and l: the 16 heads' maxima and sums over the tiles, in tile order
            float m = tmax[0][lane], l = tsum[0][lane];
#pragma unroll
            for (int u = 1; u < kTiles; u++) {
                m = fmaxf(m, tmax[u][lane]);
                l += tsum[u][lane];
            }
            float *part = a.ws + ((size_t)kvh * a.max_chunks + g) * kPart;
            part[lane] = m;
            part[kRows + lane] = l;
        }
        if (!swave) {
            // ---- O waves: O = P V for n-tiles 2nv, 2nv + 1 (16 dims each), 2 steps of 32
            // positions, merged into the running state
            f4 o[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
            for (int kk = 0; kk < 2; kk++) {
                h8 ah, al;
                __builtin_memcpy(&ah, &ps[0][r][32 * kk + 8 * kg], 16);
                __builtin_memcpy(&al, &ps[1][r][32 * kk + 8 * kg], 16);
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int n = 2 * nv + j;
                    h8 b;
                    if (VL == kVRows) {
#pragma unroll
                        for (int q = 0; q < 8; q++) b[q] = vt[32 * kk + 8 * kg + q][16 * n + r];
                    } else if (KV == kKvF16) {
                        __builtin_memcpy(&b, &vr[2 * j + kk], 16);
                    } else {
                        const int8_t *vb = (const int8_t *)&vr[2 * j + kk];
#pragma unroll
                        for (int q = 0; q < 8; q++) b[q] = (_Float16)vb[q];
                    }
                    o[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, b, o[j], 0, 0, 0);
                    o[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, b, o[j], 0, 0, 0);
                }
            }
            if (VL == kVBlocked && more) load_v(next);  // this chunk's fragments are used
            if (single) {
#pragma unroll
                for (int j = 0; j < 2; j++) oacc[j] = o[j];
            } else {
                // the chunk's max and (tile-order) sum per head, merged into the running state
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int h = 4 * kg + i;
                    float m = tmax[0][h], l = tsum[0][h];
#pragma unroll
                    for (int u = 1; u < kTiles; u++) {
                        m = fmaxf(m, tmax[u][h]);
                        l += tsum[u][h];
                    }
                    const float mn = fmaxf(Mr[i], m);  // finite: the chunk holds position p0 < seq
                    const float ea = expf(Mr[i] - mn);
                    const float eb = expf(m - mn);
                    Lr[i] = fmaf(Lr[i], ea, l * eb);
#pragma unroll
                    for (int j = 0; j < 2; j++) oacc[j][i] = fmaf(oacc[j][i], ea, o[j][i] * eb);
                    Mr[i] = mn;
                }
            }
        }
        if (!more) break;
        __syncthreads();  // 4: this chunk's P, maxima, sums and V tile are read
        chunk = next;
    }
    if (swave) return;
    // ---- the partial: m and l of the 16 heads (a single chunk's came from wave 0),
    // O[16][128] (this wave's 32 dims)
    float *part = a.ws + ((size_t)kvh * a.max_chunks + g) * kPart;
    if (LOOP && nv == 0 && r == 0) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            part[4 * kg + i] = Mr[i];
            part[kRows + 4 * kg + i] = Lr[i];
        }
    }
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) part[2 * kRows + (4 * kg + i) * kHd + 16 * (2 * nv + j) + r] = oacc[j][i];
}

template <int KV, int VL, bool PREP>
__global__ void __launch_bounds__(kChunkThreads) attn_chunk_kernel(AttnDecodeArgs a) {
    __shared__ __align__(16) ChunkLds<KV, VL, PREP> L;
    const int pos = a.pos_dev ? *a.pos_dev : a.seq_fixed - 1;
    const int seq = min(pos + 1, a.max_ctx);
    const int nc = (seq + kChunk - 1) / kChunk;
    const int stride = chunk_stride(nc, VL == kVBlocked ? 1 : 2);
    if ((int)blockIdx.y >= stride) return;  // the combine reads `stride` partials per KV head
    if (stride < nc) chunk_body<KV, VL, PREP, true>(a, L, pos, seq, nc, stride);
    else chunk_body<KV, VL, PREP, false>(a, L, pos, seq, nc, stride);
}

// Merge of the chunks' (max, sum, O): grid (query head, quarter of head_dim), 256 threads =
// 32 dims x 8 chunk groups.  Thread (d, g) takes chunks g, g + 8, ... in batches of 8 per
// thread (64 chunks = 4096 positions per batch), every load of a batch issued before any
// arithmetic: one round trip to the partials instead of three dependent ones.  Per batch:
// the max over its chunks, then sum l and O with weights exp(m_c - M) (rescaled when a later
// batch raises M); the 8 groups meet in LDS in a fixed order.
constexpr int kCombThreads = 256;
constexpr int kCombDims = kHd / 4;                    // dims per workgroup
constexpr int kCombGroups = kCombThreads / kCombDims;  // 8
constexpr int kCombPer = 8;                           // chunks per thread and batch
constexpr int kMaxChunks = 1024;                      // max_ctx <= 65536

__global__ void __launch_bounds__(kCombThreads) attn_combine_kernel(AttnDecodeArgs a) {
    __shared__ float red_m[kCombGroups], red_l[kCombGroups];
    __shared__ float part_o[kCombThreads];
    const int h = blockIdx.x, tid = threadIdx.x;
    const int kvh = h / a.gqa, hh = h % a.gqa;
    const int seq = min((a.pos_dev ? *a.pos_dev : a.seq_fixed - 1) + 1, a.max_ctx);
    const int nchunks = (seq + kChunk - 1) / kChunk;
    const int nc = chunk_stride(nchunks, a.loop_split);  // partials per KV head
    const float *base = a.ws + (size_t)kvh * a.max_chunks * kPart;
    const int dl = tid % kCombDims, g = tid / kCombDims;
    const int d = (int)blockIdx.y * kCombDims + dl;
    float M = -INFINITY, L = 0.0f, O = 0.0f;  // this thread's running state
    for (int c0 = 0; c0 < nc; c0 += kCombGroups * kCombPer) {
        float m[kCombPer], l[kCombPer], o[kCombPer];
#pragma unroll
        for (int i = 0; i < kCombPer; i++) {
            const int c = min(c0 + g + kCombGroups * i, nc - 1);  // clamped: loaded, then masked
            const float *pc = base + (size_t)c * kPart;
            m[i] = pc[hh];
            l[i] = pc[kRows + hh];
            o[i] = pc[2 * kRows + hh * kHd + d];
        }
        float bm = M;
#pragma unroll
        for (int i = 0; i < kCombPer; i++)
            if (c0 + g + kCombGroups * i < nc) bm = fmaxf(bm, m[i]);
        const float r = M == bm ? 1.0f : expf(M - bm);  // 0 when M was -inf
        L *= r;
        O *= r;
#pragma unroll
        for (int i = 0; i < kCombPer; i++) {
            const float w = c0 + g + kCombGroups * i < nc ? expf(m[i] - bm) : 0.0f;
            L = fmaf(l[i], w, L);
            O = fmaf(o[i], w, O);
        }
        M = bm;
    }
    // groups of the same dims: common max, then the sums in group order
    if (dl == 0) red_m[g] = M;
    __syncthreads();
    float gm = red_m[0];
#pragma unroll
    for (int i = 1; i < kCombGroups; i++) gm = fmaxf(gm, red_m[i]);
    const float r = M > -INFINITY ? expf(M - gm) : 0.0f;  // a group without chunks adds nothing
    if (dl == 0) red_l[g] = L * r;
    part_o[tid] = O * r;
    __syncthreads();
    if (tid < kCombDims) {
        float Ls = 0.0f, o = 0.0f;
#pragma unroll
        for (int j = 0; j < kCombGroups; j++) {
            Ls += red_l[j];
            o += part_o[tid + j * kCombDims];
        }
        a.out[(size_t)h * kHd + d] = o / Ls;
    }
}

static int check_decode_args(AttnDecodeArgs &a, int kv_type) {
    if (!a.q || !a.kc || !a.vc || !a.out || (!a.pos_dev && a.seq_fixed <= 0) || !a.ws)
        return set_error(kErrBadArg, "attention_decode: NULL pointer");
    if (a.hd != kHd) return set_error(kErrBadArg, "attention_decode: head_dim %d (this kernel: %d)", a.hd, kHd);
    if (a.nkv <= 0 || a.gqa <= 0 || a.gqa > kRows || a.nh != a.nkv * a.gqa)
        return set_error(kErrBadArg, "attention_decode: n_heads = n_kv_heads * gqa with gqa <= %d", kRows);
    if (a.max_ctx <= 0 || a.max_ctx > kMaxChunks * kChunk)
        return set_error(kErrBadArg, "attention_decode: max_ctx must be in 1..%d", kMaxChunks * kChunk);
    if (kv_type == kKvInt8 && (!a.ksc || !a.vsc)) return set_error(kErrBadArg, "attention_decode: int8 needs scales");
    if (kv_type != kKvF16 && kv_type != kKvInt8) return set_error(kErrBadArg, "attention_decode: kv_type %d", kv_type);
    if (a.v_layout != kVRows && a.v_layout != kVBlocked)
        return set_error(kErrBadArg, "attention_decode: v_layout %d", a.v_layout);
    if (a.ws_bytes < attn_decode_workspace_bytes(a.nkv, a.max_ctx))
        return set_error(kErrBadArg, "attention_decode: workspace %zu < %zu bytes", a.ws_bytes,
                         attn_decode_workspace_bytes(a.nkv, a.max_ctx));
    a.max_chunks = (a.max_ctx + kChunk - 1) / kChunk;
    a.loop_split = a.v_layout == kVBlocked ? 1 : 2;
    return 0;
}

template <bool PREP>
static int launch_decode(const AttnDecodeArgs &a, int kv_type, hipStream_t s) {
    // KV heads fastest: the workgroups are dispatched in order, so the chunks inside the
    // sequence (the lowest chunk indices) start first and those past it (which exit at once)
    // queue behind them -- with chunks fastest, a KV head's live chunks waited for the
    // previous head's whole chunk range to be dispatched (2 K positions of a 40 K cache:
    // 9.4 -> 8.3 us for the chunk and merge launches)
    const dim3 grid(a.nkv, a.max_chunks);
    if (kv_type == kKvF16) {
        if (a.v_layout == kVBlocked)
            hipLaunchKernelGGL((attn_chunk_kernel<kKvF16, kVBlocked, PREP>), grid, dim3(kChunkThreads), 0, s, a);
        else hipLaunchKernelGGL((attn_chunk_kernel<kKvF16, kVRows, PREP>), grid, dim3(kChunkThreads), 0, s, a);
    } else {
        if (a.v_layout == kVBlocked)
            hipLaunchKernelGGL((attn_chunk_kernel<kKvInt8, kVBlocked, PREP>), grid, dim3(kChunkThreads), 0, s, a);
        else hipLaunchKernelGGL((attn_chunk_kernel<kKvInt8, kVRows, PREP>), grid, dim3(kChunkThreads), 0, s, a);
    }
    hipLaunchKernelGGL(attn_combine_kernel, dim3(a.nh, kHd / kCombDims), dim3(kCombThreads), 0, s, a);
    return check_launch("attention_decode");
}

int launch_attention_decode(AttnDecodeArgs a, int kv_type, hipStream_t s) {
    if (int rc = check_decode_args(a, kv_type)) return rc;
    return launch_decode<false>(a, kv_type, s);
}

// q raw; kn / vn the raw K / V heads of the new token; the caches are written at *pos_dev
// (nothing is stored when *pos_dev >= max_ctx, and the attention covers 0..max_ctx-1).
int launch_attention_decode_prep(AttnDecodeArgs a, int kv_type, float theta, hipStream_t s) {
    if (int rc = check_decode_args(a, kv_type)) return rc;
    if (!a.kn || !a.vn || !a.kcw || !a.vcw || (kv_type == kKvInt8 && (!a.kscw || !a.vscw)))
        return set_error(kErrBadArg, "attention_decode_prep: NULL new K / V or cache pointer");
    if ((a.qw == nullptr) != (a.kw == nullptr))
        return set_error(kErrBadArg, "attention_decode_prep: give both QK-norm weights or neither");
    // the frequencies of head_pass_kernel's RoPE, computed the same way
    for (int j = 0; j < kHd / 2; j++) a.freq[j] = 1.0f / powf(theta, (float)(2 * j) / (float)kHd);
    return launch_decode<true>(a, kv_type, s);
}

// ------------------------------------------------------------------ the reference's entry points
// cuda_attention_f16kv / _int8kv: the reference's row caches (K and V [pos][n_kv][hd]) and a
// host sequence length.  At head_dim 128 and gqa <= 16 they run attention_rows_kernel plus the
// chunk merge above.  The reference captures cuda_attention_f16kv in a graph and patches the
// sequence length of the captured node before every replay (forward.c:658-666: kernelParams[6]
// of the node whose function is cuda_get_attn_f16kv_kernel_ptr(), kernels.cu:2245), so:
//  * attention_rows_kernel takes the reference kernel's parameters in the reference's order
//    (kernels.cu:1550-1554: q, kv_k, kv_v, out, head_dim, n_kv_heads, seq_len, gqa_ratio,
//    scale), then its own (workspace, split count, int8 scales);
//  * its grid does not depend on seq_len: (n_kv_heads, nsplit) workgroups, workgroup g taking
//    the 64-position chunks g, g + nsplit, ... and merging them as it goes (running max, sum
//    and O), so one workgroup leaves one partial whatever the length;
//  * it writes the number of partials to the workspace header, from which the merge launch
//    (whose arguments hold no length) reads it.
// With at most nsplit chunks every workgroup takes one chunk and the partials are exactly
// those of attn_chunk_kernel.
constexpr int kSplitTarget = 512;  // workgroups per launch (two per CU)
constexpr int kRowsMaxKv = kSplitTarget;
static int rows_nsplit(int nkv) { return max(1, kSplitTarget / nkv); }
// partials for nkv * nsplit <= kSplitTarget workgroups, then the header (one int)
constexpr size_t kRowsSlotBytes = (size_t)kSplitTarget * kPart * sizeof(float) + 256;

template <int KV>
__global__ void __launch_bounds__(kChunkThreads)
    attention_rows_kernel(const float *__restrict__ q, const void *__restrict__ kv_k, const void *__restrict__ kv_v,
                          float *out, int head_dim, int n_kv_heads, int seq_len, int gqa_ratio, float scale,
                          float *ws, int nsplit, const float *__restrict__ k_scales,
                          const float *__restrict__ v_scales) {
    (void)out;       // written by the merge launch
    (void)head_dim;  // 128: checked by the host
    __shared__ __align__(16) _Float16 qs[2][kRows][kHd + 8];
    __shared__ __align__(16) _Float16 vt[kChunk][kHd + 8];
    __shared__ __align__(16) _Float16 ps[2][kRows][kChunk + 8];
    __shared__ float tmax[kTiles][kRows], tsum[kTiles][kRows];
    const int kvh = blockIdx.x, g = blockIdx.y, lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int seq = max(seq_len, 1);
    const int nchunks = (seq + kChunk - 1) / kChunk;
    if (kvh == 0 && g == 0 && threadIdx.x == 0)  // the merge reads min(nchunks, nsplit) partials
        *(int *)(ws + (size_t)n_kv_heads * nsplit * kPart) = kChunk * min(nchunks, nsplit) - 1;
    if (g >= nchunks) return;
    const int G = gqa_ratio;
    const size_t stride = (size_t)n_kv_heads * kHd;
    const int r = lane & 15, kg = lane >> 4;
    const bool swave = wave < kTiles;
    const int t = wave & (kTiles - 1);
    const int nv = wave - kTiles;
    constexpr int EB = KV == kKvF16 ? 2 : 1;
    const uint8_t *kc = (const uint8_t *)kv_k, *vc = (const uint8_t *)kv_v;

    // Q rows (heads kvh*G .. +G-1) as f16 hi + lo, once for all chunks
    for (int e = threadIdx.x; e < kRows * kHd / 4; e += kChunkThreads) {
        const int h = e / (kHd / 4), d = 4 * (e % (kHd / 4));
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (h < G) v = *(const float4 *)(q + (size_t)(kvh * G + h) * kHd + d);
        const float vv[4] = {v.x, v.y, v.z, v.w};
        _Float16 hi[4], lo[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            hi[j] = (_Float16)vv[j];
            lo[j] = (_Float16)(vv[j] - (float)hi[j]);
        }
        __builtin_memcpy(&qs[0][h][d], hi, 8);
        __builtin_memcpy(&qs[1][h][d], lo, 8);
    }

    // running state of the O waves: rows (heads) 4kg + i, dims of n-tiles 2nv, 2nv + 1
    float Mr[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY}, Lr[4] = {0.f, 0.f, 0.f, 0.f};
    f4 oacc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    for (int chunk = g; chunk < nchunks; chunk += nsplit) {
        const int p0 = chunk * kChunk;
        // loads: K fragments of tile t (S waves), the 16-element V pieces of every wave
        const int pt = min(p0 + 16 * t + r, seq - 1);
        uint4 kr[4];
        float ksc = 1.0f, vsc = 1.0f;
        if (swave) {
#pragma unroll
            for (int st = 0; st < 4; st++) {
                const size_t off = ((size_t)pt * stride + (size_t)kvh * kHd + 32 * st + 8 * kg) * EB;
                if (KV == kKvF16) __builtin_memcpy(&kr[st], kc + off, 16);
                else __builtin_memcpy(&kr[st], kc + off, 8);
            }
            if (KV == kKvInt8) {
                ksc = k_scales[(size_t)pt * n_kv_heads + kvh];
                vsc = v_scales[(size_t)pt * n_kv_heads + kvh];
            }
        }
        uint4 vr[2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int c = lane + 64 * (2 * wave + i);
            const int p = min(p0 + (c >> 4), seq - 1);
            const size_t off = ((size_t)p * stride + (size_t)kvh * kHd + 8 * (c & 15)) * EB;
            if (KV == kKvF16) __builtin_memcpy(&vr[i], vc + off, 16);
            else __builtin_memcpy(&vr[i], vc + off, 8);
        }
        __syncthreads();  // 1: Q rows (first chunk); the previous chunk's LDS reads are done
        f4 sc = {0.f, 0.f, 0.f, 0.f};
        if (swave) {
#pragma unroll
            for (int st = 0; st < 4; st++) {
                h8 b;
                if (KV == kKvF16) {
                    __builtin_memcpy(&b, &kr[st], 16);
                } else {
                    const int8_t *kb = (const int8_t *)&kr[st];
#pragma unroll
                    for (int j = 0; j < 8; j++) b[j] = (_Float16)kb[j];
                }
                h8 ah, al;
                __builtin_memcpy(&ah, &qs[0][r][32 * st + 8 * kg], 16);
                __builtin_memcpy(&al, &qs[1][r][32 * st + 8 * kg], 16);
                sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, b, sc, 0, 0, 0);
                sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, b, sc, 0, 0, 0);
            }
            const bool ok = p0 + 16 * t + r < seq;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sc[i] = ok ? sc[i] * (scale * ksc) : -INFINITY;
                const float mx = max16(sc[i]);
                if (r == 0) tmax[t][4 * kg + i] = mx;
            }
        }
        __syncthreads();  // 2: the tiles' row maxima
        if (swave) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int h = 4 * kg + i;
                float m = tmax[0][h];
#pragma unroll
                for (int u = 1; u < kTiles; u++) m = fmaxf(m, tmax[u][h]);
                const float e = expf(sc[i] - m);
                const float sum = sum16(e);
                if (r == 0) tsum[t][h] = sum;
                const float pv = e * vsc;
                const _Float16 hi = (_Float16)pv;
                ps[0][h][16 * t + r] = hi;
                ps[1][h][16 * t + r] = (_Float16)(pv - (float)hi);
            }
        }
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int c = lane + 64 * (2 * wave + i);
            h8 v;
            if (KV == kKvF16) {
                __builtin_memcpy(&v, &vr[i], 16);
            } else {
                const int8_t *vb = (const int8_t *)&vr[i];
#pragma unroll
                for (int j = 0; j < 8; j++) v[j] = (_Float16)vb[j];
            }
            __builtin_memcpy(&vt[c >> 4][8 * (c & 15)], &v, 16);
        }
        __syncthreads();  // 3: P, the row sums and the V tile
        if (!swave) {
            f4 o[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
            for (int kk = 0; kk < 2; kk++) {
                h8 ah, al;
                __builtin_memcpy(&ah, &ps[0][r][32 * kk + 8 * kg], 16);
                __builtin_memcpy(&al, &ps[1][r][32 * kk + 8 * kg], 16);
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int n = 2 * nv + j;
                    h8 b;
#pragma unroll
                    for (int qq = 0; qq < 8; qq++) b[qq] = vt[32 * kk + 8 * kg + qq][16 * n + r];
                    o[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, b, o[j], 0, 0, 0);
                    o[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, b, o[j], 0, 0, 0);
                }
            }
            // merge into the running state: the chunk's max and (tile-order) sum per head
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int h = 4 * kg + i;
                float m = tmax[0][h], l = tsum[0][h];
#pragma unroll
                for (int u = 1; u < kTiles; u++) {
                    m = fmaxf(m, tmax[u][h]);
                    l += tsum[u][h];
                }
                const float mn = fmaxf(Mr[i], m);       // finite: the chunk holds position p0 < seq
                const float a = expf(Mr[i] - mn);       // 0 on the first chunk
                const float b = expf(m - mn);
                Lr[i] = fmaf(Lr[i], a, l * b);
#pragma unroll
                for (int j = 0; j < 2; j++) oacc[j][i] = fmaf(oacc[j][i], a, o[j][i] * b);
                Mr[i] = mn;
            }
        }
    }
    if (swave) return;
    float *part = ws + ((size_t)kvh * nsplit + g) * kPart;
    if (nv == 0 && r == 0) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            part[4 * kg + i] = Mr[i];
            part[kRows + 4 * kg + i] = Lr[i];
        }
    }
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) part[2 * kRows + (4 * kg + i) * kHd + 16 * (2 * nv + j) + r] = oacc[j][i];
}

// Workspaces of the entry points, kRowsSlotBytes each, per GPU.  A stream's eager calls use
// the slot bound to that stream (bound at its first call); a call made while its stream is
// being captured takes a free slot for good, so that the captured graph may be replayed on any
// stream while other graphs and eager calls run.  cuda_kernels_init reserves kRowsPoolInit
// free slots; mnemo_attention_reserve adds more (outside any capture: it allocates); the calls
// themselves never allocate.  A capture that finds no free slot shares its stream's slot (one
// warning is printed): such a graph must then be replayed in order with the eager calls of
// that stream.  A stream that finds none runs the per-head kernel.  Calls that overlap in time
// never share a slot otherwise.
constexpr int kRowsPoolInit = 16;
constexpr int kMaxRowsDevices = 64;
constexpr int kMaxRowsStreams = 64;
struct RowsPool {
    float *free_slots[1024];
    int nfree = 0;
    hipStream_t stream[kMaxRowsStreams];
    float *bound[kMaxRowsStreams];
    int nbound = 0;
    bool warned = false;
};
static RowsPool g_rows[kMaxRowsDevices];
static std::mutex g_rows_mu;

static int rows_reserve_locked(RowsPool &P, int n) {
    while (P.nfree < n && P.nfree < (int)(sizeof P.free_slots / sizeof P.free_slots[0])) {
        void *p = nullptr;
        if (hipMalloc(&p, kRowsSlotBytes) != hipSuccess) {
            (void)hipGetLastError();
            return kErrLaunch;
        }
        P.free_slots[P.nfree++] = (float *)p;
    }
    return P.nfree >= n ? kOk : kErrBadArg;
}

int attn_rows_reserve(int n) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxRowsDevices) return kErrLaunch;
    std::lock_guard<std::mutex> lock(g_rows_mu);
    return rows_reserve_locked(g_rows[dev], n);
}

int attn_rows_ws_init() { return attn_rows_reserve(kRowsPoolInit); }

size_t attn_rows_slot_bytes() { return kRowsSlotBytes; }

// The slot for a call on stream s, or nullptr (then the per-head kernel runs).
static float *rows_slot(hipStream_t s) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxRowsDevices) return nullptr;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess) {
        (void)hipGetLastError();
        cs = hipStreamCaptureStatusNone;
    }
    const bool capturing = cs == hipStreamCaptureStatusActive;
    std::lock_guard<std::mutex> lock(g_rows_mu);
    RowsPool &P = g_rows[dev];
    if (capturing && P.nfree > 0) return P.free_slots[--P.nfree];  // the graph's own slot
    for (int i = 0; i < P.nbound; i++)
        if (P.stream[i] == s) {
            if (capturing && !P.warned) {
                P.warned = true;
                fprintf(stderr,
                        "[mnemo] cuda_attention_*: no free workspace slot for a graph capture; it shares its "
                        "stream's slot (call mnemo_attention_reserve before capturing)\n");
            }
            return P.bound[i];
        }
    if (P.nbound == kMaxRowsStreams || P.nfree == 0) {  // no allocation here: the per-head kernel runs
        if (!P.warned) {
            P.warned = true;
            fprintf(stderr,
                    "[mnemo] cuda_attention_*: no free workspace slot for this stream; the per-head kernel runs "
                    "(call mnemo_attention_reserve)\n");
        }
        return nullptr;
    }
    P.stream[P.nbound] = s;
    P.bound[P.nbound] = P.free_slots[--P.nfree];
    return P.bound[P.nbound++];
}

void *attn_rows_kernel_ptr() { return reinterpret_cast<void *>(&attention_rows_kernel<kKvF16>); }

// Returns kErrBadArg without recording an error when the split kernels do not apply.
int launch_attention_rows(const float *q, const void *kc, const void *vc, const float *ksc, const float *vsc,
                          int kv_type, float *out, int nh, int hd, int nkv, int gqa, int seq, float scale,
                          hipStream_t s) {
    if (hd != kHd || gqa <= 0 || gqa > kRows || nkv <= 0 || nkv > kRowsMaxKv || nh != nkv * gqa || seq <= 0)
        return kErrBadArg;
    if (!q || !kc || !vc || !out || (kv_type == kKvInt8 && (!ksc || !vsc))) return kErrBadArg;
    float *ws = rows_slot(s);
    if (!ws) return kErrBadArg;
    const int nsplit = rows_nsplit(nkv);
    if (kv_type == kKvF16)
        hipLaunchKernelGGL(attention_rows_kernel<kKvF16>, dim3(nkv, nsplit), dim3(kChunkThreads), 0, s, q, kc, vc,
                           out, hd, nkv, seq, gqa, scale, ws, nsplit, ksc, vsc);
    else
        hipLaunchKernelGGL(attention_rows_kernel<kKvInt8>, dim3(nkv, nsplit), dim3(kChunkThreads), 0, s, q, kc, vc,
                           out, hd, nkv, seq, gqa, scale, ws, nsplit, ksc, vsc);
    AttnDecodeArgs a{};
    a.out = out;
    a.ws = ws;
    a.nh = nh;
    a.hd = hd;
    a.nkv = nkv;
    a.gqa = gqa;
    a.max_chunks = nsplit;
    a.max_ctx = kChunk * nsplit;
    a.pos_dev = (const int *)(ws + (size_t)nkv * nsplit * kPart);  // written by attention_rows_kernel
    hipLaunchKernelGGL(attn_combine_kernel, dim3(a.nh, kHd / kCombDims), dim3(kCombThreads), 0, s, a);
    return check_launch("cuda_attention (split)");
}

}  // namespace mnemo
