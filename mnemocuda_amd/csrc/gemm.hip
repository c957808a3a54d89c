// gemm.hip -- Q4_K / Q6_K x Q8_1 GEMM for prefill and batched experts (gfx950 MFMA).
//
// Semantics (MnemoCUDA gemm_q4k.cu:103-112, 164-166, 194):
//   out[j*M + i] = sum_k deq(W)[i][k] * deq(A)[j][k]
// with W GGUF blocks [M][K] and A the Q8_1 MMQ activations [N][K/128] x 144 B.
//
// Design: both operands become f16 tiles in LDS multiplied with v_mfma_f32_16x16x32_f16
// (fp32 accumulate).  The per-32 scales of both operands are folded into the values, so
// the MFMA accumulates across the whole K without a per-sub-block fp32 rescale (an int8
// MFMA would need one cvt + two FMAs per output per 32-K step, several times the MFMA
// time in VALU work).
//   * Activation values d8*q8 are held in f16 scaled per row by 2^-e_row, an exact power
//     of two chosen so that they stay inside the f16 range (127*max d8*2^-e <= 2^15); the
//     epilogue multiplies by 2^e.  The reference entry points (cuda_gemm_q4k,
//     mnemo_gemm_q6k) convert Q8_1 blocks per tile and allocate nothing; the grouped
//     expert path stages each activation row once in that f16 form (stage_* kernels, in
//     the caller's workspace) and copies tiles.
//   * Weights are dequantised on the fly in packed f16 arithmetic: a quant q placed under
//     the exponent byte 0x64 is the f16 1024 + q; subtracting 1024 (or 1056 for Q6_K's
//     q - 32) is exact; then one fma with (f16(d*sc), f16(-dmin*m)) (Q4_K) or one multiply
//     by f16(d*sc) (Q6_K).  Expected relative L2 error vs the fp64 product: ~4e-4.
//   * Workgroup tile 128 weight rows x 128 tokens (8 waves: quadrants of 64 x 64 = 4 x 4 MFMA
//     tiles, each quadrant split over two waves by K half),
//     K step 64 (one Q4_K nibble group, one Q6_K ql group).  Raw weight blocks and
//     activation chunks are loaded into registers ahead of their conversion; f16 tiles
//     rotate through three LDS buffers (XOR-swizzled, conflict-free); one barrier per step.
//   * When the tile grid covers at most half of the CUs, K is split across workgroups
//     and the partial tiles are summed with fp32 atomics into the output, which a small
//     fill kernel zeroes first; the tiles pass through LDS so that each atomic instruction
//     covers 64 consecutive outputs of one token.
#include <algorithm>

#include "mnemo_common.hpp"
#include "mnemo_internal.hpp"

namespace mnemo {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kKS = 64;              // K per step

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    h2 v = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, v);
}

// ------------------------------------------------------------------ raw loads (step k)
// 512 loader threads: thread t owns row (weights) / token (activations) t/4 and quarter
// q = t%4 (16 values) of the 64-wide K step.
struct RawW {
    uint4 a, b;       // Q4_K: a = header (d, dmin, 12 scale bytes), b = 16 qs bytes
                      // Q6_K: a = 16 ql bytes, b = 16 qh bytes
    uint32_t s, dd;   // Q6_K: the int8 scale of the 16 values, f16 d
};
// Activation quarter: staged f16 values, or 16 int8 of a raw Q8_1 sub-block.
template <bool Q8>
struct RawA {
    uint4 a, b;  // 16 f16 values
};
template <>
struct RawA<true> {
    uint4 a;      // 16 int8
    uint32_t ds;  // half2 (d, d*sum) of their 32-value sub-block
};

// Q4_K step ks: super-block ks/4, nibble group g = ks%4 (qs bytes 32g..32g+31).  Quarter q:
// qs bytes 32g + 16(q%2) .. +15, low nibbles (sub-block 2g) for q < 2, else high (2g+1).
__device__ __forceinline__ void load_w_q4k(const uint8_t *__restrict__ wrow, int ks, int q, RawW &r) {
    const uint8_t *blk = wrow + (size_t)(ks >> 2) * kQ4KBytes;
    r.a = ld16(blk);
    r.b = ld16(blk + 16 + 32 * (ks & 3) + 16 * (q & 1));
}

// Q6_K step ks: values 64(ks%4) .. +63 of super-block ks/4, half hh = (ks%4)/2, groups
// 2(ks%2) .. +1.  Quarter q: group grp = 2(ks%2) + q/2, values 16(q%2) .. +15 of it: ql bytes
// 64hh + 32(q/2) + 16(q%2) (low nibbles if grp < 2, else high), qh bytes 32hh + 16(q%2) at
// bit 2grp, scale byte 8hh + 2grp + q%2.
__device__ __forceinline__ void load_w_q6k(const uint8_t *__restrict__ wrow, int ks, int q, RawW &r) {
    const uint8_t *blk = wrow + (size_t)(ks >> 2) * kQ6KBytes;
    const int g = ks & 3, hh = g >> 1, grp = 2 * (g & 1) + (q >> 1);
    r.a = ld16_a2(blk + 64 * hh + 32 * (q >> 1) + 16 * (q & 1));
    r.b = ld16_a2(blk + 128 + 32 * hh + 16 * (q & 1));
    uint8_t sc;
    uint16_t dd;
    __builtin_memcpy(&sc, blk + 192 + 8 * hh + 2 * grp + (q & 1), 1);
    __builtin_memcpy(&dd, blk + 208, 2);
    r.s = sc;
    r.dd = dd;
}

// Activations of step ks, quarter q: values 64ks + 16q .. +15 of the row (staged f16 row,
// or the row's Q8_1 MMQ blocks: block v/128, sub-block (v/32)%4).
__device__ __forceinline__ void load_a(const void *__restrict__ arow, int ks, int q, RawA<false> &r) {
    const _Float16 *p = (const _Float16 *)arow + ks * kKS + 16 * q;
    r.a = ld16((const uint8_t *)(p));
    r.b = ld16((const uint8_t *)(p + 8));
}
__device__ __forceinline__ void load_a(const void *__restrict__ arow, int ks, int q, RawA<true> &r) {
    const int v0 = ks * kKS + 16 * q;
    const uint8_t *blk = (const uint8_t *)arow + (size_t)(v0 >> 7) * kQ81Bytes;
    const int sub = (v0 >> 5) & 3;
    __builtin_memcpy(&r.ds, blk + 4 * sub, 4);
    r.a = ld16(blk + 16 + (v0 & 127));
}

// ------------------------------------------------------------------ LDS tiles
// f16 tiles of 64 K-columns per row = 8 chunks of 16 B, stored without padding with the
// chunk index XOR-ed by (row % 8): the 8 rows read by one phase of an MFMA fragment load
// then fall in 8 different chunks (no bank conflicts), and conversion stores spread too.
__device__ __forceinline__ int tile_off(int row, int chunk) { return row * kKS + ((chunk ^ (row & 7)) << 3); }

__device__ __forceinline__ void put16(_Float16 *tile, int row, int chunk, uint32_t a, uint32_t b, uint32_t c,
                                      uint32_t d) {
    *(uint4 *)(tile + tile_off(row, chunk)) = make_uint4(a, b, c, d);
}

// ------------------------------------------------------------------ conversion to LDS
// Two byte-sized quants (bytes selected by `sel` from v) as the f16 pair 1024 + q.
__device__ __forceinline__ h2 magic_pair(uint32_t v, uint32_t sel) {
    return __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, v, sel));
}
// (q - 1024 + 1024) * a + b for two quants, in packed f16 (exact subtraction, one rounding)
__device__ __forceinline__ uint32_t dq_fma(uint32_t v, uint32_t sel, h2 a, h2 b) {
    const h2 off = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    const h2 q = magic_pair(v, sel) + off;
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q, a, b));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

// Row exponent e >= 0 with 127 * dmax * 2^-e <= 2^15 (dmax = largest |d8| of the row).
__device__ __forceinline__ int row_exponent(float dmax) {
    int ex = 0;
    frexpf(dmax * 127.0f, &ex);  // 127 * dmax < 2^ex
    return max(0, ex - 15);
}

// 8 int8 quants (two dwords) times the f16 scale d: q8 ^ 0x80 under the exponent byte 0x64
// is 1024 + q8 + 128 exactly; subtracting 1152 gives q8; the product is rounded once.
__device__ __forceinline__ void q8x4_to_f16(uint32_t v, h2 d2, uint32_t &o0, uint32_t &o1) {
    const h2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const uint32_t u = v ^ 0x80808080u;
    o0 = __builtin_bit_cast(uint32_t, (magic_pair(u, 0x04010400u) + off) * d2);
    o1 = __builtin_bit_cast(uint32_t, (magic_pair(u, 0x04030402u) + off) * d2);
}

// byte i of the 12 packed scale bytes held in three dwords
__device__ __forceinline__ uint32_t sbyte(uint32_t s0, uint32_t s1, uint32_t s2, int i) {
    const uint32_t w = i < 4 ? s0 : (i < 8 ? s1 : s2);
    return (w >> (8 * (i & 3))) & 0xFFu;
}

// Q4_K quarter q of step ks: sub-block j = 2(ks%4) + q/2 (get_scale_min_k4, kernels.cu:45-53),
// K columns 16q .. 16q+15 of the step (chunks 2q, 2q+1).
__device__ __forceinline__ void store_w_q4k(const RawW &r, int ks, int q, _Float16 *tile, int row) {
    const int j = 2 * (ks & 3) + (q >> 1);
    const uint32_t s0 = r.a.y, s1 = r.a.z, s2 = r.a.w;
    uint32_t sc, m;
    if ((ks & 3) < 2) {  // j < 4, written in terms of the step alone: uniform over the wave
        sc = sbyte(s0, s1, s2, j) & 63;
        m = sbyte(s0, s1, s2, j + 4) & 63;
    } else {
        sc = (sbyte(s0, s1, s2, j + 4) & 15) | ((sbyte(s0, s1, s2, j - 4) >> 6) << 4);
        m = (sbyte(s0, s1, s2, j + 4) >> 4) | ((sbyte(s0, s1, s2, j) >> 6) << 4);
    }
    const float d = h2f(r.a.x & 0xFFFFu), dmin = h2f(r.a.x >> 16);
    const _Float16 a = (_Float16)(d * (float)sc), b = (_Float16)(-dmin * (float)m);
    const h2 A = {a, a}, B = {b, b};
    const int sh = 4 * (q >> 1);
    const uint32_t w[4] = {(r.b.x >> sh) & 0x0F0F0F0Fu, (r.b.y >> sh) & 0x0F0F0F0Fu, (r.b.z >> sh) & 0x0F0F0F0Fu,
                           (r.b.w >> sh) & 0x0F0F0F0Fu};
    uint32_t o[8];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        o[2 * k] = dq_fma(w[k], 0x04010400u, A, B);
        o[2 * k + 1] = dq_fma(w[k], 0x04030402u, A, B);
    }
    put16(tile, row, 2 * q, o[0], o[1], o[2], o[3]);
    put16(tile, row, 2 * q + 1, o[4], o[5], o[6], o[7]);
}

// Q6_K quarter q of step ks: group grp = 2(ks%2) + q/2, its values 16(q%2) .. +15; K columns
// 16q .. 16q+15 of the step (chunks 2q, 2q+1).
__device__ __forceinline__ void store_w_q6k(const RawW &r, int ks, int q, _Float16 *tile, int row) {
    const int grp = 2 * (ks & 1) + (q >> 1);
    const _Float16 sc = (_Float16)(h2f(r.dd) * (float)(int8_t)(r.s & 0xFF));
    const h2 S = {sc, sc};
    const h2 off = {(_Float16)-1056.0f, (_Float16)-1056.0f};
    const uint32_t ql[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
    const uint32_t qh[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
    const int shl = grp >= 2 ? 4 : 0;
    uint32_t o[8];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        // 6-bit q in bits 0..5 of each byte
        const uint32_t lo = (ql[k] >> shl) & 0x0F0F0F0Fu;
        const uint32_t hi = (2 * grp <= 4 ? (qh[k] << (4 - 2 * grp)) : (qh[k] >> (2 * grp - 4))) & 0x30303030u;
        const uint32_t v = lo | hi;
        o[2 * k] = __builtin_bit_cast(uint32_t, (magic_pair(v, 0x04010400u) + off) * S);
        o[2 * k + 1] = __builtin_bit_cast(uint32_t, (magic_pair(v, 0x04030402u) + off) * S);
    }
    put16(tile, row, 2 * q, o[0], o[1], o[2], o[3]);
    put16(tile, row, 2 * q + 1, o[4], o[5], o[6], o[7]);
}

// Quarter q: K columns 16q .. 16q+15 (chunks 2q, 2q+1) of the activation row.
__device__ __forceinline__ void store_a(const RawA<false> &r, int q, _Float16 *tile, int row, float) {
    put16(tile, row, 2 * q, r.a.x, r.a.y, r.a.z, r.a.w);
    put16(tile, row, 2 * q + 1, r.b.x, r.b.y, r.b.z, r.b.w);
}
// Raw Q8_1: d8 * 2^-e (exact) times q8, as the staging kernel computes it.
__device__ __forceinline__ void store_a(const RawA<true> &r, int q, _Float16 *tile, int row, float as) {
    const _Float16 d = (_Float16)(h2f(r.ds & 0xFFFF) * as);
    const h2 d2 = {d, d};
    const uint32_t w[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
    uint32_t o[8];
#pragma unroll
    for (int k = 0; k < 4; k++) q8x4_to_f16(w[k], d2, o[2 * k], o[2 * k + 1]);
    put16(tile, row, 2 * q, o[0], o[1], o[2], o[3]);
    put16(tile, row, 2 * q + 1, o[4], o[5], o[6], o[7]);
}

// ------------------------------------------------------------------ kernel
// Workgroup of 8 waves computes a 128 x 128 tile (weights x tokens) over one K slice
// (blockIdx.z of `splits`).  Wave w owns rows 64*(w%2) .. +63 and tokens 64*((w/2)%2) .. +63
// (4 x 4 MFMA tiles) and K half w/4 of every 64-wide step; the two K halves are summed
// through LDS at the end (fixed order).  Two waves per SIMD let one wave's conversion
// overlap the other's MFMAs.  Raw blocks are loaded into a ring of kPF register slots (the
// loop is unrolled by lcm(kPF, 3) so every ring index is static and the waits the
// compiler inserts count exactly the outstanding steps).  With splits > 1 the partial
// tiles are added into the (pre-zeroed) output with fp32 atomics, in an order that may
// differ from run to run.
constexpr int kThreads = 512;
constexpr int kBM = 128, kBN = 128;
// raw ring slots: loads run kPF-2 steps ahead of their conversion.  3 (one step of
// lookahead, the rest hidden by the three LDS buffers) measured faster than 4-6: the deeper
// rings cost registers (Q6_K: 246-256 VGPRs with spills at 5-6 against 202 at 3) for
// latency the other wave of the SIMD already hides (Q6_K 4096x1536x512: 34.1 -> 32.2 us,
// Q4_K 8192x4096x512: 65.5 -> 63.3 us, grouped MoE prefill -4 %)
constexpr int kPF = 3;
constexpr int kUnroll = 3;  // lcm(kPF, 3 LDS buffers)

// act: this thread's activation row is inside the tile's token count (rows past it are
// neither loaded nor converted; their LDS rows only feed output columns that are dropped).
template <int TYPE, bool Q8>
__device__ __forceinline__ void load_step(const uint8_t *wrow, const void *arow, int ks, int h, RawW &rw,
                                          RawA<Q8> &ra, bool act) {
    if (TYPE == kTypeQ4K) load_w_q4k(wrow, ks, h, rw);
    else load_w_q6k(wrow, ks, h, rw);
    if (act) load_a(arow, ks, h, ra);
}

template <int TYPE, bool Q8>
__device__ __forceinline__ void store_step(const RawW &rw, const RawA<Q8> &ra, int ks, int h, _Float16 *at,
                                           _Float16 *bt, int row, float as, bool act) {
    if (TYPE == kTypeQ4K) store_w_q4k(rw, ks, h, at, row);
    else store_w_q6k(rw, ks, h, at, row);
    if (act) store_a(ra, h, bt, row, as);
}

// Fragments of one 32-wide K half (kh) of a step for 4 x 4 MFMA 16x16x32 tiles.
// nb (wave-uniform): token tiles of the wave that hold tokens; the others are skipped.
__device__ __forceinline__ void read_frags(const _Float16 *as, const _Float16 *bs, int wi, int wj, int kh, int lane,
                                           h8 (&af)[4], h8 (&bf)[4], int nb) {
    const int chunk = 4 * kh + (lane >> 4);
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int ra = wi + 16 * t + (lane & 15), rb = wj + 16 * t + (lane & 15);
        af[t] = *(const h8 *)(as + tile_off(ra, chunk));
        if (t < nb) bf[t] = *(const h8 *)(bs + tile_off(rb, chunk));
    }
}
__device__ __forceinline__ void mfma_frags(const h8 (&af)[4], const h8 (&bf)[4], f4 (&acc)[4][4], int nb) {
#pragma unroll
    for (int b = 0; b < 4; b++) {
        if (b < nb) {
#pragma unroll
            for (int a = 0; a < 4; a++)
                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[a], bf[b], acc[a][b], 0, 0, 0);
        }
    }
}

// Epilogue / operand-addressing modes of the kernel:
//   kModePlain   : W [M][K], activations rows j = token, out[j*M + i] (column-major [N][M])
//   kModeSwiGLU  : grouped experts; a tile covers 64 features with 64 gate rows and 64 up
//                  rows interleaved; activation rows are tokens gathered through perm[];
//                  out[q*ld + f] = silu(gate) * up for expert-sorted row q
//   kModeGrouped : grouped experts; activation rows are the expert-sorted rows q themselves;
//                  out[q*ld + i]
enum GemmMode : int { kModePlain = 0, kModeSwiGLU = 1, kModeGrouped = 2 };

struct GemmArgs {
    const uint8_t *W;  // plain: weights; grouped: expert table base
    const void *A;           // activation rows: staged f16 (K values) or Q8_1 MMQ blocks
    const float *a_unscale;  // staged rows: 2^e per row
    float *out;
    int M, K, N, splits;
    int out_ld;
    // grouped modes
    size_t expert_stride, w_off, w_off2;  // expert e's matrix at W + e*stride + w_off (up: w_off2)
    const int *counts;                   // [n_experts] rows per expert
    const int *offsets;                  // [n_experts] first expert-sorted row
    const int *perm;                     // [rows] expert-sorted row -> token (SwiGLU gather)
    const int *tiles;                    // [max_tiles] (expert << 16) | n_tile; tiles[-1] = count
    int skip_upto;                       // grouped: tiles of at most this many rows are left to
                                         // the skinny kernel (0: none)
};

template <int TYPE, int MODE, bool ATOMIC, bool Q8>
__global__ void __launch_bounds__(kThreads) gemm_q8_1_kernel(GemmArgs g) {
    __shared__ __align__(16) _Float16 lds[3][2][kBM * kKS];  // [buffer][weights | tokens]
    const int tid = threadIdx.x;
    // the wave index as a scalar, so that every per-wave decision below is a scalar branch
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int K = g.K;
    const int wi = (wave & 1) * 64, wj = ((wave >> 1) & 1) * 64, kh = wave >> 2;
    const size_t wrow_bytes = (size_t)(K / 256) * (TYPE == kTypeQ4K ? kQ4KBytes : kQ6KBytes);
    const int nks_all = K / kKS;
    const int ks0 = (int)((long)nks_all * blockIdx.z / g.splits);
    const int ks1 = (int)((long)nks_all * (blockIdx.z + 1) / g.splits);
    const int last = ks1 - 1;

    // tile coordinates: weights i0 (features for SwiGLU), activation rows j0 .. j0+127 of
    // [row_base, row_base + n_rows)
    int i0, j0, n_rows, row_base = 0;
    const uint8_t *Wm = g.W, *Wm2 = g.W;
    if (MODE == kModePlain) {
        i0 = blockIdx.x * kBM;
        j0 = blockIdx.y * kBN;
        n_rows = g.N;
    } else {
        if ((int)blockIdx.y >= g.tiles[-1]) return;  // uniform: past the tile list
        const int t = g.tiles[blockIdx.y];
        const int e = t >> 16, nt = t & 0xFFFF;
        n_rows = g.counts[e];
        row_base = g.offsets[e];
        j0 = nt * kGroupTile;
        if (min(kGroupTile, n_rows - j0) <= g.skip_upto) return;  // uniform: a skinny tile
        i0 = blockIdx.x * (MODE == kModeSwiGLU ? kBM / 2 : kBM);
        Wm = g.W + (size_t)e * g.expert_stride + g.w_off;
        Wm2 = g.W + (size_t)e * g.expert_stride + g.w_off2;
    }

    // loader role: thread -> (LDS row lr, quarter lh); rows past the end re-read the last
    const int lr = tid >> 2, lh = tid & 3;
    const uint8_t *wrow;
    if (MODE == kModeSwiGLU) {
        // LDS rows 64w .. 64w+31 = gate features i0 + 32w + (0..31), 64w+32 .. = up features
        const int w = lr >> 6, rr = lr & 63;
        const int f = min(i0 + 32 * w + (rr & 31), g.M - 1);
        wrow = (rr < 32 ? Wm : Wm2) + (size_t)f * wrow_bytes;
    } else {
        wrow = Wm + (size_t)min(i0 + lr, g.M - 1) * wrow_bytes;
    }
    // tokens of this tile: activation rows past them are skipped, and so are the MFMAs of a
    // wave's 16-token tiles that hold none (the small experts of a grouped launch)
    // (grouped launches only: a plain GEMM's tiles are full but for the last)
    const int nvalid = min(kBN, n_rows - j0);
    const bool act = MODE == kModePlain || lr < nvalid;
    const int nb = MODE == kModePlain ? 4 : min(4, max(0, (nvalid - wj + 15) / 16));
    const int jr = min(j0 + lr, n_rows - 1);
    const int arow_idx = MODE == kModePlain ? jr : MODE == kModeSwiGLU ? g.perm[row_base + jr] : row_base + jr;
    __shared__ float row_unscale[kBN];
    float a_scale = 1.0f;
    const void *arow;
    if constexpr (Q8) {
        // f16 staging of d8*q8 overflows once |d8*q8| > 65504: scale the row by an exact
        // power of two 2^-e from its largest d8 (127 * max d8 * 2^-e <= 2^15) and undo it
        // in the epilogue (the staging kernels do the same for staged rows)
        const uint8_t *ar = (const uint8_t *)g.A + (size_t)arow_idx * (K / 128) * kQ81Bytes;
        arow = ar;
        float dmax = 0.0f;
        for (int b = lh; b < K / 128; b += 4) {
            const uint4 hd = ld16(ar + (size_t)b * kQ81Bytes);
            dmax = fmaxf(dmax, fmaxf(fmaxf(fabsf(h2f(hd.x & 0xFFFF)), fabsf(h2f(hd.y & 0xFFFF))),
                                     fmaxf(fabsf(h2f(hd.z & 0xFFFF)), fabsf(h2f(hd.w & 0xFFFF)))));
        }
        dmax = fmaxf(dmax, __shfl_xor(dmax, 1));
        dmax = fmaxf(dmax, __shfl_xor(dmax, 2));
        const int e = row_exponent(dmax);
        a_scale = ldexpf(1.0f, -e);
        if (lh == 0) row_unscale[lr] = ldexpf(1.0f, e);
    } else {
        arow = (const _Float16 *)g.A + (size_t)arow_idx * K;
        if (lh == 0) row_unscale[lr] = g.a_unscale[arow_idx];
    }

    f4 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};

    // Pipeline: three LDS tile buffers.  In step ks a wave multiplies the fragments of step
    // ks (read during step ks-1), reads the fragments of step ks+1 (its tile was completed
    // before the previous barrier), converts step ks+2 into the third buffer, then meets
    // the barrier.  Raw blocks sit in a ring of kPF register slots, loaded kPF-2 steps
    // before their conversion.  The loop is unrolled by lcm(kPF, 3) so all indices are static.
    RawW rw[kPF];
    RawA<Q8> ra[kPF];
#pragma unroll
    for (int p = 0; p < kPF; p++) load_step<TYPE, Q8>(wrow, arow, min(ks0 + p, last), lh, rw[p], ra[p], act);
    store_step<TYPE, Q8>(rw[0], ra[0], ks0, lh, lds[0][0], lds[0][1], lr, a_scale, act);
    store_step<TYPE, Q8>(rw[1], ra[1], ks0 + 1, lh, lds[1][0], lds[1][1], lr, a_scale, act);
    __syncthreads();
    h8 af[4], bf[4];
    read_frags(lds[0][0], lds[0][1], wi, wj, kh, lane, af, bf, nb);

    for (int kb = ks0; kb < ks1; kb += kUnroll) {
#pragma unroll
        for (int p = 0; p < kUnroll; p++) {
            const int ks = kb + p;
            if (ks < ks1) {  // uniform
                // kb - ks0 is a multiple of kUnroll, so these are compile-time constants
                const int r = p % kPF, b = p % 3;
                load_step<TYPE, Q8>(wrow, arow, min(ks + kPF, last), lh, rw[r], ra[r], act);
                mfma_frags(af, bf, acc, nb);
                // (past the end these read and fill idle buffers with data nobody uses)
                read_frags(lds[(b + 1) % 3][0], lds[(b + 1) % 3][1], wi, wj, kh, lane, af, bf, nb);
                store_step<TYPE, Q8>(rw[(r + 2) % kPF], ra[(r + 2) % kPF], ks + 2, lh, lds[(b + 2) % 3][0],
                                     lds[(b + 2) % 3][1], lr, a_scale, act);
                __syncthreads();
            }
        }
    }
    // sum the two K halves: waves 4..7 hand their tiles to waves 0..3 through the (now idle)
    // tile buffers, laid out lane-minor so the accesses are conflict-free
    __syncthreads();
    float *red = (float *)&lds[0][0][0] + (size_t)(wave & 3) * (64 * 64);
    if (kh) {
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int b = 0; b < 4; b++)
#pragma unroll
                for (int e = 0; e < 4; e++) red[((a * 4 + b) * 4 + e) * 64 + lane] = acc[a][b][e];
    }
    __syncthreads();
    if (kh) return;
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[a][b][e] += red[((a * 4 + b) * 4 + e) * 64 + lane];
    // D layout (16x16 f32): lane l holds rows 4*(l/16)+e, column l%16.  Rows index
    // weights (A operand), columns activation rows (B operand).
    if (MODE == kModeSwiGLU) {
        // gate tile a pairs with up tile a+2: feature i0 + 32*(wave&1) + 16a + 4*(l/16) + e
#pragma unroll
        for (int a = 0; a < 2; a++)
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const int j = j0 + wj + 16 * b + (lane & 15);
                const int f = i0 + 32 * (wave & 1) + 16 * a + 4 * (lane >> 4);
                if (j >= n_rows) continue;
                const float us = row_unscale[wj + 16 * b + (lane & 15)];
                float *o = g.out + (size_t)(row_base + j) * g.out_ld + f;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float gt = acc[a][b][e] * us, up = acc[a + 2][b][e] * us;
                    if (f + e < g.M) o[e] = gt / (1.0f + expf(-gt)) * up;
                }
            }
        return;
    }
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int j = j0 + wj + 16 * b + (lane & 15);
            const int ib = i0 + wi + 16 * a + 4 * (lane >> 4);
            if (j >= n_rows) continue;
            const float us = row_unscale[wj + 16 * b + (lane & 15)];
#pragma unroll
            for (int e = 0; e < 4; e++) acc[a][b][e] *= us;
            float *o = g.out + (size_t)(row_base + j) * g.out_ld + ib;
            if (ATOMIC) {
                // to the wave's own (idle) reduction buffer, token-major, 16-byte groups
                // XOR-swizzled by token so that the row-wise reads below are conflict-free
                *(f4 *)(red + (16 * b + (lane & 15)) * 64 + (((4 * a + (lane >> 4)) ^ (lane & 15)) << 2)) = acc[a][b];
            } else if (ib + 3 < g.M && ((g.out_ld & 3) == 0)) {
                *(f4 *)o = acc[a][b];
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (ib + e < g.M) o[e] = acc[a][b][e];
            }
        }
    if (ATOMIC) {
        // one atomic instruction per token covers 64 consecutive outputs (two cache lines);
        // the MFMA layout would spread each instruction over 16 token rows, which measured
        // twice as slow in the L2 atomic units
        const int ib = i0 + wi + lane;
        for (int t = 0; t < 64; t++) {
            const int j = j0 + wj + t;
            if (j >= n_rows) break;
            if (ib < g.M)
                __hip_atomic_fetch_add(g.out + (size_t)(row_base + j) * g.out_ld + ib,
                                       red[t * 64 + ((((lane >> 2) ^ (t & 15)) << 2) | (lane & 3))], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ------------------------------------------------------------------ activation staging
// One wave per activation row, 4 rows per 256-thread block.
constexpr int kStageThreads = 256;

// Q8_1 MMQ rows [N][K/128] x 144 B -> f16 rows d8*q8*2^-e, unscale[row] = 2^e.
__global__ void __launch_bounds__(kStageThreads) stage_q8_1_kernel(const uint8_t *__restrict__ A, int K, int N,
                                                                   _Float16 *__restrict__ out,
                                                                   float *__restrict__ unscale) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (kStageThreads / 64) + (threadIdx.x >> 6);
    if (row >= N) return;
    const uint8_t *ar = A + (size_t)row * (K / 128) * kQ81Bytes;
    float dmax = 0.0f;
    for (int b = lane; b < K / 128; b += 64) {
        const uint4 hd = ld16(ar + (size_t)b * kQ81Bytes);
        dmax = fmaxf(dmax, fmaxf(fmaxf(fabsf(h2f(hd.x & 0xFFFF)), fabsf(h2f(hd.y & 0xFFFF))),
                                 fmaxf(fabsf(h2f(hd.z & 0xFFFF)), fabsf(h2f(hd.w & 0xFFFF)))));
    }
    const int e = row_exponent(wave_max(dmax));
    const float as = ldexpf(1.0f, -e);
    if (lane == 0) unscale[row] = ldexpf(1.0f, e);
    _Float16 *orow = out + (size_t)row * K;
    for (int c = lane; c < K / 16; c += 64) {  // 16 values per chunk
        const uint8_t *blk = ar + (size_t)(c >> 3) * kQ81Bytes;
        uint16_t dbits;
        __builtin_memcpy(&dbits, blk + 4 * ((c & 7) >> 1), 2);
        const _Float16 d = (_Float16)(h2f(dbits) * as);  // exact: power-of-two scaling
        const h2 d2 = {d, d};
        const uint4 q = ld16(blk + 16 + 16 * (c & 7));
        uint4 o0, o1;
        q8x4_to_f16(q.x, d2, o0.x, o0.y);
        q8x4_to_f16(q.y, d2, o0.z, o0.w);
        q8x4_to_f16(q.z, d2, o1.x, o1.y);
        q8x4_to_f16(q.w, d2, o1.z, o1.w);
        *(uint4 *)(orow + 16 * c) = o0;
        *(uint4 *)(orow + 16 * c + 8) = o1;
    }
}

// fp32 rows [N][K] -> the same staged form as stage_q8_1_kernel applied to
// cuda_quantize_mmq_q8_1's output: per 32 values d = f16(amax/127), q = rint(x*127/amax)
// clamped to +-127 (gemm_q4k.cu:327-358), staged value f16(d*2^-e) * q.
__global__ void __launch_bounds__(kStageThreads) stage_f32_kernel(const float *__restrict__ x, int K, int N,
                                                                  _Float16 *__restrict__ out,
                                                                  float *__restrict__ unscale) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (kStageThreads / 64) + (threadIdx.x >> 6);
    if (row >= N) return;
    const float4 *xr = (const float4 *)(x + (size_t)row * K);
    float dmax = 0.0f;
    for (int b = lane; b < K / 32; b += 64) {
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 v = xr[8 * b + i];
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
        float d = amax / 127.0f;
        asm volatile("" : "+v"(d));  // round d to fp32 before the f16 conversion
        dmax = fmaxf(dmax, (float)(_Float16)d);
    }
    const int e = row_exponent(wave_max(dmax));
    const float as = ldexpf(1.0f, -e);
    if (lane == 0) unscale[row] = ldexpf(1.0f, e);
    _Float16 *orow = out + (size_t)row * K;
    for (int b = lane; b < K / 32; b += 64) {
        float xv[32];
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 v = xr[8 * b + i];
            xv[4 * i] = v.x; xv[4 * i + 1] = v.y; xv[4 * i + 2] = v.z; xv[4 * i + 3] = v.w;
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
        float d = amax / 127.0f;
        asm volatile("" : "+v"(d));
        const float id = amax > 0.0f ? 127.0f / amax : 0.0f;
        const _Float16 ds = (_Float16)((float)(_Float16)d * as);
        uint32_t o[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float r0 = fminf(fmaxf(rintf(xv[2 * i] * id), -127.0f), 127.0f);
            const float r1 = fminf(fmaxf(rintf(xv[2 * i + 1] * id), -127.0f), 127.0f);
            const h2 q = {(_Float16)r0, (_Float16)r1};
            const h2 d2 = {ds, ds};
            o[i] = __builtin_bit_cast(uint32_t, q * d2);
        }
        uint4 *dst = (uint4 *)(orow + 32 * b);
#pragma unroll
        for (int i = 0; i < 4; i++) dst[i] = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
    }
}

int launch_stage_q8_1(const void *act, int K, int N, _Float16 *out, float *unscale, hipStream_t s) {
    hipLaunchKernelGGL(stage_q8_1_kernel, dim3((N + 3) / 4), dim3(kStageThreads), 0, s, (const uint8_t *)act, K, N,
                       out, unscale);
    return check_launch("stage_q8_1");
}

int launch_stage_f32(const float *x, int K, int N, _Float16 *out, float *unscale, hipStream_t s) {
    hipLaunchKernelGGL(stage_f32_kernel, dim3((N + 3) / 4), dim3(kStageThreads), 0, s, x, K, N, out, unscale);
    return check_launch("stage_f32");
}

__global__ void zero_kernel(float4 *__restrict__ p, long n4) {
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n4; i += (long)gridDim.x * blockDim.x)
        p[i] = make_float4(0.f, 0.f, 0.f, 0.f);
}

static int device_cus_gemm() {
    static int cus = 0;
    if (!cus) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            cus = n;
        else
            cus = 256;
    }
    return cus;
}

template <int MODE, bool Q8>
static void launch_mode(int type, bool atomic, dim3 grid, const GemmArgs &g, hipStream_t stream) {
#define MNEMO_GEMM_LAUNCH(T_, A_) \
    hipLaunchKernelGGL((gemm_q8_1_kernel<T_, MODE, A_, Q8>), grid, dim3(kThreads), 0, stream, g)
    if (type == kTypeQ4K) {
        if (atomic) MNEMO_GEMM_LAUNCH(kTypeQ4K, true);
        else MNEMO_GEMM_LAUNCH(kTypeQ4K, false);
    } else {
        if (atomic) MNEMO_GEMM_LAUNCH(kTypeQ6K, true);
        else MNEMO_GEMM_LAUNCH(kTypeQ6K, false);
    }
#undef MNEMO_GEMM_LAUNCH
}

int launch_gemm_q8_1(int type, const void *w, const void *act, float *out, int M, int K, int N,
                     hipStream_t stream) {
    if (!w || !act || !out || M <= 0 || N <= 0 || K <= 0 || K % 256 != 0)
        return set_error(kErrBadArg, "gemm: need non-null pointers, M, N > 0 and K %% 256 == 0");
    if (type != kTypeQ4K && type != kTypeQ6K) return set_error(kErrUnsupportedType, "gemm: unsupported type %d", type);
    if (((uintptr_t)out & 15) != 0) return set_error(kErrBadArg, "gemm: output must be 16-byte aligned");
    if (((uintptr_t)act & 3) != 0) return set_error(kErrBadArg, "gemm: activation blocks must be 4-byte aligned");
    const int tm = (M + kBM - 1) / kBM, tn = (N + kBN - 1) / kBN;
    // split K while the split grid still fits the CUs once (one workgroup per CU at a time),
    // keeping at least 8 steps of 64 per split: measured, M x 512 x K = 1536 x 4096 best at 4
    // splits (31 us against 59 unsplit), 512 x 4096 at 8, 4096 x 8192 at 2 (75 against 100)
    const int nks = K / kKS;
    int splits = 1;
    while (2 * tm * tn * splits <= device_cus_gemm() && nks / (splits * 2) >= 8) splits *= 2;
    if (((long)M * N) % 4 != 0) splits = 1;  // the fill kernel clears float4s
    // activations are read as Q8_1 blocks and converted per tile: nothing is allocated, so
    // the call may sit inside a graph capture
    GemmArgs g{};
    g.W = (const uint8_t *)w;
    g.A = act;
    g.out = out;
    g.M = M;
    g.K = K;
    g.N = N;
    g.splits = splits;
    g.out_ld = M;
    if (splits > 1) {
        const long n = (long)M * N;
        hipLaunchKernelGGL(zero_kernel, dim3((unsigned)std::min<long>((n / 4 + 255) / 256, 4096)), dim3(256), 0,
                           stream, (float4 *)out, n / 4);
    }
    launch_mode<kModePlain, true>(type, splits > 1, dim3(tm, tn, splits), g, stream);
    return check_launch("gemm_q8_1");
}

// ------------------------------------------------------------------ skinny grouped kernel
// Most token tiles of a grouped launch hold few rows (an expert of the MoE prefill receives
// a few tens of tokens), and then the tiled kernel above spends its time converting 128
// weight rows per step into LDS for a handful of MFMA columns.  This kernel serves the
// tiles of at most kSkTok rows without staging weights at all: every lane loads the raw
// bytes of its own A-operand values and converts them in registers, straight into the
// 16x16x32 f16 MFMA.  The K order inside an MFMA is free as long as both operands follow
// it, so each lane takes whole 16-byte chunks of a super-block (lane group q = lane/16,
// MFMA t = 0..7 of a 256-value block):
//   Q4_K: qs chunk m = q + 4(t/4): values 64(m/2) + 32h + 16(m%2) + 8s .. +7, with h = (t/2)%2
//         the nibble (sub-block 2(m/2) + h) and s = t%2 the dword pair of the chunk;
//   Q6_K: half H = t/4, ql chunk 64H + 16q, qh chunk 32H + 16(q%2), nibble n = (t/2)%2:
//         group grp = q/2 + 2n, values 128H + 32grp + 16(q%2) + 8s .. +7, scale 8H + q + 4n.
// The tile's activation rows (staged f16) are copied per block into LDS in that order, so
// a B fragment is one 16-byte read.  Conversion arithmetic is the tiled kernel's (same f16
// roundings), so the two kernels agree to the fp32 accumulation order.
#ifndef MNEMO_SKTOK
#define MNEMO_SKTOK 64
#endif
#ifndef MNEMO_SK_THREADS
#define MNEMO_SK_THREADS 512
#endif
constexpr int kSkThreads = MNEMO_SK_THREADS;  // 8 waves
constexpr int kSkStage = kSkThreads / 32;        // activation rows staged per pass
constexpr int kSkWaves = kSkThreads / 64;
constexpr int kSkTok = MNEMO_SKTOK;       // rows per tile served here: 4 column tiles of 16
// weight rows per wave: SwiGLU one gate and one up tile of 16 (same features); grouped
#ifndef MNEMO_SK_RPLAIN
#define MNEMO_SK_RPLAIN 2
#endif
template <int MODE>
constexpr int sk_rows_per_wave() { return MODE == kModeSwiGLU ? 32 : 16 * MNEMO_SK_RPLAIN; }
template <int TYPE>
__device__ __forceinline__ int sk_k0(int t, int q) {
    if (TYPE == kTypeQ4K) {
        const int m = q + 4 * (t >> 2);
        return 64 * (m >> 1) + 32 * ((t >> 1) & 1) + 16 * (m & 1) + 8 * (t & 1);
    }
    return 128 * (t >> 2) + 32 * ((q >> 1) + 2 * ((t >> 1) & 1)) + 16 * (q & 1) + 8 * (t & 1);
}

// raw bytes of one row tile's lane values for one 256-value block
struct SkRaw {
    uint4 c[2];   // Q4_K: qs chunks q, q+4;  Q6_K: ql chunks of halves 0, 1
    uint4 h;      // Q4_K: the header (d, dmin, 12 scale bytes);  Q6_K: the lane's qh bits,
                  // two dwords per half (below)
    uint32_t sc;  // Q6_K: scale bytes q, q+4, q+8, q+12
    uint32_t d;   // Q6_K: f16 d
};

template <int TYPE>
__device__ __forceinline__ void sk_load(const uint8_t *__restrict__ blk, int q, SkRaw &r) {
    if (TYPE == kTypeQ4K) {
        r.h = ld16(blk);
        r.c[0] = ld16(blk + 16 + 16 * q);
        r.c[1] = ld16(blk + 80 + 16 * q);
    } else {
        r.c[0] = ld16_a2(blk + 16 * q);
        r.c[1] = ld16_a2(blk + 64 + 16 * q);
        const uint4 h0 = ld16_a2(blk + 128 + 16 * (q & 1)), h1 = ld16_a2(blk + 160 + 16 * (q & 1));
        const uint4 sc = ld16_a2(blk + 192);
        uint16_t dd;
        __builtin_memcpy(&dd, blk + 208, 2);
        r.d = dd;
        // scale byte i of the lane is byte q of dword i
        const uint32_t lo = __builtin_amdgcn_perm(sc.y, sc.x, 0x0C0C0400u + 0x00000101u * (uint32_t)q);
        const uint32_t hi = __builtin_amdgcn_perm(sc.w, sc.z, 0x0C0C0400u + 0x00000101u * (uint32_t)q);
        r.sc = (lo & 0xFFFFu) | (hi << 16);
        // of each qh byte the lane needs groups q/2 (bits 2(q/2)..+1) and q/2 + 2 (bits
        // 2(q/2)+4..+5); packed: byte i of dword 2H+s holds, for values i (dword 2s) and
        // 4+i (dword 2s+1) of the chunk, bits 0-1 / 2-3 (low nibble group) and 4-5 / 6-7
        const int sh = 2 * (q >> 1);
        auto pk = [sh](uint32_t a, uint32_t b) {
            return ((a >> sh) & 0x33333333u) | (((b >> sh) & 0x33333333u) << 2);
        };
        r.h = make_uint4(pk(h0.x, h0.y), pk(h0.z, h0.w), pk(h1.x, h1.y), pk(h1.z, h1.w));
    }
}

__device__ __forceinline__ uint32_t dw(const uint4 &v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

// per-block scale pairs of a lane: Q4_K (d*sc, -dmin*m) of its 4 sub-blocks (index 2L + h);
// Q6_K d*sc of its 4 scales (index 2H + n)
template <int TYPE>
__device__ __forceinline__ void sk_scales(const SkRaw &r, int q, h2 (&A)[4], h2 (&B)[4]) {
    if (TYPE == kTypeQ4K) {
        const uint32_t s0 = r.h.y, s1 = r.h.z, s2 = r.h.w;
        const float d = h2f(r.h.x & 0xFFFFu), dmin = h2f(r.h.x >> 16);
#pragma unroll
        for (int L = 0; L < 2; L++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int j = 2 * ((q >> 1) + 2 * L) + h;  // get_scale_min_k4 (kernels.cu:45-53)
                uint32_t sc, m;
                if (L == 0) {
                    sc = sbyte(s0, s1, s2, j) & 63;
                    m = sbyte(s0, s1, s2, j + 4) & 63;
                } else {
                    sc = (sbyte(s0, s1, s2, j + 4) & 15) | ((sbyte(s0, s1, s2, j - 4) >> 6) << 4);
                    m = (sbyte(s0, s1, s2, j + 4) >> 4) | ((sbyte(s0, s1, s2, j) >> 6) << 4);
                }
                const _Float16 a = (_Float16)(d * (float)sc), b = (_Float16)(-dmin * (float)m);
                A[2 * L + h] = h2{a, a};
                B[2 * L + h] = h2{b, b};
            }
    } else {
        const float d = h2f(r.d);
#pragma unroll
        for (int H = 0; H < 2; H++)
#pragma unroll
            for (int n = 0; n < 2; n++) {  // scale 8H + q + 4n = lane byte 2H + n
                const int8_t sc = (int8_t)((r.sc >> (8 * (2 * H + n))) & 0xFF);
                const _Float16 a = (_Float16)(d * (float)sc);
                A[2 * H + n] = h2{a, a};
            }
    }
}

// the 8 f16 A-operand values of MFMA t
template <int TYPE>
__device__ __forceinline__ h8 sk_operand(const SkRaw &r, int t, const h2 (&A)[4], const h2 (&B)[4]) {
    const int L = t >> 2, h = (t >> 1) & 1, s = t & 1;
    uint32_t o[4];
    if (TYPE == kTypeQ4K) {
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const uint32_t w = (dw(r.c[L], 2 * s + k) >> (4 * h)) & 0x0F0F0F0Fu;
            o[2 * k] = dq_fma(w, 0x04010400u, A[2 * L + h], B[2 * L + h]);
            o[2 * k + 1] = dq_fma(w, 0x04030402u, A[2 * L + h], B[2 * L + h]);
        }
    } else {
        const h2 off = {(_Float16)-1056.0f, (_Float16)-1056.0f};
        const uint32_t P = dw(r.h, 2 * L + s);
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const uint32_t lo = (dw(r.c[L], 2 * s + k) >> (4 * h)) & 0x0F0F0F0Fu;
            const int sh = 2 * k + 4 * h;  // the two bits of these values, moved to bits 4-5
            const uint32_t hi = (sh <= 4 ? (P << (4 - sh)) : (P >> (sh - 4))) & 0x30303030u;
            const uint32_t v = lo | hi;
            o[2 * k] = __builtin_bit_cast(uint32_t, (magic_pair(v, 0x04010400u) + off) * A[2 * L + h]);
            o[2 * k + 1] = __builtin_bit_cast(uint32_t, (magic_pair(v, 0x04030402u) + off) * A[2 * L + h]);
        }
    }
    const uint4 u = make_uint4(o[0], o[1], o[2], o[3]);
    return __builtin_bit_cast(h8, u);
}

// B slot u = 4t + q of token row r, 16-byte columns XOR-swizzled by the row so that the
// 16 rows of a fragment read hit distinct banks
__device__ __forceinline__ int sk_slot(int r, int u) { return r * 256 + ((u ^ (r & 31)) << 3); }

// One 256-value block: multiply block k (raw weights in `cur`, activations in LDS buffer
// k%2) while the weights of block k+1 load into `nxt` and its activations into the other
// LDS buffer (straight from memory, global_load_lds: lane l of a wave fills 16 bytes at
// base + 16l).  The wait for those LDS writes before the barrier also covers the weight
// loads issued after them (memory loads complete in issue order), so one block ahead is
// what the pipeline can hold.
template <int TYPE, int NB, int R>
__device__ __forceinline__ void sk_block(int k, int nkb, int bbytes, int q, int c, int wave, const uint8_t *const (&wrow)[R],
                                         const _Float16 *const (&arow)[NB * 16 / kSkStage], _Float16 (*bs)[kSkTok * 256],
                                         const SkRaw (&cur)[R], SkRaw (&nxt)[R], f4 (&acc)[R][NB]) {
    // past the end the last block is loaded again (into the idle buffer and registers)
    const int kn = min(k + 1, nkb - 1);
#pragma unroll
    for (int i = 0; i < NB * 16 / kSkStage; i++)
        __builtin_amdgcn_global_load_lds((const void *)(arow[i] + kn * 256),
                                         (__attribute__((address_space(3))) void *)&bs[(k + 1) & 1][(2 * wave + kSkStage * i) * 256],
                                         16, 0, 0);
#pragma unroll
    for (int a = 0; a < R; a++) sk_load<TYPE>(wrow[a] + (size_t)kn * bbytes, q, nxt[a]);
    // keep the loads here, ahead of the multiplication (the scheduler would otherwise sink
    // them past it to save registers, and nothing would be in flight during the MFMAs)
    __builtin_amdgcn_sched_barrier(0);
    h2 A[R][4], B[R][4];
#pragma unroll
    for (int a = 0; a < R; a++) sk_scales<TYPE>(cur[a], q, A[a], B[a]);
    const _Float16 *bb = bs[k & 1];
#pragma unroll
    for (int t = 0; t < 8; t++) {
        h8 bf[NB];
#pragma unroll
        for (int b = 0; b < NB; b++) bf[b] = *(const h8 *)(bb + sk_slot(16 * b + c, 4 * t + q));
#pragma unroll
        for (int a = 0; a < R; a++) {
            const h8 af = sk_operand<TYPE>(cur[a], t, A[a], B[a]);
#pragma unroll
            for (int b = 0; b < NB; b++) acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[b], acc[a][b], 0, 0, 0);
        }
    }
    __syncthreads();
}

template <int TYPE, int MODE, int NB>
__device__ __forceinline__ void sk_tile(const GemmArgs &g, _Float16 (*bs)[kSkTok * 256], int wave, int lane, int tid,
                                        int e, int j0, int n_rows, int row_base) {
    constexpr int R = sk_rows_per_wave<MODE>() / 16;
    constexpr int H = R / 2;  // SwiGLU: gate tiles 0 .. H-1, up tiles H .. 2H-1
    const int q = lane >> 4, c = lane & 15;
    const int K = g.K, nkb = K / 256;
    const int bbytes = TYPE == kTypeQ4K ? kQ4KBytes : kQ6KBytes;
    const size_t wrow_bytes = (size_t)nkb * bbytes;
    const uint8_t *Wm = g.W + (size_t)e * g.expert_stride + g.w_off;
    const uint8_t *Wm2 = g.W + (size_t)e * g.expert_stride + g.w_off2;

    // this lane's weight row of each row tile (rows past M re-read the last)
    const uint8_t *wrow[R];
    int base;  // SwiGLU: first feature of the wave; grouped: first row
    if (MODE == kModeSwiGLU) {
        base = (blockIdx.x * kSkWaves + wave) * (16 * H);
#pragma unroll
        for (int a = 0; a < R; a++) {
            const int f = min(base + 16 * (a % H) + c, g.M - 1);
            wrow[a] = (a < H ? Wm : Wm2) + (size_t)f * wrow_bytes;
        }
    } else {
        base = (blockIdx.x * kSkWaves + wave) * (16 * R);
#pragma unroll
        for (int a = 0; a < R; a++) wrow[a] = Wm + (size_t)min(base + 16 * a + c, g.M - 1) * wrow_bytes;
    }
    // activation staging role: physical slot tid % 32 of rows r = tid/32 + kSkStage i, which
    // holds the logical slot (tid % 32) ^ (r % 32)
    const int sr0 = tid >> 5;
    const _Float16 *arow[NB * 16 / kSkStage];
#pragma unroll
    for (int i = 0; i < NB * 16 / kSkStage; i++) {
        const int r = sr0 + kSkStage * i, u = (tid & 31) ^ (r & 31);
        const int j = min(j0 + r, n_rows - 1);
        const int idx = MODE == kModeSwiGLU ? g.perm[row_base + j] : row_base + j;
        arow[i] = (const _Float16 *)g.A + (size_t)idx * K + sk_k0<TYPE>(u >> 2, u & 3);
    }
    f4 acc[R][NB];
#pragma unroll
    for (int a = 0; a < R; a++)
#pragma unroll
        for (int b = 0; b < NB; b++) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};
    SkRaw r0[R], r1[R];
#pragma unroll
    for (int i = 0; i < NB * 16 / kSkStage; i++)
        __builtin_amdgcn_global_load_lds((const void *)arow[i],
                                         (__attribute__((address_space(3))) void *)&bs[0][(2 * wave + kSkStage * i) * 256],
                                         16, 0, 0);
#pragma unroll
    for (int a = 0; a < R; a++) sk_load<TYPE>(wrow[a], q, r0[a]);
    __syncthreads();
    // two raw slots, the loop unrolled by two so that both are static
    for (int k = 0; k < nkb; k += 2) {
        sk_block<TYPE, NB, R>(k, nkb, bbytes, q, c, wave, wrow, arow, bs, r0, r1, acc);
        if (k + 1 >= nkb) break;
        sk_block<TYPE, NB, R>(k + 1, nkb, bbytes, q, c, wave, wrow, arow, bs, r1, r0, acc);
    }

    // D layout: lane holds weight rows 4q + e of each 16-row tile, token column c
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const int j = j0 + 16 * b + c;
        if (j >= n_rows) continue;
        const int idx = MODE == kModeSwiGLU ? g.perm[row_base + j] : row_base + j;
        const float us = g.a_unscale[idx];
        float *orow = g.out + (size_t)(row_base + j) * g.out_ld;
        if (MODE == kModeSwiGLU) {
#pragma unroll
            for (int a = 0; a < H; a++) {
                const int f = base + 16 * a + 4 * q;
#pragma unroll
                for (int x = 0; x < 4; x++) {
                    const float gt = acc[a][b][x] * us, up = acc[a + H][b][x] * us;
                    if (f + x < g.M) orow[f + x] = gt / (1.0f + expf(-gt)) * up;
                }
            }
        } else {
#pragma unroll
            for (int a = 0; a < R; a++) {
                const int i = base + 16 * a + 4 * q;
#pragma unroll
                for (int x = 0; x < 4; x++)
                    if (i + x < g.M) orow[i + x] = acc[a][b][x] * us;
            }
        }
    }
}

template <int TYPE, int MODE>
__global__ void __launch_bounds__(kSkThreads) gemm_skinny_kernel(GemmArgs g) {
    __shared__ __align__(16) _Float16 bs[2][kSkTok * 256];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    if ((int)blockIdx.y >= g.tiles[-1]) return;
    const int tl = g.tiles[blockIdx.y];
    const int e = tl >> 16, nt = tl & 0xFFFF;
    const int n_rows = g.counts[e], row_base = g.offsets[e], j0 = nt * kGroupTile;
    const int nvalid = min(kGroupTile, n_rows - j0);
    if (nvalid > kSkTok) return;  // uniform: the tiled kernel's tile
    // one instantiation per count of 16-row column tiles, so every MFMA is unconditional
    switch ((nvalid + 15) >> 4) {
    case 1: sk_tile<TYPE, MODE, 1>(g, bs, wave, lane, tid, e, j0, n_rows, row_base); break;
    case 2: sk_tile<TYPE, MODE, 2>(g, bs, wave, lane, tid, e, j0, n_rows, row_base); break;
    case 3: sk_tile<TYPE, MODE, 3>(g, bs, wave, lane, tid, e, j0, n_rows, row_base); break;
    case 4: sk_tile<TYPE, MODE, 4>(g, bs, wave, lane, tid, e, j0, n_rows, row_base); break;
#if MNEMO_SKTOK == 128
    case 5: sk_tile<TYPE, MODE, 5>(g, bs, wave, lane, tid, e, j0, n_rows, row_base); break;
    case 6: sk_tile<TYPE, MODE, 6>(g, bs, wave, lane, tid, e, j0, n_rows, row_base); break;
    case 7: sk_tile<TYPE, MODE, 7>(g, bs, wave, lane, tid, e, j0, n_rows, row_base); break;
    default: sk_tile<TYPE, MODE, 8>(g, bs, wave, lane, tid, e, j0, n_rows, row_base); break;
#endif
    }
}

// Grouped launches used by the MoE prefill path (moe.hip): tiles[] and the routing arrays
// live in device memory, the grid covers max_tiles tile-list entries.
int launch_gemm_grouped(int type, int swiglu, const void *experts, size_t expert_stride, size_t w_off,
                        size_t w_off2, const _Float16 *act, const float *act_unscale, const int *counts, const int *offsets, const int *perm,
                        const int *tiles, int max_tiles, float *out, int out_ld, int M, int K,
                        hipStream_t stream) {
    GemmArgs g{};
    g.W = (const uint8_t *)experts;
    g.A = act;
    g.a_unscale = act_unscale;
    g.out = out;
    g.M = M;
    g.K = K;
    g.N = 0;
    g.splits = 1;
    g.out_ld = out_ld;
    g.expert_stride = expert_stride;
    g.w_off = w_off;
    g.w_off2 = w_off2;
    g.counts = counts;
    g.offsets = offsets;
    g.perm = perm;
    g.tiles = tiles;
    g.skip_upto = kSkTok;
    // tiles of at most kSkTok rows: the skinny kernel; the rest: the tiled kernel
    const int sk_rows = swiglu ? sk_rows_per_wave<kModeSwiGLU>() / 2 * kSkWaves : sk_rows_per_wave<kModeGrouped>() * kSkWaves;
    const dim3 sk_grid((M + sk_rows - 1) / sk_rows, max_tiles, 1);
#define MNEMO_SKINNY(T_, M_) hipLaunchKernelGGL((gemm_skinny_kernel<T_, M_>), sk_grid, dim3(kSkThreads), 0, stream, g)
    if (swiglu) {
        if (type == kTypeQ4K) MNEMO_SKINNY(kTypeQ4K, kModeSwiGLU);
        else MNEMO_SKINNY(kTypeQ6K, kModeSwiGLU);
    } else {
        if (type == kTypeQ4K) MNEMO_SKINNY(kTypeQ4K, kModeGrouped);
        else MNEMO_SKINNY(kTypeQ6K, kModeGrouped);
    }
#undef MNEMO_SKINNY
    if (kGroupTile <= kSkTok) return check_launch("gemm_grouped");  // no tile is left
    if (swiglu) launch_mode<kModeSwiGLU, false>(type, false, dim3((M + kBM / 2 - 1) / (kBM / 2), max_tiles, 1), g, stream);
    else launch_mode<kModeGrouped, false>(type, false, dim3((M + kBM - 1) / kBM, max_tiles, 1), g, stream);
    return check_launch("gemm_grouped");
}

}  // namespace mnemo
