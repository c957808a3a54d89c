// gemm.hip -- Q4_K / Q6_K x Q8_1 GEMM for prefill and batched experts (gfx950 MFMA).
//
// Semantics (MnemoCUDA gemm_q4k.cu:103-112, 164-166, 194), per 32-value sub-block s:
//   Q4_K: out[j*M + i] = sum_s (d*sc_s)_i * d8_js * (sum_{k in s} q_ik * q8_jk) - (dmin*m_s)_i * ds_js
//   Q6_K: out[j*M + i] = sum_s d_i * d8_js * (sum over the two 16-value groups g of s of
//                                            sc_g * sum_{k in g} (q_ik - 32) * q8_jk)
// with W GGUF blocks [M][K], the activations Q8_1 MMQ blocks [N][K/128] x 144 B
// (half2 (d8, ds) per 32 values, ds = d8 * sum of the unquantized values), and the output
// column-major [N][M].  The scales d*sc and dmin*m are exact in fp32 (the reference rounds
// them to f16 in registers, gemm_q4k.cu:106-111; this build keeps the GEMV's fp32
// dequantisation, kernels.cu:114-136).
//
// Exact integer sub-block sums on f16 matrix cores.
//   * Operands are integers that f16 holds exactly: A = sc * q (Q4_K, <= 63 * 15 = 945) and
//     B = q8 (|q8| <= 127).  A 16x16x32 f16 MFMA over one sub-block sums 32 exact products
//     below 2^22 in fp32, so its result t is the exact integer sub-block sum.  Q6_K's
//     sc * (q - 32) reaches 4096 in magnitude, where f16 holds only even integers: it is
//     split into two exact planes, (sc - b) * (q - 32) (even) and b * (q - 32) with
//     b = sc & 1, and the two MFMAs chain into t (|t| < 2^24, still exact).
//   * The fp32 rescale is a running scale: the accumulator holds the sum in units of the
//     current (row scale d) x (token scale d8).  Every sub-block multiplies acc by
//     rho = d8_prev / d8 of the token (one multiply per output per sub-block) and the MFMA
//     then adds the sub-block's products straight into that rescaled accumulator, so t is
//     never formed on its own: each step rounds like an fp32 sum of the exact products onto
//     acc * rho.  At a super-block boundary the rows' acc is multiplied by d_prev / d once.  The epilogue
//     multiplies by the last d8 * d.  A zero scale leaves the running scale unchanged and
//     zeroes its block's operand (its products are zero).
//   * Q4_K's min term, sum_s -(dmin*m_s) * ds_js, is one more product over the sub-block
//     index: -dmin*m (an f16 times a 6-bit integer, 17 significant bits) is split into an
//     f16 hi + lo pair that is exact, ds is an f16 already, and two MFMAs per 32 sub-blocks
//     add it to the finished absolute accumulator.
//   Against the fp64 value the roundings are the rescale multiply and the MFMA's fp32
//   accumulation per output per sub-block, and the rho quotients (measured ~1e-7 relative
//   L2).
//
// An int8 MFMA does not fit this product on gfx950: v_mfma_i32_16x16x64_i8 sums 64 values,
// two sub-blocks with different token scales, and the 32-deep v_mfma_i32_16x16x32_i8 runs
// at the f16 MFMA's rate (16 cycles for 16x16x32, measured) while needing three VALU
// operations per output per sub-block (int -> float, the product of the row and token
// scales, the fma) where the exact f16 form needs one.
#include <algorithm>

#include "mnemo_common.hpp"
#include "mnemo_internal.hpp"

namespace mnemo {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ operand conversions
// Byte selectors placing bytes (0, 1) / (2, 3) of a dword under the f16 exponent byte 0x64:
// the pair (1024 + b0, 1024 + b1) exactly.
constexpr uint32_t kSelLo = 0x04010400u, kSelHi = 0x04030402u;

__device__ __forceinline__ h2 magic_pair(uint32_t v, uint32_t sel) {
    return __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, v, sel));
}
// q * sc for two 4-bit quants: (1024 + q) * sc - 1024 * sc in one fused f16 fma, whose
// result q * sc <= 945 is an integer f16 holds exactly
__device__ __forceinline__ uint32_t q4_scaled(uint32_t v, uint32_t sel, h2 sc, h2 nsc) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(magic_pair(v, sel), sc, nsc));
}
// q8 as f16 integers: q8 ^ 0x80 under 0x64 is 1152 + q8 exactly
__device__ __forceinline__ void q8x4_exact(uint32_t v, uint32_t &o0, uint32_t &o1) {
    const h2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const uint32_t u = v ^ 0x80808080u;
    o0 = __builtin_bit_cast(uint32_t, magic_pair(u, kSelLo) + off);
    o1 = __builtin_bit_cast(uint32_t, magic_pair(u, kSelHi) + off);
}
// Q6_K: two 6-bit quant bytes as the f16 pair (q - 32), exactly
__device__ __forceinline__ h2 q6_centered(uint32_t v, uint32_t sel) {
    const h2 off = {(_Float16)-1056.0f, (_Float16)-1056.0f};
    return magic_pair(v, sel) + off;
}
__device__ __forceinline__ uint32_t h2u(h2 v) { return __builtin_bit_cast(uint32_t, v); }

// byte i of the 12 packed scale bytes held in three dwords
__device__ __forceinline__ uint32_t sbyte(uint32_t s0, uint32_t s1, uint32_t s2, int i) {
    const uint32_t w = i < 4 ? s0 : (i < 8 ? s1 : s2);
    return (w >> (8 * (i & 3))) & 0xFFu;
}
// (sc, m) of sub-block j (get_scale_min_k4, kernels.cu:45-53)
__device__ __forceinline__ void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j, uint32_t &sc,
                                              uint32_t &m) {
    if (j < 4) {
        sc = sbyte(s0, s1, s2, j) & 63;
        m = sbyte(s0, s1, s2, j + 4) & 63;
    } else {
        sc = (sbyte(s0, s1, s2, j + 4) & 15) | ((sbyte(s0, s1, s2, j - 4) >> 6) << 4);
        m = (sbyte(s0, s1, s2, j + 4) >> 4) | ((sbyte(s0, s1, s2, j) >> 6) << 4);
    }
}

// The 8 six-bit mins of a Q4_K super-block as bytes, sub-blocks 0-3 / 4-7 (the packed form of
// get_scale_min_k4, kernels.cu:45-53: m_j = scales[j+4] & 63 for j < 4, else
// (scales[j+4] >> 4) | ((scales[j] >> 6) << 4)); hdr.z, hdr.w hold scale bytes 4-7, 8-11.
__device__ __forceinline__ uint2 q4k_mins(const uint4 &hdr) {
    return make_uint2(hdr.z & 0x3F3F3F3Fu, ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u));
}
// Q4_K min-term operand of one super-block: for its 8 sub-blocks, -dmin * m_s as an exact
// f16 hi + lo pair (dmin is an f16, m a 6-bit integer: 17 significant bits), in packed f16:
// hi = the product rounded, lo = fma(m, -dmin, -hi), the remainder (at most 6 significant
// bits, a multiple of dmin's last place: exact, also in the subnormal range)
__device__ __forceinline__ void q4k_min_operand_m(uint2 mins, uint32_t dmin_bits, h8 &hi, h8 &lo) {
    const _Float16 nd = -__builtin_bit_cast(_Float16, (uint16_t)dmin_bits);
    const h2 ndd = {nd, nd};
    const h2 off = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    uint32_t H[4], L[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const h2 m = magic_pair(i < 2 ? mins.x : mins.y, (i & 1) ? kSelHi : kSelLo) + off;  // exact
        const h2 h = m * ndd;
        H[i] = h2u(h);
        L[i] = h2u(__builtin_elementwise_fma(m, ndd, -h));
    }
    hi = __builtin_bit_cast(h8, make_uint4(H[0], H[1], H[2], H[3]));
    lo = __builtin_bit_cast(h8, make_uint4(L[0], L[1], L[2], L[3]));
}
__device__ __forceinline__ void q4k_min_operand(const uint4 &hdr, h8 &hi, h8 &lo) {
    q4k_min_operand_m(q4k_mins(hdr), hdr.x >> 16, hi, lo);
}
// the ds halves of the 8 sub-blocks of a super-block: two Q8_1 block headers
__device__ __forceinline__ h8 ds_operand(const uint4 &b0, const uint4 &b1) {
    const uint32_t sel = 0x07060302u;  // the high halves of two dwords
    const uint4 u = make_uint4(__builtin_amdgcn_perm(b0.y, b0.x, sel), __builtin_amdgcn_perm(b0.w, b0.z, sel),
                               __builtin_amdgcn_perm(b1.y, b1.x, sel), __builtin_amdgcn_perm(b1.w, b1.z, sel));
    return __builtin_bit_cast(h8, u);
}

// The same after LDS writes made by global_load_lds: those complete with the wave's vector
// memory counter, so the wave waits until at most N vector memory operations (the ones it
// issued after the LDS loads) are outstanding.
template <int N>
__device__ __forceinline__ void lds_dma_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
    lds_barrier();
}

__device__ __forceinline__ f4 mfma(const h8 &a, const h8 &b, const f4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f4 mfma0(const h8 &a, const h8 &b) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
}

// ------------------------------------------------------------------ tiled kernel
// A workgroup computes a 128 x 128 tile (weight rows x tokens) over one K slice (blockIdx.z
// of `splits`, whole super-blocks).  Its waves form a 2 (rows: 64 each) x kWC (tokens) x 2
// (sub-block parity) grid: wave (wi, wj, kh) multiplies rows wi .. wi+63 with tokens
// wj .. wj+kWTok-1 over sub-block kh of every 64-wide K step (the step's sub-blocks 2ks and
// 2ks + 1); the two parities are summed through LDS at the end.  All threads load and
// convert the step's weights and activations once into LDS: thread t owns weight row /
// token t / kParts and part t % kParts (kVP values) of the step.
#ifndef MNEMO_GEMM_THREADS
#define MNEMO_GEMM_THREADS 512
#endif
constexpr int kThreads = MNEMO_GEMM_THREADS;  // 512 or 1024
constexpr int kWaves = kThreads / 64;
constexpr int kBM = 128, kBN = 128;
constexpr int kKS = 64;                // K per step
constexpr int kWC = kWaves / 4;        // token groups
constexpr int kWTok = kBN / kWC;       // tokens per wave
constexpr int kNB = kWTok / 16;        // 16-token MFMA columns per wave
constexpr int kParts = kThreads / 128; // loader parts per row and step
constexpr int kVP = kKS / kParts;      // values per part (16 or 8)
static_assert(kVP == 8 || kVP == 16, "loader parts of 8 or 16 values");
// raw ring slots: loads run kPF-2 steps ahead of their conversion
#ifndef MNEMO_GEMM_PF
#define MNEMO_GEMM_PF 3
#endif
constexpr int kPF = MNEMO_GEMM_PF;
// lcm(kPF, 3 LDS stages, 4 steps per super-block): every ring slot, stage and super-block
// boundary of the unrolled loop is a compile-time constant
constexpr int kUnroll = 12;
static_assert(kUnroll % kPF == 0, "ring size must divide the unroll");

// kVP raw bytes as dwords
struct PartBytes {
    uint32_t w[kVP / 4];
};
__device__ __forceinline__ PartBytes ld_part(const uint8_t *p) {
    PartBytes r;
    if constexpr (kVP == 16) {
        const uint4 v = ld16(p);
        r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
    } else {
        const uint2 v = ld8(p);
        r.w[0] = v.x; r.w[1] = v.y;
    }
    return r;
}
__device__ __forceinline__ PartBytes ld_part_a2(const uint8_t *p) {
    PartBytes r;
    if constexpr (kVP == 16) {
        const uint4 v = ld16_a2(p);
        r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
    } else {
        const uint2 v = ld8_a2(p);
        r.w[0] = v.x; r.w[1] = v.y;
    }
    return r;
}

struct RawW {
    uint4 h;         // Q4_K: the super-block header (d, dmin, 12 scale bytes)
    PartBytes a, b;  // Q4_K: a = qs bytes;  Q6_K: a = ql bytes, b = qh bytes
    uint32_t s, dd;  // Q6_K: the int8 scale of the values, f16 d
};
struct RawA {
    PartBytes q;  // int8 quants
    uint32_t ds;  // half2 (d8, ds) of their 32-value sub-block
};

// Part p of step ks covers K columns kVP*p .. +kVP-1 of the step: sub-block 2(ks%4) + c/32 of
// super-block ks/4, positions c%32 .. (c = kVP*p).
// Q4_K: qs bytes 32(ks%4) + c%32 .., the low (c < 32) or high nibbles.
__device__ __forceinline__ void load_w_q4k(const uint8_t *__restrict__ wrow, int ks, int p, RawW &r) {
    const uint8_t *blk = wrow + (size_t)(ks >> 2) * kQ4KBytes;
    r.h = ld16(blk);
    r.a = ld_part(blk + 16 + 32 * (ks & 3) + ((kVP * p) & 31));
}
// Q6_K: values v0 = 64(ks%4) + c of the super-block: half hh = (ks%4)/2, group
// grp = 2(ks%2) + c/32, positions l0 = c%32: ql bytes 64hh + 32(grp%2) + l0 (high nibbles if
// grp >= 2), qh bytes 32hh + l0 at bit 2grp, scale byte 8hh + 2grp + l0/16.
__device__ __forceinline__ void load_w_q6k(const uint8_t *__restrict__ wrow, int ks, int p, RawW &r) {
    const uint8_t *blk = wrow + (size_t)(ks >> 2) * kQ6KBytes;
    const int c = kVP * p, hh = (ks & 3) >> 1, grp = 2 * (ks & 1) + (c >> 5), l0 = c & 31;
    r.a = ld_part_a2(blk + 64 * hh + 32 * (grp & 1) + l0);
    r.b = ld_part_a2(blk + 128 + 32 * hh + l0);
    uint8_t sc;
    uint16_t dd;
    __builtin_memcpy(&sc, blk + 192 + 8 * hh + 2 * grp + (l0 >> 4), 1);
    __builtin_memcpy(&dd, blk + 208, 2);
    r.s = sc;
    r.dd = dd;
}
// Activations of step ks, part p: values 64ks + kVP*p .. of the token's Q8_1 MMQ row
// (block v/128, sub-block (v/32)%4).
__device__ __forceinline__ void load_a(const uint8_t *__restrict__ arow, int ks, int p, RawA &r) {
    const int v0 = ks * kKS + kVP * p;
    const uint8_t *blk = arow + (size_t)(v0 >> 7) * kQ81Bytes;
    __builtin_memcpy(&r.ds, blk + 4 * ((v0 >> 5) & 3), 4);
    r.q = ld_part(blk + 16 + (v0 & 127));
}

// f16 tiles of 64 K-columns per row = 8 chunks of 16 B (a row is 128 B, half of the 64 x 4 B
// LDS banks), stored without padding with the chunk index XOR-ed by (row / 2) % 8: the 16
// rows of an MFMA fragment read (one chunk each) cover the 64 banks once, and so do the
// lanes of a conversion store.
__device__ __forceinline__ int tile_off(int row, int chunk) { return row * kKS + ((chunk ^ ((row >> 1) & 7)) << 3); }
// the part's converted values (kVP / 2 dwords of f16 pairs) into its chunks
__device__ __forceinline__ void put_part(_Float16 *tile, int row, int p, const uint32_t (&o)[kVP / 2]) {
#pragma unroll
    for (int c = 0; c < kVP / 8; c++)
        *(uint4 *)(tile + tile_off(row, (kVP / 8) * p + c)) = make_uint4(o[4 * c], o[4 * c + 1], o[4 * c + 2], o[4 * c + 3]);
}

// One LDS stage: the step's operand tiles and the running-scale factors.
template <int TYPE>
struct Stage {
    static constexpr int kPlanes = TYPE == kTypeQ4K ? 1 : 2;
    _Float16 a[kPlanes][kBM * kKS];  // weights: sc*q (Q4_K) or the two Q6_K planes
    _Float16 b[kBN * kKS];           // q8
    float rho[2][kBN];               // token scale ratio of sub-block 2ks + p
    float sig[kBM];                  // row scale ratio (written at super-block starts)
};

// Running scales of a loader thread: the last nonzero d of its weight row (part 0 threads)
// and the last nonzero d8 of its token for the sub-block parity of its part (the first part
// of each sub-block).  Both start at 1.
struct LoaderState {
    float deff, d8eff;
};

__device__ __forceinline__ void row_scale_step(float d, int ks, int p, float *sig, int row, LoaderState &ls, bool live) {
    if (p == 0 && (ks & 3) == 0 && live) {  // super-block start: the row scale changes
        const float dn = d != 0.0f ? d : ls.deff;
        sig[row] = ls.deff * __builtin_amdgcn_rcpf(dn);
        ls.deff = dn;
    }
}

__device__ __forceinline__ void store_w_q4k(const RawW &r, int ks, int p, Stage<kTypeQ4K> &st, int row,
                                            LoaderState &ls, bool live) {
    const int c = kVP * p;
    const int j = 2 * (ks & 3) + (c >> 5);
    uint32_t sc, m;
    q4k_scale_min(r.h.y, r.h.z, r.h.w, j, sc, m);
    const float d = h2f(r.h.x & 0xFFFFu);
    if (d == 0.0f) sc = 0;  // the block's products are zero
    // the pair (sc, -1024 sc) from sc under the 0x64 exponent; high nibbles are taken in
    // place as the bytes 16 q with (sc / 16, -64 sc): (1024 + 16 q) sc / 16 - 64 sc = q sc
    const bool hi = (c >> 5) != 0;
    const h2 F = hi ? h2{(_Float16)0.0625f, (_Float16)0.0625f} : h2{(_Float16)1.0f, (_Float16)1.0f};
    const h2 mk = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    const h2 S = __builtin_elementwise_fma(magic_pair(sc, 0x04000400u), F, F * mk);
    const h2 N = S * mk;
    const uint32_t msk = hi ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
    uint32_t o[kVP / 2];
#pragma unroll
    for (int k = 0; k < kVP / 4; k++) {
        const uint32_t w = r.a.w[k] & msk;
        o[2 * k] = q4_scaled(w, kSelLo, S, N);
        o[2 * k + 1] = q4_scaled(w, kSelHi, S, N);
    }
    put_part(st.a[0], row, p, o);
    row_scale_step(d, ks, p, st.sig, row, ls, live);
}

// Q6_K planes (sc - b)(q - 32) and b(q - 32), b = sc & 1
__device__ __forceinline__ void store_w_q6k(const RawW &r, int ks, int p, Stage<kTypeQ6K> &st, int row,
                                            LoaderState &ls, bool live) {
    const int c = kVP * p, grp = 2 * (ks & 1) + (c >> 5);
    const float d = h2f(r.dd);
    int sc = (int)(int8_t)(r.s & 0xFF);
    if (d == 0.0f) sc = 0;
    const int b1 = sc & 1;
    const _Float16 e = (_Float16)(float)(sc - b1), bb = (_Float16)(float)b1;
    const h2 E = {e, e}, B = {bb, bb};
    const int shl = grp >= 2 ? 4 : 0;
    uint32_t o1[kVP / 2], o2[kVP / 2];
#pragma unroll
    for (int k = 0; k < kVP / 4; k++) {
        const uint32_t lo = (r.a.w[k] >> shl) & 0x0F0F0F0Fu;
        const uint32_t qh = r.b.w[k];
        const uint32_t hi = (2 * grp <= 4 ? (qh << (4 - 2 * grp)) : (qh >> (2 * grp - 4))) & 0x30303030u;
        const uint32_t v = lo | hi;
        const h2 c0 = q6_centered(v, kSelLo), c1 = q6_centered(v, kSelHi);
        o1[2 * k] = h2u(c0 * E);
        o1[2 * k + 1] = h2u(c1 * E);
        o2[2 * k] = h2u(c0 * B);
        o2[2 * k + 1] = h2u(c1 * B);
    }
    put_part(st.a[0], row, p, o1);
    put_part(st.a[1], row, p, o2);
    row_scale_step(d, ks, p, st.sig, row, ls, live);
}

template <int TYPE>
__device__ __forceinline__ void store_a(const RawA &r, int p, Stage<TYPE> &st, int row, LoaderState &ls, bool live) {
    const float d8 = h2f(r.ds & 0xFFFFu);
    const bool zero = d8 == 0.0f;  // x = 0 * q8 = 0 whatever the quants hold (a block whose d
                                   // rounds to f16 zero keeps quants up to +-127)
    uint32_t o[kVP / 2];
#pragma unroll
    for (int k = 0; k < kVP / 4; k++) q8x4_exact(zero ? 0u : r.q.w[k], o[2 * k], o[2 * k + 1]);
    put_part(st.b, row, p, o);
    const int c = kVP * p;
    if ((c & 31) == 0 && live) {  // first part of a sub-block: its token scale ratio
        const float dn = zero ? ls.d8eff : d8;
        st.rho[c >> 5][row] = ls.d8eff * __builtin_amdgcn_rcpf(dn);
        ls.d8eff = dn;
    }
}

template <int TYPE>
__device__ __forceinline__ void load_step(const uint8_t *wrow, const uint8_t *arow, int ks, int p, RawW &rw,
                                          RawA &ra) {
    if (TYPE == kTypeQ4K) load_w_q4k(wrow, ks, p, rw);
    else load_w_q6k(wrow, ks, p, rw);
    load_a(arow, ks, p, ra);
}
template <int TYPE>
__device__ __forceinline__ void store_step(const RawW &rw, const RawA &ra, int ks, int p, Stage<TYPE> &st, int row,
                                           LoaderState &ls, bool live) {
    if constexpr (TYPE == kTypeQ4K) store_w_q4k(rw, ks, p, st, row, ls, live);
    else store_w_q6k(rw, ks, p, st, row, ls, live);
    store_a<TYPE>(ra, p, st, row, ls, live);
}

// A wave's operands of one step: fragments of its sub-block (kh) for 4 x kNB MFMA tiles, the
// token scale ratios of its 16-token columns, and (at super-block starts) the row ratios of
// the rows its accumulators hold.
template <int TYPE>
struct Frags {
    h8 a[Stage<TYPE>::kPlanes][4];
    h8 b[kNB];
    float rho[kNB];
};
template <int TYPE>
__device__ __forceinline__ void read_frags(const Stage<TYPE> &st, int wi, int wj, int kh, int lane, Frags<TYPE> &f) {
    const int chunk = 4 * kh + (lane >> 4);
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int ra = wi + 16 * t + (lane & 15);
#pragma unroll
        for (int p = 0; p < Stage<TYPE>::kPlanes; p++) f.a[p][t] = *(const h8 *)(st.a[p] + tile_off(ra, chunk));
    }
#pragma unroll
    for (int t = 0; t < kNB; t++) {
        const int rb = wj + 16 * t + (lane & 15);
        f.b[t] = *(const h8 *)(st.b + tile_off(rb, chunk));
        f.rho[t] = st.rho[kh][rb];
    }
}

// acc = acc * rho, then the MFMA adds the step's exact products to the rescaled accumulator
// (rounded as fp32 sums onto it)
// (at a super-block start the row ratios come first, read from the step's own stage, which
// no thread writes during the step)
template <int TYPE>
__device__ __forceinline__ void mfma_step(const Frags<TYPE> &f, const Stage<TYPE> &st, int wi, int lane,
                                          f4 (&acc)[4][kNB], bool sb_start) {
    if (sb_start) {
#pragma unroll
        for (int a = 0; a < 4; a++) {
            const f4 sg = *(const f4 *)(st.sig + wi + 16 * a + 4 * (lane >> 4));
#pragma unroll
            for (int b = 0; b < kNB; b++) acc[a][b] *= sg;
        }
    }
#pragma unroll
    for (int b = 0; b < kNB; b++) {
#pragma unroll
        for (int a = 0; a < 4; a++) {
            acc[a][b] *= f.rho[b];
            acc[a][b] = mfma(f.a[0][a], f.b[b], acc[a][b]);
            if constexpr (TYPE == kTypeQ6K) acc[a][b] = mfma(f.a[1][a], f.b[b], acc[a][b]);
        }
    }
}

struct GemmArgs {
    const uint8_t *W;   // weights [M][K] (plain); expert table base (grouped)
    const void *A;      // Q8_1 MMQ rows (plain); staged q8 rows, f16 integers (grouped)
    const float *a_rho;      // grouped: [rows][K/32] token scale ratios
    const uint16_t *a_ds;    // grouped: [rows][K/32] f16 ds
    const float *a_dlast;    // grouped: [rows] last nonzero d8 (1 if none)
    float *out;
    int M, K, N, splits;
    int out_ld;
    // grouped launches
    size_t expert_stride, w_off, w_off2;  // expert e's matrix at W + e*stride + w_off (up: w_off2)
    const int *counts;                   // [n_experts] rows per expert
    const int *offsets;                  // [n_experts] first expert-sorted row
    const int *perm;                     // [rows] expert-sorted row -> token (SwiGLU gather)
    const int *tiles;                    // [max_tiles] (expert << 16) | n_tile; tiles[-1] = count
};

template <int TYPE, bool ATOMIC>
__global__ void __launch_bounds__(kThreads) gemm_q8_1_kernel(GemmArgs g) {
    __shared__ __align__(16) Stage<TYPE> lds[3];
    __shared__ float dlast[kBM], d8last[2][kBN];
    // Q4_K min term: the operands of the split's super-blocks (up to kMhSb), kept as the
    // loaders pass them -- per weight row and super-block the 8 six-bit mins (one byte each)
    // and dmin, per token and sub-block the f16 ds of its Q8_1 block
    constexpr int kMhSb = 16;
    constexpr int kQ4 = TYPE == kTypeQ4K;
    __shared__ uint2 mhm[kQ4 ? kBM * kMhSb : 1];
    __shared__ uint16_t mhd[kQ4 ? kBM * kMhSb : 1];
    __shared__ __align__(16) uint16_t dsk[kQ4 ? kBN * kMhSb * 8 : 8];
    const int tid = threadIdx.x;
    // the wave index as a scalar, so that every per-wave decision below is a scalar branch
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int K = g.K;
    const int wi = (wave & 1) * 64, wj = ((wave >> 1) % kWC) * kWTok, kh = wave / (2 * kWC);
    const int bbytes = TYPE == kTypeQ4K ? kQ4KBytes : kQ6KBytes;
    const size_t wrow_bytes = (size_t)(K / 256) * bbytes;
    // this split's super-blocks [sb0, sb1) = steps [ks0, ks1)
    const int nsb = K / 256;
    const int sb0 = (int)((long)nsb * blockIdx.z / g.splits), sb1 = (int)((long)nsb * (blockIdx.z + 1) / g.splits);
    const int ks0 = 4 * sb0, ks1 = 4 * sb1, last = ks1 - 1;
    const int i0 = blockIdx.x * kBM, j0 = blockIdx.y * kBN;

    // loader role: thread -> (row / token lr, part lp); rows past the end re-read the last
    const int lr = tid / kParts, lp = tid % kParts;
    const uint8_t *wrow = g.W + (size_t)min(i0 + lr, g.M - 1) * wrow_bytes;
    const uint8_t *arow = (const uint8_t *)g.A + (size_t)min(j0 + lr, g.N - 1) * (K / 128) * kQ81Bytes;
    LoaderState ls{1.0f, 1.0f};

    f4 acc[4][kNB];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < kNB; b++) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};

    // Pipeline: three LDS stages.  In step ks a wave multiplies the fragments of step ks
    // (read during step ks-1), reads the fragments of step ks+1 (its stage was completed
    // before the previous barrier), converts step ks+2 into the third stage, then meets
    // the barrier.  Raw blocks sit in a ring of kPF register slots, loaded kPF-2 steps
    // before their conversion.  Conversions past the last step fill idle stages and leave
    // the running scales alone.
    RawW rw[kPF];
    RawA ra[kPF];
#pragma unroll
    for (int p = 0; p < kPF; p++) load_step<TYPE>(wrow, arow, min(ks0 + p, last), lp, rw[p], ra[p]);
    const bool keep_min = TYPE == kTypeQ4K && sb1 - sb0 <= kMhSb;  // uniform
    // step q (relative to ks0) of the split: the loader of a row's first part keeps its mins
    // and dmin at the super-block's first step, the loader of a sub-block's first values its ds
    auto keep = [&](const RawW &w, const RawA &a, int q, bool first_step, bool live) {
        if (!keep_min || !live) return;
        if (lp == 0 && first_step) {
            mhm[lr * kMhSb + (q >> 2)] = q4k_mins(w.h);
            mhd[lr * kMhSb + (q >> 2)] = (uint16_t)(w.h.x >> 16);
        }
        if (((kVP * lp) & 31) == 0)
            dsk[lr * kMhSb * 8 + (q >> 2) * 8 + 2 * (q & 3) + ((kVP * lp) >> 5)] = (uint16_t)(a.ds >> 16);
    };
    store_step<TYPE>(rw[0], ra[0], ks0, lp, lds[0], lr, ls, true);
    keep(rw[0], ra[0], 0, true, true);
    store_step<TYPE>(rw[1], ra[1], ks0 + 1, lp, lds[1], lr, ls, ks0 + 1 < ks1);
    keep(rw[1], ra[1], 1, false, ks0 + 1 < ks1);
    lds_barrier();
    Frags<TYPE> fr;
    read_frags<TYPE>(lds[0], wi, wj, kh, lane, fr);

    for (int kb = ks0; kb < ks1; kb += kUnroll) {
#pragma unroll
        for (int p = 0; p < kUnroll; p++) {
            const int ks = kb + p;
            if (ks < ks1) {  // uniform
                // kb - ks0 is a multiple of kUnroll and ks0 of 4, so these are compile-time
                // constants
                const int r = p % kPF, b = p % 3;
                load_step<TYPE>(wrow, arow, min(ks + kPF, last), lp, rw[r], ra[r]);
                mfma_step<TYPE>(fr, lds[b], wi, lane, acc, p % 4 == 0);
                read_frags<TYPE>(lds[(b + 1) % 3], wi, wj, kh, lane, fr);
                store_step<TYPE>(rw[(r + 2) % kPF], ra[(r + 2) % kPF], ks + 2, lp, lds[(b + 2) % 3], lr, ls,
                                 ks + 2 < ks1);
                // (ks + 2 - ks0) % 4 == (p + 2) % 4: a compile-time test
                keep(rw[(r + 2) % kPF], ra[(r + 2) % kPF], ks + 2 - ks0, ((p + 2) & 3) == 0, ks + 2 < ks1);
                lds_barrier();
            }
        }
    }
    // absolute values: the last nonzero scales of each row and each token (per parity)
    if (lp == 0) dlast[lr] = ls.deff;
    if (((kVP * lp) & 31) == 0) d8last[(kVP * lp) >> 5][lr] = ls.d8eff;
    __syncthreads();
#pragma unroll
    for (int a = 0; a < 4; a++) {
        const f4 dr = *(const f4 *)(dlast + wi + 16 * a + 4 * (lane >> 4));
#pragma unroll
        for (int b = 0; b < kNB; b++) {
            const float dt = d8last[kh][wj + 16 * b + (lane & 15)];
#pragma unroll
            for (int e = 0; e < 4; e++) acc[a][b][e] *= dr[e] * dt;
        }
    }

    // Q4_K min term, sum_s -(dmin*m_s)_i * ds_js, added to the absolute accumulator after
    // the loop, from the operands the loaders kept in LDS (up to 16 super-blocks per split;
    // reading the headers and the Q8_1 block heads again from memory touched every weight
    // line a second time and 4096 activation lines per workgroup).  Windows of 32 sub-blocks
    // (4 super-blocks), wave parity kh taking windows kh, kh+2, ...; lane group q = lane/16
    // holds super-block 4w + q of its row / token (K index 8q + s of the MFMA = sub-block s of
    // that super-block).
    if constexpr (TYPE == kTypeQ4K) {
        const int q = lane >> 4;
        const int nwin = (sb1 - sb0 + 3) / 4;
        for (int w = kh; w < nwin; w += 2) {
            const int sb = sb0 + 4 * w + q;
            const bool valid = sb < sb1;
            uint4 hdr[4], blk[kNB][2];
            if (keep_min) {  // the operands the loaders kept: no second pass over weights or activations
                const int rs = valid ? sb - sb0 : 0;
                h8 bd[kNB];
#pragma unroll
                for (int b = 0; b < kNB; b++) {
                    bd[b] = *(const h8 *)&dsk[(wj + 16 * b + (lane & 15)) * kMhSb * 8 + rs * 8];
                    if (!valid) bd[b] = h8{};
                }
#pragma unroll
                for (int a = 0; a < 4; a++) {
                    const int row = wi + 16 * a + (lane & 15);
                    h8 hi, lo;
                    q4k_min_operand_m(mhm[row * kMhSb + rs], valid ? mhd[row * kMhSb + rs] : 0u, hi, lo);
#pragma unroll
                    for (int b = 0; b < kNB; b++) acc[a][b] = mfma(lo, bd[b], mfma(hi, bd[b], acc[a][b]));
                }
                continue;
            }
#pragma unroll
            for (int a = 0; a < 4; a++) {
                const uint8_t *rp = g.W + (size_t)min(i0 + wi + 16 * a + (lane & 15), g.M - 1) * wrow_bytes;
                hdr[a] = valid ? ld16(rp + (size_t)sb * kQ4KBytes) : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (int b = 0; b < kNB; b++) {
                const uint8_t *ap = (const uint8_t *)g.A +
                                    (size_t)min(j0 + wj + 16 * b + (lane & 15), g.N - 1) * (K / 128) * kQ81Bytes;
                blk[b][0] = valid ? ld16(ap + (size_t)(2 * sb) * kQ81Bytes) : make_uint4(0, 0, 0, 0);
                blk[b][1] = valid ? ld16(ap + (size_t)(2 * sb + 1) * kQ81Bytes) : make_uint4(0, 0, 0, 0);
            }
            h8 bd[kNB];
#pragma unroll
            for (int b = 0; b < kNB; b++) bd[b] = ds_operand(blk[b][0], blk[b][1]);
#pragma unroll
            for (int a = 0; a < 4; a++) {
                h8 hi, lo;
                q4k_min_operand(hdr[a], hi, lo);
#pragma unroll
                for (int b = 0; b < kNB; b++) acc[a][b] = mfma(lo, bd[b], mfma(hi, bd[b], acc[a][b]));
            }
        }
    }

    // sum the two parities: the kh = 1 waves hand their tiles to their kh = 0 counterparts
    // through the (now idle) stages, laid out lane-minor so the accesses are conflict-free
    __syncthreads();
    float *red = (float *)&lds[0] + (size_t)(wave % (kWaves / 2)) * (64 * kWTok);
    if (kh) {
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int b = 0; b < kNB; b++)
#pragma unroll
                for (int e = 0; e < 4; e++) red[((a * kNB + b) * 4 + e) * 64 + lane] = acc[a][b][e];
    }
    __syncthreads();
    if (kh) return;
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < kNB; b++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[a][b][e] += red[((a * kNB + b) * 4 + e) * 64 + lane];
    // D layout (16x16 f32): lane l holds rows 4*(l/16)+e, column l%16.  Rows index
    // weights (A operand), columns tokens (B operand).
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < kNB; b++) {
            const int j = j0 + wj + 16 * b + (lane & 15);
            const int ib = i0 + wi + 16 * a + 4 * (lane >> 4);
            if (j >= g.N) continue;
            float *o = g.out + (size_t)j * g.out_ld + ib;
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
        for (int t = 0; t < kWTok; t++) {
            const int j = j0 + wj + t;
            if (j >= g.N) break;
            if (ib < g.M)
                __hip_atomic_fetch_add(g.out + (size_t)j * g.out_ld + ib,
                                       red[t * 64 + ((((lane >> 2) ^ (t & 15)) << 2) | (lane & 3))], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ------------------------------------------------------------------ activation staging
// fp32 rows [N][K] -> the grouped kernel's operand form of cuda_quantize_mmq_q8_1's output
// (per 32 values d = amax/127, q = rint(x*127/amax) clamped to +-127, ds = f16(d * sum x);
// gemm_q4k.cu:327-358): q8 as f16 integers [N][K], the f16 ds [N][K/32], the running-scale
// ratio rho_s = d8eff_{s-1} / d8eff_s [N][K/32] (d8eff: the last nonzero f16 d8 at or before
// s, 1 before the first) and the last d8eff of the row [N].  One wave per row.
constexpr int kStageThreads = 256;

__global__ void __launch_bounds__(kStageThreads) stage_f32_kernel(const float *__restrict__ x, int K, int N,
                                                                  _Float16 *__restrict__ q8, float *__restrict__ rho,
                                                                  uint16_t *__restrict__ dsv,
                                                                  float *__restrict__ dlast) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (kStageThreads / 64) + (threadIdx.x >> 6);
    if (row >= N) return;
    const int nsub = K / 32;
    const float4 *xr = (const float4 *)(x + (size_t)row * K);
    _Float16 *qrow = q8 + (size_t)row * K;
    float carry = 1.0f;  // d8eff before this pass's first block
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    for (int b0 = 0; b0 < nsub; b0 += 64) {
        const int b = b0 + lane;
        float d8 = 0.0f;
        if (b < nsub) {
            // the arithmetic of quantize_q8_1_kernel (router.hip), so the values agree bit
            // for bit with cuda_quantize_mmq_q8_1
            float xv[32];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 v = xr[8 * b + i];
                xv[4 * i] = v.x; xv[4 * i + 1] = v.y; xv[4 * i + 2] = v.z; xv[4 * i + 3] = v.w;
            }
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(xv[i]));
            const float d = amax / 127.0f;
            const float id = (amax > 0.0f) ? 127.0f / amax : 0.0f;
            float sum = 0.0f;
            uint32_t o[16];
#pragma unroll
            for (int i = 0; i < 16; i++) {
                float r0 = rintf(xv[2 * i] * id), r1 = rintf(xv[2 * i + 1] * id);
                r0 = fminf(fmaxf(r0, -127.0f), 127.0f);
                r1 = fminf(fmaxf(r1, -127.0f), 127.0f);
                sum += xv[2 * i];
                sum += xv[2 * i + 1];
                o[i] = h2u(h2{(_Float16)r0, (_Float16)r1});
            }
            float dsum = d * sum;
            asm volatile("" : "+v"(dsum));  // fp32 product, then the f16 rounding
            const uint16_t dh = f2h_bits(d);
            d8 = h2f(dh);
            dsv[(size_t)row * nsub + b] = f2h_bits(dsum);
            // a block whose d rounds to f16 zero (amax < 2^-25 * 127) still has quants up to
            // +-127; its values d8 * q8 are zero, and so are the staged operands (the running
            // scale skips the block)
            const uint32_t keep = d8 != 0.0f ? ~0u : 0u;
            uint4 *dst = (uint4 *)(qrow + 32 * b);
#pragma unroll
            for (int i = 0; i < 4; i++)
                dst[i] = make_uint4(o[4 * i] & keep, o[4 * i + 1] & keep, o[4 * i + 2] & keep, o[4 * i + 3] & keep);
        }
        // running scale: the last nonzero d8 before each block (the carry if none in this pass)
        const uint64_t nz = __ballot(d8 != 0.0f);
        const uint64_t m = nz & below;
        const int src = m ? 63 - __builtin_clzll(m) : 0;
        const float prev_in = __shfl(d8, src);
        const float prev = m ? prev_in : carry;
        const float cur = d8 != 0.0f ? d8 : prev;
        if (b < nsub) rho[(size_t)row * nsub + b] = prev / cur;
        carry = __shfl(cur, 63);
    }
    if (lane == 0) dlast[row] = carry;
}

int launch_stage_f32(const float *x, int K, int N, StagedAct sa, hipStream_t s) {
    hipLaunchKernelGGL(stage_f32_kernel, dim3((N + 3) / 4), dim3(kStageThreads), 0, s, x, K, N, sa.q8, sa.rho, sa.ds,
                       sa.dlast);
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

int launch_gemm_q8_1(int type, const void *w, const void *act, float *out, int M, int K, int N,
                     hipStream_t stream) {
    if (!w || !act || !out || M <= 0 || N <= 0 || K <= 0 || K % 256 != 0)
        return set_error(kErrBadArg, "gemm: need non-null pointers, M, N > 0 and K %% 256 == 0");
    if (type != kTypeQ4K && type != kTypeQ6K) return set_error(kErrUnsupportedType, "gemm: unsupported type %d", type);
    if (((uintptr_t)out & 15) != 0) return set_error(kErrBadArg, "gemm: output must be 16-byte aligned");
    if (((uintptr_t)act & 3) != 0) return set_error(kErrBadArg, "gemm: activation blocks must be 4-byte aligned");
    const int tm = (M + kBM - 1) / kBM, tn = (N + kBN - 1) / kBN;
    // split K (whole super-blocks) while the split grid still fits the CUs once, keeping
    // at least 2 super-blocks per split
    const int nsb = K / 256;
    int splits = 1;
    while (2 * tm * tn * splits <= device_cus_gemm() && nsb / (splits * 2) >= 2) splits *= 2;
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
    const dim3 grid(tm, tn, splits);
#define MNEMO_GEMM_LAUNCH(T_, A_) hipLaunchKernelGGL((gemm_q8_1_kernel<T_, A_>), grid, dim3(kThreads), 0, stream, g)
    if (type == kTypeQ4K) {
        if (splits > 1) MNEMO_GEMM_LAUNCH(kTypeQ4K, true);
        else MNEMO_GEMM_LAUNCH(kTypeQ4K, false);
    } else {
        if (splits > 1) MNEMO_GEMM_LAUNCH(kTypeQ6K, true);
        else MNEMO_GEMM_LAUNCH(kTypeQ6K, false);
    }
#undef MNEMO_GEMM_LAUNCH
    return check_launch("gemm_q8_1");
}

// ------------------------------------------------------------------ skinny grouped kernel
// The grouped expert GEMMs of the MoE prefill: an expert receives a few tens of tokens, so a
// tile is at most kGroupTile (64) token rows and the weights dominate the traffic.  A
// workgroup of 8 waves multiplies one token tile with 8 x 16R weight rows; every wave owns R
// row tiles of 16 and converts its own A operands in registers, and the tile's staged
// activation rows are shared through LDS.  Each MFMA covers one sub-block (the running scale
// needs the exact per-sub-block sums): lane group q = lane/16 holds values 8q .. 8q+7 of the
// sub-block, i.e.
//   Q4_K sub-block j = 2g + h: qs bytes 32g + 8q .. +7, nibble h;
//   Q6_K sub-block j = 4H + grp: ql bytes 64H + 32(grp%2) + 8q .. +7 (nibble grp/2), qh bytes
//        32H + 8q .. +7 (bits 2grp), scale 8H + 2grp + q/2;
// and the activation fragment is the staged row's values 32j + 8q .. +7 (natural order).
// Q4_K weights reach the wave through its own LDS area: the 16 rows x 144 B of a tile's
// block are 144 row-contiguous 16-byte chunks copied with global_load_lds (whole cache lines
// per request, no registers held while they are in flight -- lanes loading their own 8-byte
// pieces touch 16 rows per instruction and kept the L1 busy at ~3 TB/s in a read test
// against ~4.8 TB/s for the copies), then read back per lane.  Q6_K blocks (210 B, 2-byte
// aligned) are copied as dwords (sk_copy_q6).
constexpr int kSkTok = kGroupTile;  // token rows per tile: up to 4 column tiles of 16
// weight rows per wave: SwiGLU one gate and one up tile of 16 (same features); grouped two
// tiles of 16 (Q4_K) or one (Q6_K, whose raw blocks take more registers)
template <int TYPE, int MODE>
constexpr int sk_rows_per_wave() { return MODE == 1 || TYPE == kTypeQ4K ? 32 : 16; }
// waves per workgroup: Q4_K 8 (one workgroup per CU: its double-buffered weight areas fill
// the LDS), Q6_K 16 (single-buffered weight areas, four waves per SIMD within 128 registers)
template <int TYPE>
constexpr int sk_waves() { return TYPE == kTypeQ6K ? 16 : 8; }
// activation staging passes of a workgroup of W waves (2W rows of 32 chunks per pass); rows
// past NB 16 repeat the tile's last token into the unused rest of the buffer
template <int NB, int W>
constexpr int sk_passes() { return (NB * 16 + 2 * W - 1) / (2 * W); }
// One block of a 16-row tile is 2304 B = 144 chunks of 16 B.  Every copy instruction is
// issued by the whole wave (a lane-predicated copy invites the compiler to merge it with its
// neighbour and derive the wave-uniform LDS address from the wrong lane): chunks 0-127 of
// tile a go to bytes 2048a .. of the wave's area with two copies, chunks 128-143 of all
// tiles to the tail at 2048R + 256a with one copy, whose lanes past 16R repeat a chunk into
// the unused rest of the tail.
template <int R>
constexpr int sk_q4_area() { return 2048 * R + 1024; }
template <int R>
constexpr int sk_q4_copies() { return 2 * R + 1; }

// Q6_K raw bytes of one row tile's lane values for one block
struct SkRaw6 {
    uint2 ql[4];  // ql bytes 64H + 32p + 8q .. +7 (index 2H + p)
    uint2 qh[2];  // qh bytes 32H + 8q .. +7
    uint32_t sc[2];  // the lane's scale bytes of halves 0 / 1 (byte grp: scale 8H + 2grp + q/2)
    uint32_t d;      // f16 d
};
// Q6_K blocks reach the wave through its LDS area by 16-byte copies (lanes loading their
// own 8-byte pieces touch 16 rows per instruction; with those loads replaced by constants the
// cfg5 prefill took 0.75 instead of 1.01 ms).  A block is 210 B, so every other one starts at
// 2 mod 4: row r's window starts at the dword that holds the block's first byte (sh = block
// offset & 2 bytes before it) and occupies chunk slots 15 r .. 15 r + 14 of the area (240 B
// per row: the 16 rows' reads fall in distinct banks).  Chunks 0-12 are window bytes
// 16 ch ..; chunk 13 is window bytes 196-211 when sh = 2 (block bytes 194-209) and a repeat of
// chunk 12 when sh = 0; chunk 14 repeats chunk 12.  So no copy reads past its block, and the
// block's bytes 0-207 are in the area; d (bytes 208-209) is loaded by the lanes themselves.
// Slot t = 64 i + lane is written by copy i; slots past 239 repeat row 15's chunk 12.
constexpr int kSk6Slots = 15;
constexpr int kSk6Copies = 4;
constexpr int kSk6Area = kSk6Copies * 1024;
// vector memory instructions per block: the copies and the 2-byte d
constexpr int kSk6Loads = kSk6Copies + 1;

// the copies of block k: x6[i] = (offset of the slot's row from the tile's 4-byte aligned
// start) + window offset of the chunk, bit 0 set for chunk 13 (moved 4 bytes on when sh = 2)
__device__ __forceinline__ void sk_copy_q6(const uint8_t *tile, const uint32_t (&x6)[kSk6Copies], int k,
                                           uint8_t *dst) {
#pragma unroll
    for (int i = 0; i < kSk6Copies; i++) {
        const uint32_t a = x6[i] + (uint32_t)(kQ6KBytes * k);
        const uint32_t o = (a & ~3u) + ((a & 1u) ? (a & 2u) << 1 : 0u);
        __builtin_amdgcn_global_load_lds((const void *)(tile + o),
                                         (__attribute__((address_space(3))) void *)(dst + 1024 * i), 16, 0, 0);
    }
}

// the lane's raw values of row c's block from the wave's LDS area (sh: the block's
// misalignment, 0 or 2 bytes); d arrives separately
__device__ __forceinline__ void sk_read6(const uint8_t *area, int c, int q, uint32_t sh, SkRaw6 &r) {
    const uint32_t *a = (const uint32_t *)area + 4 * kSk6Slots * c;
    auto rd8 = [&](int o) {  // block bytes o .. o + 7, o a multiple of 8
        const uint32_t w0 = a[o >> 2], w1 = a[(o >> 2) + 1], w2 = a[(o >> 2) + 2];
        return make_uint2(__builtin_amdgcn_alignbyte(w1, w0, sh), __builtin_amdgcn_alignbyte(w2, w1, sh));
    };
#pragma unroll
    for (int i = 0; i < 4; i++) r.ql[i] = rd8(64 * (i >> 1) + 32 * (i & 1) + 8 * q);
#pragma unroll
    for (int H = 0; H < 2; H++) r.qh[H] = rd8(128 + 32 * H + 8 * q);
    // of the 16 scale bytes the lane needs 8H + 2grp + q/2: bytes q/2, 2 + q/2, .. of each
    // dword, packed per half; window dword 52 (sh = 2 only) is the last of chunk 13
    uint32_t w[5];
#pragma unroll
    for (int i = 0; i < 4; i++) w[i] = a[48 + i];
    w[4] = a[sh ? 55 : 52];
    uint4 sc;
    sc.x = __builtin_amdgcn_alignbyte(w[1], w[0], sh);
    sc.y = __builtin_amdgcn_alignbyte(w[2], w[1], sh);
    sc.z = __builtin_amdgcn_alignbyte(w[3], w[2], sh);
    sc.w = __builtin_amdgcn_alignbyte(w[4], w[3], sh);
    const uint32_t sel = 0x06040200u + 0x01010101u * (uint32_t)(q >> 1);
    r.sc[0] = __builtin_amdgcn_perm(sc.y, sc.x, sel);
    r.sc[1] = __builtin_amdgcn_perm(sc.w, sc.z, sel);
}

// Q4_K lane view of a tile's block: the header (d, dmin, scales) and the lane's qs bytes
struct SkQ4 {
    uint4 h;
    uint2 a[4];  // qs bytes 32g + 8q .. +7
};
// byte o of tile a's block in the wave's LDS area (reads of 8 or 16 aligned bytes never
// straddle the split at 2048)
template <int R>
__device__ __forceinline__ const uint8_t *sk_q4_at(const uint8_t *area, int a, int o) {
    return o < 2048 ? area + 2048 * a + o : area + 2048 * R + 256 * a + (o - 2048);
}
template <int R>
__device__ __forceinline__ SkQ4 sk_read_q4(const uint8_t *area, int a, int c, int q) {
    SkQ4 r;
    const int row = c * kQ4KBytes;
    r.h = *(const uint4 *)sk_q4_at<R>(area, a, row);
#pragma unroll
    for (int g = 0; g < 4; g++) r.a[g] = *(const uint2 *)sk_q4_at<R>(area, a, row + 16 + 32 * g + 8 * q);
    return r;
}
// the 8 six-bit scales of a Q4_K block as bytes (get_scale_min_k4, kernels.cu:45-53): sub-blocks
// 0-3 are the low 6 bits of bytes 0-3, 4-7 the low nibbles of bytes 8-11 with bits 6-7 of
// bytes 0-3 above them (the packed form of gemm_q4k.cu:53-56)
__device__ __forceinline__ void q4k_scales8(const uint4 &h, uint32_t &lo, uint32_t &hi) {
    lo = h.y & 0x3F3F3F3Fu;
    hi = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
}
// sub-block j's A operand, sc*q for its 8 values: the pair (1024 + sc) from the scale byte
// under 0x64, so that (sc, -1024 sc) cost three packed operations
// the scales of sub-blocks 4H + g as f16 pairs (g = 0, 1 | 2, 3) and their products with -1024
// (odd sub-blocks, the high nibbles, are taken in place as bytes 16 q: their pair is
// (sc / 16, -64 sc), and (1024 + 16 q) * sc / 16 - 64 sc = q * sc in the same exact fma)
struct Sk4Scales {
    h2 s[2], n[2];
};
__device__ __forceinline__ Sk4Scales sk_scales4(uint32_t sc4) {
    Sk4Scales o;
    const h2 m = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    const h2 f = {(_Float16)1.0f, (_Float16)0.0625f};
    o.s[0] = (magic_pair(sc4, kSelLo) + m) * f;
    o.s[1] = (magic_pair(sc4, kSelHi) + m) * f;
    o.n[0] = o.s[0] * m;
    o.n[1] = o.s[1] * m;
    return o;
}
__device__ __forceinline__ h8 sk_operand4(const SkQ4 &r, const Sk4Scales &T, int j) {
    const _Float16 sj = T.s[(j & 3) >> 1][j & 1], nj = T.n[(j & 3) >> 1][j & 1];
    const h2 S = {sj, sj}, N = {nj, nj};
    const uint2 c = r.a[j >> 1];
    const uint32_t msk = (j & 1) ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
    const uint32_t w0 = c.x & msk, w1 = c.y & msk;
    return __builtin_bit_cast(h8, make_uint4(q4_scaled(w0, kSelLo, S, N), q4_scaled(w0, kSelHi, S, N),
                                             q4_scaled(w1, kSelLo, S, N), q4_scaled(w1, kSelHi, S, N)));
}
// Q6_K: the two factors of the lane's 4 scales of half H (sc - b and b, b = sc & 1) as f16
// pairs, for the half's four sub-blocks at once: e6[g/2] / b6[g/2] hold those of sub-blocks
// 4H + g (g even, g + 1); zero when d is zero
struct Sk6Scales {
    uint32_t e6[2], b6[2];
};
__device__ __forceinline__ Sk6Scales sk_scales6(const SkRaw6 &r, int H, bool dzero) {
    Sk6Scales o;
    const h2 off = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    const uint32_t sc = dzero ? 0u : r.sc[H];
    q8x4_exact(sc & 0xFEFEFEFEu, o.e6[0], o.e6[1]);  // the even parts of the signed bytes
    const uint32_t b = sc & 0x01010101u;
    o.b6[0] = h2u(magic_pair(b, kSelLo) + off);
    o.b6[1] = h2u(magic_pair(b, kSelHi) + off);
    return o;
}
// Q6_K: the planes (sc - b)(q - 32) and b(q - 32) of sub-block j (S: its half's scales)
__device__ __forceinline__ void sk_operand6(const SkRaw6 &r, const Sk6Scales &S, int j, h8 &a1, h8 &a2) {
    const int H = j >> 2, grp = j & 3;
    const h2 ep = __builtin_bit_cast(h2, S.e6[grp >> 1]);
    const h2 bp = __builtin_bit_cast(h2, S.b6[grp >> 1]);
    const h2 E = {ep[grp & 1], ep[grp & 1]}, B = {bp[grp & 1], bp[grp & 1]};
    const uint2 l = r.ql[2 * H + (grp & 1)], hq = r.qh[H];
    const int shl = 4 * (grp >> 1), shh = 2 * grp;
    const uint32_t v0 = ((l.x >> shl) & 0x0F0F0F0Fu) | (((hq.x >> shh) & 0x03030303u) << 4);
    const uint32_t v1 = ((l.y >> shl) & 0x0F0F0F0Fu) | (((hq.y >> shh) & 0x03030303u) << 4);
    const h2 c0 = q6_centered(v0, kSelLo), c1 = q6_centered(v0, kSelHi), c2 = q6_centered(v1, kSelLo),
             c3 = q6_centered(v1, kSelHi);
    a1 = __builtin_bit_cast(h8, make_uint4(h2u(c0 * E), h2u(c1 * E), h2u(c2 * E), h2u(c3 * E)));
    a2 = __builtin_bit_cast(h8, make_uint4(h2u(c0 * B), h2u(c1 * B), h2u(c2 * B), h2u(c3 * B)));
}

// staged activation chunk u (16 B = 8 values) of token row r, XOR-swizzled by the row so
// that the 16 rows of a fragment read hit distinct banks
__device__ __forceinline__ int sk_slot(int r, int u) { return r * 256 + ((u ^ (r & 31)) << 3); }

template <int TYPE, int R>
struct SkLds {
    static constexpr int kW = TYPE == kTypeQ4K ? sk_q4_area<R>() : kSk6Area;
    static constexpr int kWBufs = TYPE == kTypeQ4K ? 2 : 1;
    _Float16 b[2][kSkTok * 256];               // staged q8 of one 256-value block, double-buffered
    float rho[2][kSkTok * 8];                  // the rows' scale ratios of that block's 8 sub-blocks
    uint8_t w[kWBufs][sk_waves<TYPE>()][kW];   // each wave's row tiles of one block (Q4_K double-buffered)
};

// the running row scales at a block start: lane c owns A row c of each tile (its running d
// and the ratio for this block); the lane's outputs are rows 4q + e, whose ratios come from
// lanes 4q + e
template <int NB, int R>
__device__ __forceinline__ void sk_row_scales(const float (&d)[R], int q, float (&deff)[R], f4 (&acc)[R][NB]) {
#pragma unroll
    for (int a = 0; a < R; a++) {
        const float nd = d[a] == 0.0f ? deff[a] : d[a];
        const float sg = deff[a] * __builtin_amdgcn_rcpf(nd);
        deff[a] = nd;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float se = __shfl(sg, 4 * q + e);
#pragma unroll
            for (int b = 0; b < NB; b++) acc[a][b][e] *= se;
        }
    }
}

// copies of block kb of the wave's Q4_K row tiles into its LDS area: copy 2a + i moves
// chunk 64i + lane of tile a, copy 2R the tail chunks (sources from sk_tile's tile_src)
template <int R>
__device__ __forceinline__ void sk_copy_q4(const uint8_t *const (&src)[sk_q4_copies<R>()], int kb, uint8_t *dst) {
#pragma unroll
    for (int i = 0; i < sk_q4_copies<R>(); i++)
        __builtin_amdgcn_global_load_lds((const void *)(src[i] + (size_t)kb * kQ4KBytes),
                                         (__attribute__((address_space(3))) void *)(dst + 1024 * i), 16, 0, 0);
}

// One 256-value block k: the activations (and ratios) of block k+1 are copied into the other
// LDS buffer, the weights of block k+1 into the wave's other LDS area (Q4_K) or into its
// single area (Q6_K, once the lanes have read block k out of it), then block k is
// multiplied.  The barrier at the end waits for the activation copies only (they were issued
// first; memory operations complete in issue order): the weights stay in flight until the
// next block needs them.
// Q6_K copy state of a wave: the 4-byte aligned address at or below its first row, the
// copies' lane offsets (sk_copy_q6), their clamp, row c's offset and the next block's d
struct Sk6 {
    const uint8_t *tile;
    uint32_t x6[kSk6Copies];
    uint32_t roff, dn;
};
template <int TYPE, int NB, int R>
__device__ __forceinline__ void sk_block(int k, int nkb, int q, int c, int wave, int lane, int tid,
                                         const uint8_t *const (&tile_src)[sk_q4_copies<R>()],
                                         const _Float16 *const (&arow)[sk_passes<NB, sk_waves<TYPE>()>()],
                                         const float *rrow, SkLds<TYPE, R> &L, Sk6 &st, float (&deff)[R],
                                         f4 (&acc)[R][NB], bool late_min, uint32_t (&mring)[4][R][2]) {
    constexpr int W = sk_waves<TYPE>();
    // past the end the last block is copied again (into the idle buffers)
    const int kn = min(k + 1, nkb - 1);
    // block k's weights have landed in the wave's LDS area (the memory clobber keeps the
    // compiler from moving the LDS reads above the wait)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    SkRaw6 cur[R];
    if constexpr (TYPE == kTypeQ6K) {
        sk_read6(L.w[0][wave], c, q, (st.roff + (uint32_t)(kQ6KBytes * k)) & 2u, cur[0]);
        cur[0].d = st.dn;
        // the reads have returned before the area is refilled below
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
#pragma unroll
    for (int i = 0; i < sk_passes<NB, W>(); i++)
        __builtin_amdgcn_global_load_lds((const void *)(arow[i] + kn * 256),
                                         (__attribute__((address_space(3))) void *)&L.b[(k + 1) & 1][(2 * wave + 2 * W * i) * 256],
                                         16, 0, 0);
    if (wave < (NB * 32 + 63) / 64)  // the ratios: two 16-byte chunks per row, whole waves
        __builtin_amdgcn_global_load_lds((const void *)(rrow + kn * 8),
                                         (__attribute__((address_space(3))) void *)&L.rho[(k + 1) & 1][(tid & ~63) * 4], 16,
                                         0, 0);
    __builtin_amdgcn_sched_barrier(0);  // the shared copies go first (the barrier below counts on it)
    if constexpr (TYPE == kTypeQ4K) {
        sk_copy_q4<R>(tile_src, kn, L.w[(k + 1) & 1][wave]);
    } else {
        sk_copy_q6(st.tile, st.x6, kn, L.w[0][wave]);
        uint16_t dd;
        __builtin_memcpy(&dd, st.tile + st.roff + (size_t)kn * kQ6KBytes + 208, 2);
        st.dn = dd;
    }
    // keep the loads here, ahead of the multiplication (the scheduler would otherwise sink
    // them past it to save registers, and nothing would be in flight during the MFMAs)
    __builtin_amdgcn_sched_barrier(0);

    SkQ4 w4[R];
    uint32_t slo[R], shi[R];
    Sk6Scales s6[R];
    Sk4Scales s4[R];
    float d[R];
#pragma unroll
    for (int a = 0; a < R; a++) {
        if constexpr (TYPE == kTypeQ4K) {
            w4[a] = sk_read_q4<R>(L.w[k & 1][wave], a, c, q);
            if (late_min) {
                // the min term's operand of row c: lane group q keeps super-block k when k % 4 == q,
                // in a ring of four (window order: the newest in slot 0), moved up one slot at
                // each window's first block (a uniform branch)
                if ((k & 3) == 0) {
#pragma unroll
                    for (int i = 0; i < 2; i++)
#pragma unroll
                        for (int j = 3; j > 0; j--) mring[j][a][i] = mring[j - 1][a][i];
                }
                const bool cap = (k & 3) == q;
                // the 8 six-bit mins in 48 bits (m_j at bit 6j) and dmin in the top 16
                const uint2 mn = q4k_mins(w4[a].h);
                const uint32_t p0 = (mn.x & 0x3Fu) | ((mn.x >> 2) & 0xFC0u) | ((mn.x >> 4) & 0x3F000u) |
                                    ((mn.x >> 6) & 0xFC0000u) | ((mn.y & 0x3Fu) << 24) | ((mn.y & 0x300u) << 22);
                const uint32_t p1 = ((mn.y >> 10) & 0xFu) | ((mn.y >> 12) & 0x3F0u) | ((mn.y >> 14) & 0xFC00u) |
                                    (w4[a].h.x & 0xFFFF0000u);
                mring[0][a][0] = cap ? p0 : mring[0][a][0];
                mring[0][a][1] = cap ? p1 : mring[0][a][1];
            }
            d[a] = h2f(w4[a].h.x & 0xFFFFu);
            q4k_scales8(w4[a].h, slo[a], shi[a]);
            if (d[a] == 0.0f) slo[a] = shi[a] = 0u;  // the block's products are zero
        } else {
            d[a] = h2f(cur[a].d);
        }
    }
    sk_row_scales<NB, R>(d, q, deff, acc);
    const _Float16 *bb = L.b[k & 1];
    const float *rb = L.rho[k & 1];
    // the 8 ratios of each token column: two 16-byte reads (Q4_K); Q6_K reads each where it
    // is used, to fit its 128-register budget
    f4 rr[NB][2];
    if constexpr (TYPE == kTypeQ4K) {
#pragma unroll
        for (int b = 0; b < NB; b++) {
            rr[b][0] = *(const f4 *)(rb + (16 * b + c) * 8);
            rr[b][1] = *(const f4 *)(rb + (16 * b + c) * 8 + 4);
        }
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
        h8 bf[NB];
#pragma unroll
        for (int b = 0; b < NB; b++) bf[b] = *(const h8 *)(bb + sk_slot(16 * b + c, 4 * j + q));
#pragma unroll
        for (int a = 0; a < R; a++) {
            if (TYPE == kTypeQ6K && (j & 3) == 0) s6[a] = sk_scales6(cur[a], j >> 2, d[a] == 0.0f);
            h8 a1, a2;
            if constexpr (TYPE == kTypeQ4K) {
                if ((j & 3) == 0) s4[a] = sk_scales4(j < 4 ? slo[a] : shi[a]);
                a1 = sk_operand4(w4[a], s4[a], j);
            }
            else sk_operand6(cur[a], s6[a], j, a1, a2);
#pragma unroll
            for (int b = 0; b < NB; b++) {
                if constexpr (TYPE == kTypeQ4K) acc[a][b] *= rr[b][j >> 2][j & 3];
                else acc[a][b] *= rb[(16 * b + c) * 8 + j];
                acc[a][b] = mfma(a1, bf[b], acc[a][b]);
                if constexpr (TYPE == kTypeQ6K) acc[a][b] = mfma(a2, bf[b], acc[a][b]);
            }
        }
        // Q6_K: one sub-block's fragment reads at a time (fewer spills under the budget)
        if constexpr (TYPE == kTypeQ6K) __builtin_amdgcn_sched_barrier(0);
    }
    lds_dma_barrier<TYPE == kTypeQ4K ? sk_q4_copies<R>() : R * kSk6Loads>();
}

template <int TYPE, int MODE, int NB>
__device__ __forceinline__ void sk_tile(const GemmArgs &g, SkLds<TYPE, sk_rows_per_wave<TYPE, MODE>() / 16> &L,
                                        int wave, int lane, int tid, int e, int j0, int n_rows, int row_base) {
    constexpr int R = sk_rows_per_wave<TYPE, MODE>() / 16;
    constexpr int H = R / 2;  // SwiGLU: gate tiles 0 .. H-1, up tiles H .. 2H-1
    constexpr int W = sk_waves<TYPE>();
    constexpr int P = sk_passes<NB, W>();
    const int q = lane >> 4, c = lane & 15;
    const int K = g.K, nkb = K / 256;
    const int bbytes = TYPE == kTypeQ4K ? kQ4KBytes : kQ6KBytes;
    const size_t wrow_bytes = (size_t)nkb * bbytes;
    const uint8_t *Wm = g.W + (size_t)e * g.expert_stride + g.w_off;
    const uint8_t *Wm2 = g.W + (size_t)e * g.expert_stride + g.w_off2;

    // weight row r of tile a (rows past M re-read the last)
    int base;  // SwiGLU: first feature of the wave; grouped: first row
    if (MODE == 1) base = (blockIdx.x * W + wave) * (16 * H);
    else base = (blockIdx.x * W + wave) * (16 * R);
    auto row_ptr = [&](int a, int r) {
        if (MODE == 1) return (a < H ? Wm : Wm2) + (size_t)min(base + 16 * (a % H) + r, g.M - 1) * wrow_bytes;
        return Wm + (size_t)min(base + 16 * a + r, g.M - 1) * wrow_bytes;
    };
    const uint8_t *wrow[R];  // the lane's own A row c of each tile
    // Q4_K copy sources: chunk ch of a tile is row ch/9, bytes 16(ch%9) .. of the block
    const uint8_t *tile_src[sk_q4_copies<R>()];
    auto chunk_ptr = [&](int a, int ch) { return row_ptr(a, ch / 9) + 16 * (ch % 9); };
#pragma unroll
    for (int a = 0; a < R; a++) {
        wrow[a] = row_ptr(a, c);
#pragma unroll
        for (int i = 0; i < 2; i++) tile_src[2 * a + i] = chunk_ptr(a, 64 * i + lane);
    }
    tile_src[2 * R] = lane < 16 * R ? chunk_ptr(lane >> 4, 128 + (lane & 15)) : chunk_ptr(R - 1, 143);
    // Q6_K copies (one tile of 16 consecutive rows): offsets from the 4-byte aligned address
    // at or below the first (clamped) row, tb its misalignment
    Sk6 st;
    if constexpr (TYPE == kTypeQ6K) {
        const int r0 = min(base, g.M - 1);
        const uint8_t *t0 = Wm + (size_t)r0 * wrow_bytes;
        const uint32_t tb = (uint32_t)(uintptr_t)t0 & 3u;
        st.tile = t0 - tb;
        auto rel = [&](int r) { return (uint32_t)((min(base + r, g.M - 1) - r0) * wrow_bytes) + tb; };
#pragma unroll
        for (int i = 0; i < kSk6Copies; i++) {
            const int t = 64 * i + lane, row = t < 16 * kSk6Slots ? t / kSk6Slots : 15;
            const int ch = t < 16 * kSk6Slots ? t % kSk6Slots : 12;
            st.x6[i] = rel(row) + (ch <= 12 ? 16u * (uint32_t)ch : ch == 13 ? 192u + 1u : 192u);
        }
        st.roff = rel(c);
    }
    // activation staging role: physical slot tid % 32 of rows r = tid/32 + 2W i, which
    // holds the logical slot (tid % 32) ^ (r % 32); ratio staging: threads below 2 NB 16 copy
    // 16-byte chunk tid % 2 of row tid / 2
    const int sr0 = tid >> 5;
    const _Float16 *arow[P];
    auto stage_row = [&](int r) {
        const int j = min(j0 + r, n_rows - 1);
        return MODE == 1 ? g.perm[row_base + j] : row_base + j;
    };
#pragma unroll
    for (int i = 0; i < P; i++) {
        const int r = sr0 + 2 * W * i, u = (tid & 31) ^ (r & 31);
        arow[i] = (const _Float16 *)g.A + (size_t)stage_row(r) * K + 8 * u;
    }
    const float *rrow = g.a_rho + (size_t)stage_row(min(tid >> 1, NB * 16 - 1)) * (K / 32) + 4 * (tid & 1);
    f4 acc[R][NB];
    float deff[R];  // running d of the lane's A row c of each tile
#pragma unroll
    for (int a = 0; a < R; a++) {
#pragma unroll
        for (int b = 0; b < NB; b++) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};
        deff[a] = 1.0f;
    }
    int tok[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) tok[b] = stage_row(16 * b + c);
#pragma unroll
    for (int i = 0; i < P; i++)
        __builtin_amdgcn_global_load_lds((const void *)arow[i],
                                         (__attribute__((address_space(3))) void *)&L.b[0][(2 * wave + 2 * W * i) * 256],
                                         16, 0, 0);
    if (wave < (NB * 32 + 63) / 64)  // whole waves (rows past NB 16 repeat the last)
        __builtin_amdgcn_global_load_lds((const void *)rrow,
                                         (__attribute__((address_space(3))) void *)&L.rho[0][(tid & ~63) * 4], 16, 0,
                                         0);
    if constexpr (TYPE == kTypeQ4K) {
        sk_copy_q4<R>(tile_src, 0, L.w[0][wave]);
    } else {
        sk_copy_q6(st.tile, st.x6, 0, L.w[0][wave]);
        uint16_t dd;
        __builtin_memcpy(&dd, st.tile + st.roff + 208, 2);
        st.dn = dd;
    }
    // Q4_K's min term, sum_s -(dmin*m_s)_i * ds_js, first: the accumulator starts as this
    // absolute value (the running scales start at 1 and their ratios telescope to
    // 1 / (last d * last d8), which the epilogue multiplies back).  Windows of 32 sub-blocks,
    // lane group q holding super-block 4w + q of its A row / token; the loads of up to four
    // windows are issued together, after the copies of the first block (the two round trips
    // overlap; no measurable change).  Reading the headers here fetches every weight line of
    // the tile once more before the main loop.
    // Q4_K with whole windows and at most four of them (K a multiple of 1024, <= 4096) skips
    // that: lane group q keeps the mins and dmin of the super-blocks it reads from LDS in the
    // main loop (64 bits per row and window, four windows), and the term is added to the
    // absolute values after the loop (cfg5 prefill ~1.04 -> ~1.01 ms, 0 spills at 228 VGPRs;
    // the same ring unpacked to three dwords spilled 44 VGPRs and was slower).
    const bool late_min = TYPE == kTypeQ4K && (nkb & 3) == 0 && nkb <= 16;  // uniform
    uint32_t mring[4][R][2] = {};
    if (TYPE == kTypeQ4K && !late_min) {
        const int nwin = (nkb + 3) / 4;
        for (int w0 = 0; w0 < nwin; w0 += 4) {
            uint4 hdr[4][R], dsv[4][NB];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int sb = 4 * (w0 + u) + q;
                const bool valid = sb < nkb;
#pragma unroll
                for (int a = 0; a < R; a++)
                    hdr[u][a] = valid ? ld16(wrow[a] + (size_t)sb * kQ4KBytes) : make_uint4(0, 0, 0, 0);
#pragma unroll
                for (int b = 0; b < NB; b++)
                    dsv[u][b] = valid ? ld16((const uint8_t *)(g.a_ds + (size_t)tok[b] * (K / 32) + 8 * sb))
                                      : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int a = 0; a < R; a++) {
                    h8 hi, lo;
                    q4k_min_operand(hdr[u][a], hi, lo);
#pragma unroll
                    for (int b = 0; b < NB; b++) {
                        const h8 bd = __builtin_bit_cast(h8, dsv[u][b]);
                        acc[a][b] = mfma(lo, bd, mfma(hi, bd, acc[a][b]));
                    }
                }
        }
    }
    __syncthreads();
    // the loop unrolled by two
    for (int k = 0; k < nkb; k += 2) {
        sk_block<TYPE, NB, R>(k, nkb, q, c, wave, lane, tid, tile_src, arow, rrow, L, st, deff, acc, late_min, mring);
        if (k + 1 >= nkb) break;
        sk_block<TYPE, NB, R>(k + 1, nkb, q, c, wave, lane, tid, tile_src, arow, rrow, L, st, deff, acc, late_min,
                              mring);
    }
    // the copies issued past the last block land before the workgroup's LDS is released
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // absolute values: the last nonzero d of the rows (from lanes 4q + x) and d8 of the tokens
    float dt[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) dt[b] = g.a_dlast[tok[b]];
#pragma unroll
    for (int a = 0; a < R; a++)
#pragma unroll
        for (int x = 0; x < 4; x++) {
            const float dr = __shfl(deff[a], 4 * q + x);
#pragma unroll
            for (int b = 0; b < NB; b++) acc[a][b][x] *= dr * dt[b];
        }
    if (late_min) {
        // the min term on the absolute values: slot j holds window nwin - 1 - j
        const int nwin = nkb >> 2;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (j >= nwin) break;  // uniform
            const int sb = 4 * (nwin - 1 - j) + q;
            h8 bd[NB];
#pragma unroll
            for (int b = 0; b < NB; b++)
                bd[b] = __builtin_bit_cast(h8, ld16((const uint8_t *)(g.a_ds + (size_t)tok[b] * (K / 32) + 8 * sb)));
#pragma unroll
            for (int a = 0; a < R; a++) {
                h8 hi, lo;
                const uint32_t p0 = mring[j][a][0], p1 = mring[j][a][1];
                const uint2 mn = make_uint2((p0 & 0x3Fu) | ((p0 << 2) & 0x3F00u) | ((p0 << 4) & 0x3F0000u) |
                                                ((p0 << 6) & 0x3F000000u),
                                            ((p0 >> 24) & 0x3Fu) | ((p0 >> 22) & 0x300u) | ((p1 << 10) & 0x3C00u) |
                                                ((p1 << 12) & 0x3F0000u) | ((p1 << 14) & 0x3F000000u));
                q4k_min_operand_m(mn, p1 >> 16, hi, lo);
#pragma unroll
                for (int b = 0; b < NB; b++) acc[a][b] = mfma(lo, bd[b], mfma(hi, bd[b], acc[a][b]));
            }
        }
    }

    // D layout: lane holds weight rows 4q + x of each 16-row tile, token column c
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const int j = j0 + 16 * b + c;
        if (j >= n_rows) continue;
        float *orow = g.out + (size_t)(row_base + j) * g.out_ld;
        if (MODE == 1) {
#pragma unroll
            for (int a = 0; a < H; a++) {
                const int f = base + 16 * a + 4 * q;
#pragma unroll
                for (int x = 0; x < 4; x++) {
                    const float gt = acc[a][b][x], up = acc[a + H][b][x];
                    if (f + x < g.M) orow[f + x] = gt / (1.0f + expf(-gt)) * up;
                }
            }
        } else {
#pragma unroll
            for (int a = 0; a < R; a++) {
                const int i = base + 16 * a + 4 * q;
#pragma unroll
                for (int x = 0; x < 4; x++)
                    if (i + x < g.M) orow[i + x] = acc[a][b][x];
            }
        }
    }
}

// MODE 1: SwiGLU (gate and up rows of the same features, activation rows gathered through
// perm[], out[q*ld + f] = silu(gate) * up); MODE 2: the expert-sorted rows themselves.
// The Q6_K kernel's 16 waves (124 KB of LDS, one workgroup per CU) run four per SIMD within
// 128 registers (a few spill).  The Q4_K kernels' 150 KB of LDS allow one 8-wave workgroup
// per CU whatever the registers.
template <int TYPE, int MODE>
__global__ void __launch_bounds__(TYPE == kTypeQ6K ? 1024 : 512)
    __attribute__((amdgpu_waves_per_eu(TYPE == kTypeQ6K ? 4 : 1, 8)))
gemm_skinny_kernel(GemmArgs g) {
    __shared__ __align__(16) SkLds<TYPE, sk_rows_per_wave<TYPE, MODE>() / 16> L;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    if ((int)blockIdx.y >= g.tiles[-1]) return;
    const int tl = g.tiles[blockIdx.y];
    const int e = tl >> 16, nt = tl & 0xFFFF;
    const int n_rows = g.counts[e], row_base = g.offsets[e], j0 = nt * kGroupTile;
    const int nvalid = min(kGroupTile, n_rows - j0);
    // one instantiation per count of 16-row column tiles, so every MFMA is unconditional
    switch ((nvalid + 15) >> 4) {
    case 1: sk_tile<TYPE, MODE, 1>(g, L, wave, lane, tid, e, j0, n_rows, row_base); break;
    case 2: sk_tile<TYPE, MODE, 2>(g, L, wave, lane, tid, e, j0, n_rows, row_base); break;
    case 3: sk_tile<TYPE, MODE, 3>(g, L, wave, lane, tid, e, j0, n_rows, row_base); break;
    default: sk_tile<TYPE, MODE, 4>(g, L, wave, lane, tid, e, j0, n_rows, row_base); break;
    }
}

// Grouped launches used by the MoE prefill path (moe.hip): tiles[] and the routing arrays
// live in device memory, the grid covers max_tiles tile-list entries.
int launch_gemm_grouped(int type, int swiglu, const void *experts, size_t expert_stride, size_t w_off,
                        size_t w_off2, StagedAct act, const int *counts, const int *offsets, const int *perm,
                        const int *tiles, int max_tiles, float *out, int out_ld, int M, int K, hipStream_t stream) {
    GemmArgs g{};
    g.W = (const uint8_t *)experts;
    g.A = act.q8;
    g.a_rho = act.rho;
    g.a_ds = act.ds;
    g.a_dlast = act.dlast;
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
    if (swiglu && type != kTypeQ4K)
        return set_error(kErrUnsupportedType, "grouped gate/up GEMM: Q4_K only (type %d)", type);
#define MNEMO_SKINNY(T_, M_)                                                                                    \
    do {                                                                                                        \
        const int rows = sk_rows_per_wave<T_, M_>() / (M_ == 1 ? 2 : 1) * sk_waves<T_>();                      \
        hipLaunchKernelGGL((gemm_skinny_kernel<T_, M_>), dim3((M + rows - 1) / rows, max_tiles, 1),            \
                           dim3(64 * sk_waves<T_>()),                                                          \
                           0, stream, g);                                                                       \
    } while (0)
    if (swiglu) MNEMO_SKINNY(kTypeQ4K, 1);
    else if (type == kTypeQ4K) MNEMO_SKINNY(kTypeQ4K, 2);
    else MNEMO_SKINNY(kTypeQ6K, 2);
#undef MNEMO_SKINNY
    return check_launch("gemm_grouped");
}

}  // namespace mnemo
