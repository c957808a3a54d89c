// gemm.hip -- Q4_K / Q6_K x Q8_1 GEMM for prefill and batched experts (gfx950 MFMA).
//
// Semantics (MnemoCUDA gemm_q4k.cu:103-112, 164-166, 194):
//   out[j*M + i] = sum_k deq(W)[i][k] * deq(A)[j][k]
// with W GGUF blocks [M][K] and A the Q8_1 MMQ activations [N][K/128] x 144 B.
//
// Design: both operands are dequantised on the fly into f16 tiles in LDS and multiplied
// with v_mfma_f32_16x16x32_f16 (fp32 accumulate).  The per-32 scales of both operands are
// thereby folded into the values, so the MFMA accumulates across the whole K without a
// per-sub-block fp32 rescale (an int8 MFMA would need one cvt + two FMAs per output per
// 32-K step, several times the MFMA time in VALU work).
//   * W value w = d*sc*q - dmin*m (Q4_K) or d*sc*(q-32) (Q6_K) is computed exactly in fp32
//     and rounded once to f16; A value d8*q8 is formed in packed f16 arithmetic
//     (q8 exact, one rounding of the product).  Expected relative L2 error vs the fp64
//     product: ~4e-4 (two independent f16 roundings).
//   * Workgroup tile 128 weight rows x 128 tokens (4 waves of 64 x 64 = 4 x 4 MFMA tiles),
//     K step 64 (one Q4_K nibble group, one Q6_K ql group, half a Q8_1 block).  The raw
//     blocks of each step are prefetched three steps ahead into registers; f16 tiles are
//     double-buffered in LDS (XOR-swizzled, conflict-free); one barrier per step.
//   * When the tile grid covers less than half of the CUs, K is split across workgroups
//     and the partial tiles are summed with fp32 atomics into the output, which a small
//     fill kernel zeroes first.
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
// Each thread owns one row (weights) / one token (activations) and one half (32 values)
// of the 64-wide K step.
struct RawW {
    uint4 a, b, c, d;  // Q4_K: a = header, b = 16 qs bytes;  Q6_K: a,b = 32 ql, c,d = 32 qh
    uint32_t s, dd;    // Q6_K: two int8 scales, f16 d
};
struct RawA {
    uint4 a, b;   // 32 int8
    uint32_t ds;  // half2 (d, d*sum)
};

// Q4_K step ks = super-block ks/4, nibble group g = ks%4 (qs bytes 32g..32g+31); half h
// takes bytes 32g+16h .. +15: 16 weights of sub-block 2g (low nibbles) and 16 of 2g+1.
__device__ __forceinline__ void load_w_q4k(const uint8_t *__restrict__ wrow, int ks, int h, RawW &r) {
    const uint8_t *blk = wrow + (size_t)(ks >> 2) * kQ4KBytes;
    r.a = ld16(blk);
    r.b = ld16(blk + 16 + 32 * (ks & 3) + 16 * h);
}

// Q6_K step ks covers values 64*(ks%4) .. +63 of super-block ks/4: half hh = (ks%4)/2,
// groups 2(ks%2) and 2(ks%2)+1; half h takes group grp = 2(ks%2) + h, i.e. ql bytes
// [64hh + 32h, +32) (low nibbles if grp < 2, else high) and qh bytes [32hh, +32) at 2grp.
__device__ __forceinline__ void load_w_q6k(const uint8_t *__restrict__ wrow, int ks, int h, RawW &r) {
    const uint8_t *blk = wrow + (size_t)(ks >> 2) * kQ6KBytes;
    const int g = ks & 3, hh = g >> 1, grp = 2 * (g & 1) + h;
    r.a = ld16(blk + 64 * hh + 32 * h);
    r.b = ld16(blk + 64 * hh + 32 * h + 16);
    r.c = ld16(blk + 128 + 32 * hh);
    r.d = ld16(blk + 128 + 32 * hh + 16);
    uint16_t s, dd;
    __builtin_memcpy(&s, blk + 192 + 8 * hh + 2 * grp, 2);
    __builtin_memcpy(&dd, blk + 208, 2);
    r.s = s;
    r.dd = dd;
}

// Activations of step ks, half h: values 64ks + 32h .. +31 = one Q8_1 sub-block.
__device__ __forceinline__ void load_a(const uint8_t *__restrict__ arow, int ks, int h, RawA &r) {
    const int v0 = ks * kKS + 32 * h;
    const uint8_t *blk = arow + (size_t)(v0 >> 7) * kQ81Bytes;
    const int sub = (v0 >> 5) & 3;
    r.ds = *(const uint32_t *)(blk + 4 * sub);
    r.a = ld16(blk + 16 + 32 * sub);
    r.b = ld16(blk + 32 + 32 * sub);
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
// Q4_K: half h of step ks holds 16 weights of sub-block 2g (K columns 16h .. 16h+15 of the
// step: chunks 2h, 2h+1) and 16 of sub-block 2g+1 (columns 32+16h ..: chunks 4+2h, 5+2h).
__device__ __forceinline__ void store_w_q4k(const RawW &r, int ks, int h, _Float16 *tile, int row) {
    const int g = ks & 3;
    const uint32_t s0 = r.a.y, s1 = r.a.z, s2 = r.a.w;
    uint32_t sc0, m0, sc1, m1;
    if (g < 2) {  // uniform per step
        const int sh = 16 * g;
        sc0 = (s0 >> sh) & 63; m0 = (s1 >> sh) & 63;
        sc1 = (s0 >> (sh + 8)) & 63; m1 = (s1 >> (sh + 8)) & 63;
    } else {
        const int sh = 16 * (g - 2);
        sc0 = ((s2 >> sh) & 15) | (((s0 >> (sh + 6)) & 3) << 4);
        m0 = ((s2 >> (sh + 4)) & 15) | (((s1 >> (sh + 6)) & 3) << 4);
        sc1 = ((s2 >> (sh + 8)) & 15) | (((s0 >> (sh + 14)) & 3) << 4);
        m1 = ((s2 >> (sh + 12)) & 15) | (((s1 >> (sh + 14)) & 3) << 4);
    }
    const float d = h2f(r.a.x & 0xFFFFu), dmin = h2f(r.a.x >> 16);
    const float a0 = d * (float)sc0, b0 = dmin * (float)m0;
    const float a1 = d * (float)sc1, b1 = dmin * (float)m1;
    const uint32_t w[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t ml = w[k] & 0x0F0F0F0Fu, mh = (w[k] >> 4) & 0x0F0F0F0Fu;
        // (float)(byte j of a masked dword) compiles to v_cvt_f32_ubyte{j}
        lo[2 * k] = pack_h2(fmaf(a0, (float)(ml & 0xFF), -b0), fmaf(a0, (float)((ml >> 8) & 0xFF), -b0));
        lo[2 * k + 1] = pack_h2(fmaf(a0, (float)((ml >> 16) & 0xFF), -b0), fmaf(a0, (float)(ml >> 24), -b0));
        hi[2 * k] = pack_h2(fmaf(a1, (float)(mh & 0xFF), -b1), fmaf(a1, (float)((mh >> 8) & 0xFF), -b1));
        hi[2 * k + 1] = pack_h2(fmaf(a1, (float)((mh >> 16) & 0xFF), -b1), fmaf(a1, (float)(mh >> 24), -b1));
    }
    put16(tile, row, 2 * h, lo[0], lo[1], lo[2], lo[3]);
    put16(tile, row, 2 * h + 1, lo[4], lo[5], lo[6], lo[7]);
    put16(tile, row, 4 + 2 * h, hi[0], hi[1], hi[2], hi[3]);
    put16(tile, row, 5 + 2 * h, hi[4], hi[5], hi[6], hi[7]);
}

// Q6_K: half h of step ks = group 2(ks%2) + h, K columns 32h .. 32h+31 (chunks 4h .. 4h+3).
__device__ __forceinline__ void store_w_q6k(const RawW &r, int ks, int h, _Float16 *tile, int row) {
    const int grp = 2 * (ks & 1) + h;
    const float d = h2f(r.dd);
    const float s0 = d * (float)(int8_t)(r.s & 0xFF), s1 = d * (float)(int8_t)(r.s >> 8);
    const uint32_t ql[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
    const uint32_t qh[8] = {r.c.x, r.c.y, r.c.z, r.c.w, r.d.x, r.d.y, r.d.z, r.d.w};
    const int shl = grp >= 2 ? 4 : 0;
    uint32_t o[16];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        // 6-bit q in bits 0..5 of each byte
        const uint32_t lo = (ql[k] >> shl) & 0x0F0F0F0Fu;
        const uint32_t hi = (2 * grp <= 4 ? (qh[k] << (4 - 2 * grp)) : (qh[k] >> (2 * grp - 4))) & 0x30303030u;
        const uint32_t q = lo | hi;
        const float s = k < 4 ? s0 : s1;
        o[2 * k] = pack_h2(s * (float)((int)(q & 0xFF) - 32), s * (float)((int)((q >> 8) & 0xFF) - 32));
        o[2 * k + 1] = pack_h2(s * (float)((int)((q >> 16) & 0xFF) - 32), s * (float)((int)(q >> 24) - 32));
    }
#pragma unroll
    for (int k = 0; k < 4; k++) put16(tile, row, 4 * h + k, o[4 * k], o[4 * k + 1], o[4 * k + 2], o[4 * k + 3]);
}

// d8 * q8 in packed f16: q8 ^ 0x80 placed under the exponent byte 0x64 is 1024 + q8 + 128
// exactly; subtracting 1152 gives q8 exactly; the product with d8 is rounded once.
// Half h: K columns 32h .. 32h+31 (chunks 4h .. 4h+3).
__device__ __forceinline__ void store_a(const RawA &r, int h, _Float16 *tile, int row) {
    const h2 d2 = {__builtin_bit_cast(_Float16, (uint16_t)(r.ds & 0xFFFF)),
                   __builtin_bit_cast(_Float16, (uint16_t)(r.ds & 0xFFFF))};
    const h2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
    uint32_t o[16];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t u = w[k] ^ 0x80808080u;
        const uint32_t e01 = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // [u0, 64, u1, 64]
        const uint32_t e23 = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // [u2, 64, u3, 64]
        const h2 q01 = __builtin_bit_cast(h2, e01) + off, q23 = __builtin_bit_cast(h2, e23) + off;
        o[2 * k] = __builtin_bit_cast(uint32_t, q01 * d2);
        o[2 * k + 1] = __builtin_bit_cast(uint32_t, q23 * d2);
    }
#pragma unroll
    for (int k = 0; k < 4; k++) put16(tile, row, 4 * h + k, o[4 * k], o[4 * k + 1], o[4 * k + 2], o[4 * k + 3]);
}

// ------------------------------------------------------------------ kernel
// Workgroup of 4 waves computes a 128 x 128 tile (weights x tokens) over one K slice
// (blockIdx.z of `splits`); wave w owns rows 64*(w%2) .. +63 and tokens 64*(w/2) .. +63
// (4 x 4 MFMA tiles).  Raw blocks are prefetched kPF-1 steps ahead into a ring of
// registers (the loop is unrolled by kPF so every ring index is static and the waits the
// compiler inserts count exactly the outstanding steps).  With splits > 1 the partial
// tiles are added into the (pre-zeroed) output with fp32 atomics, in an order that may
// differ from run to run.
constexpr int kThreads = 256;
constexpr int kBM = 128, kBN = 128;
constexpr int kPF = 4;

template <int TYPE>
__device__ __forceinline__ void load_step(const uint8_t *wrow, const uint8_t *arow, int ks, int h, RawW &rw,
                                          RawA &ra) {
    if (TYPE == kTypeQ4K) load_w_q4k(wrow, ks, h, rw);
    else load_w_q6k(wrow, ks, h, rw);
    load_a(arow, ks, h, ra);
}

template <int TYPE>
__device__ __forceinline__ void store_step(const RawW &rw, const RawA &ra, int ks, int h, _Float16 *at,
                                           _Float16 *bt, int row) {
    if (TYPE == kTypeQ4K) store_w_q4k(rw, ks, h, at, row);
    else store_w_q6k(rw, ks, h, at, row);
    store_a(ra, h, bt, row);
}

__device__ __forceinline__ void mfma_step(const _Float16 *as, const _Float16 *bs, int wi, int wj, int lane,
                                          f4 (&acc)[4][4]) {
#pragma unroll
    for (int kk = 0; kk < 2; kk++) {
        h8 af[4], bf[4];
        const int chunk = 4 * kk + (lane >> 4);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int ra = wi + 16 * t + (lane & 15), rb = wj + 16 * t + (lane & 15);
            af[t] = *(const h8 *)(as + tile_off(ra, chunk));
            bf[t] = *(const h8 *)(bs + tile_off(rb, chunk));
        }
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int b = 0; b < 4; b++)
                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[a], bf[b], acc[a][b], 0, 0, 0);
    }
}

template <int TYPE, bool ATOMIC>
__global__ void __launch_bounds__(kThreads) gemm_q8_1_kernel(const uint8_t *__restrict__ W,
                                                              const uint8_t *__restrict__ A,
                                                              float *__restrict__ out, int M, int K, int N,
                                                              int splits) {
    __shared__ __align__(16) _Float16 lds[2][2][kBM * kKS];  // [buffer][weights | tokens]
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int i0 = blockIdx.x * kBM, j0 = blockIdx.y * kBN;
    const int wi = (wave & 1) * 64, wj = (wave >> 1) * 64;
    const size_t wrow_bytes = (size_t)(K / 256) * (TYPE == kTypeQ4K ? kQ4KBytes : kQ6KBytes);
    const size_t arow_bytes = (size_t)(K / 128) * kQ81Bytes;
    const int nks_all = K / kKS;
    const int ks0 = (int)((long)nks_all * blockIdx.z / splits);
    const int ks1 = (int)((long)nks_all * (blockIdx.z + 1) / splits);
    const int last = ks1 - 1;

    // loader role: thread -> (row/token lr, half lh); rows past the end re-read the last
    const int lr = tid >> 1, lh = tid & 1;
    const uint8_t *wrow = W + (size_t)min(i0 + lr, M - 1) * wrow_bytes;
    const uint8_t *arow = A + (size_t)min(j0 + lr, N - 1) * arow_bytes;

    f4 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};

    RawW rw[kPF];
    RawA ra[kPF];
    // prologue: steps ks0 .. ks0+kPF-2 in flight (clamped to the last step, unconditional)
#pragma unroll
    for (int p = 0; p < kPF - 1; p++) load_step<TYPE>(wrow, arow, min(ks0 + p, last), lh, rw[p], ra[p]);
    store_step<TYPE>(rw[0], ra[0], ks0, lh, lds[0][0], lds[0][1], lr);
    __syncthreads();

    for (int kb = ks0; kb < ks1; kb += kPF) {
#pragma unroll
        for (int p = 0; p < kPF; p++) {
            const int ks = kb + p;
            if (ks < ks1) {  // uniform
                load_step<TYPE>(wrow, arow, min(ks + kPF - 1, last), lh, rw[(p + kPF - 1) % kPF],
                                ra[(p + kPF - 1) % kPF]);
                const int cur = (ks - ks0) & 1;
                mfma_step(lds[cur][0], lds[cur][1], wi, wj, lane, acc);
                if (ks + 1 < ks1)
                    store_step<TYPE>(rw[(p + 1) % kPF], ra[(p + 1) % kPF], ks + 1, lh, lds[cur ^ 1][0],
                                     lds[cur ^ 1][1], lr);
                __syncthreads();
            }
        }
    }
    // D layout (16x16 f32): lane l holds rows 4*(l/16)+e, column l%16.  Rows index
    // weights i (A operand), columns tokens j (B operand).
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int j = j0 + wj + 16 * b + (lane & 15);
            const int ib = i0 + wi + 16 * a + 4 * (lane >> 4);
            if (j >= N) continue;
            float *o = out + (size_t)j * M + ib;
            if (ATOMIC) {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (ib + e < M) __hip_atomic_fetch_add(o + e, acc[a][b][e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else if (ib + 3 < M && ((M & 3) == 0)) {
                *(f4 *)o = acc[a][b];
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (ib + e < M) o[e] = acc[a][b][e];
            }
        }
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
    // split K only while the tile grid covers less than half of the CUs (the atomics cost
    // more than idle CUs otherwise), keeping at least 16 steps of 64 per split
    const int nks = K / kKS;
    int splits = 1;
    while (2 * tm * tn * splits < device_cus_gemm() && nks / (splits * 2) >= 16) splits *= 2;
    const size_t lds = 0;
    dim3 grid(tm, tn, splits);
    if (splits > 1) {
        const long n = (long)M * N;
        if (n % 4 != 0) return set_error(kErrBadArg, "gemm: M*N must be a multiple of 4 for split-K");
        hipLaunchKernelGGL(zero_kernel, dim3((unsigned)std::min<long>((n / 4 + 255) / 256, 4096)), dim3(256), 0,
                           stream, (float4 *)out, n / 4);
    }
#define MNEMO_GEMM_LAUNCH(T_, A_)                                                                          \
    hipLaunchKernelGGL((gemm_q8_1_kernel<T_, A_>), grid, dim3(kThreads), lds, stream, (const uint8_t *)w, \
                       (const uint8_t *)act, out, M, K, N, splits)
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

}  // namespace mnemo
