// mnemo_common.hpp -- shared device helpers for the gfx950 (CDNA4) kernels.
//
// GGUF block geometry (MnemoCUDA kernels.cu:20-32, gemm_q4k.cu:19-33):
//   Q4_K : 144 B / 256 weights  = f16 d | f16 dmin | 12 B packed 6-bit (sc, m) | 128 B nibbles
//   Q6_K : 210 B / 256 weights  = ql[128] | qh[64] | int8 scales[16] | f16 d
//   Q8_1 (MMQ) : 144 B / 128 values = 4 x (half d, half d*sum) | 128 int8
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mnemo {

constexpr int kQK = 256;
constexpr int kQ4KBytes = 144;
constexpr int kQ6KBytes = 210;
constexpr int kQ81Bytes = 144;
constexpr int kTypeF32 = 0;
constexpr int kTypeQ4K = 12;
constexpr int kTypeQ6K = 14;

// ---------------------------------------------------------------- loads
// Weight super-blocks are only 2-byte aligned for Q6_K (210 B stride).  gfx950 global
// memory accepts unaligned dword accesses, so a 16-byte memcpy compiles to one
// global_load_dwordx4 regardless of alignment.
__device__ __forceinline__ uint4 ld16(const uint8_t *p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}
// N 16-byte words from a 2-byte aligned address p.  Q6_K blocks are 210 B, so every other
// block starts at 2 mod 4, and on gfx950 a 16-byte load from an address that is not 4-byte
// aligned streams at ~2/3 of the aligned rate.  The words are loaded from the 4-byte
// aligned address at or below p, plus one dword, and shifted into place with v_alignbyte.
// Reads stay inside [p - 2, p + 16N): with p 4-byte aligned the extra dword is the last
// one of the range again (unused).
template <int N>
__device__ __forceinline__ void ld16_a2(const uint8_t *p, uint4 (&out)[N]) {
    const uint32_t sh = (uint32_t)(uintptr_t)p & 2u;
    const uint32_t *a = (const uint32_t *)(p - sh);
    uint32_t w[4 * N + 1];
#pragma unroll
    for (int i = 0; i < N; i++) __builtin_memcpy(&w[4 * i], a + 4 * i, 16);
    w[4 * N] = a[4 * N - (sh ? 0 : 1)];
#pragma unroll
    for (int i = 0; i < N; i++) {
        out[i].x = __builtin_amdgcn_alignbyte(w[4 * i + 1], w[4 * i], sh);
        out[i].y = __builtin_amdgcn_alignbyte(w[4 * i + 2], w[4 * i + 1], sh);
        out[i].z = __builtin_amdgcn_alignbyte(w[4 * i + 3], w[4 * i + 2], sh);
        out[i].w = __builtin_amdgcn_alignbyte(w[4 * i + 4], w[4 * i + 3], sh);
    }
}
__device__ __forceinline__ uint4 ld16_a2(const uint8_t *p) {
    uint4 o[1];
    ld16_a2<1>(p, o);
    return o[0];
}

__device__ __forceinline__ uint2 ld8(const uint8_t *p) {
    uint2 v;
    __builtin_memcpy(&v, p, 8);
    return v;
}
// 8 bytes from a 2-byte aligned address: three aligned dwords at or below p, shifted into
// place (reads stay inside [p - 2, p + 10)).
__device__ __forceinline__ uint2 ld8_a2(const uint8_t *p) {
    const uint32_t sh = (uint32_t)(uintptr_t)p & 2u;
    const uint32_t *a = (const uint32_t *)(p - sh);
    uint32_t w[3];
    __builtin_memcpy(&w[0], a, 8);
    w[2] = a[sh ? 2 : 1];
    return make_uint2(__builtin_amdgcn_alignbyte(w[1], w[0], sh), __builtin_amdgcn_alignbyte(w[2], w[1], sh));
}

__device__ __forceinline__ uint4 ld16_nt(const uint8_t *p) {
    // streaming weights: read once per call, do not keep them in the caches
    uint4 v;
    v.x = __builtin_nontemporal_load((const uint32_t *)p + 0);
    v.y = __builtin_nontemporal_load((const uint32_t *)p + 1);
    v.z = __builtin_nontemporal_load((const uint32_t *)p + 2);
    v.w = __builtin_nontemporal_load((const uint32_t *)p + 3);
    return v;
}

// ---------------------------------------------------------------- f16
__device__ __forceinline__ float h2f(uint32_t bits16) {
    _Float16 h;
    uint16_t b = (uint16_t)bits16;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}
__device__ __forceinline__ uint16_t f2h_bits(float f) {
    _Float16 h = (_Float16)f;  // v_cvt_f16_f32: round to nearest even
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}

// ---------------------------------------------------------------- DPP wave reductions
// quad_perm / row controls of the gfx9 DPP encoding.
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
constexpr int kDppRowBcast15 = 0x142;
constexpr int kDppRowBcast31 = 0x143;

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, false));
}

// Sum over aligned groups of 4 lanes; every lane of the group gets the sum.
__device__ __forceinline__ float sum4(float v) {
    v += dpp_f<kDppXor1>(v);
    v += dpp_f<kDppXor2>(v);
    return v;
}
// Sum over aligned groups of 16 lanes (one DPP row); every lane gets the sum.
__device__ __forceinline__ float sum16(float v) {
    v = sum4(v);
    v += dpp_f<kDppRowHalfMirror>(v);
    v += dpp_f<kDppRowMirror>(v);
    return v;
}
// Full 64-lane sum; valid in lane 63 only.
__device__ __forceinline__ float sum64_lane63(float v) {
    v = sum16(v);
    v += dpp_f<kDppRowBcast15, 0xA>(v);
    v += dpp_f<kDppRowBcast31, 0xC>(v);
    return v;
}

// The top-k order of the router: value descending, ties to the lower index.
__device__ __forceinline__ bool better(float v, int i, float v2, int i2) {
    return (v > v2) || (v == v2 && i < i2);
}

// the sum (max) of v over the wave, in every lane
__device__ __forceinline__ float wave_sum_all(float v) {
    v = sum64_lane63(v);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ float wave_max_all(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

// Sum over aligned 32-lane halves; valid in lanes 31 and 63.
__device__ __forceinline__ float sum32_lane31(float v) {
    v = sum16(v);
    v += dpp_f<kDppRowBcast15, 0xA>(v);
    return v;
}
// Max over aligned groups of 8 lanes; every lane of the group gets the max.
__device__ __forceinline__ float max8(float v) {
    v = fmaxf(v, dpp_f<kDppXor1>(v));
    v = fmaxf(v, dpp_f<kDppXor2>(v));
    v = fmaxf(v, dpp_f<kDppRowHalfMirror>(v));
    return v;
}
// Max over aligned groups of 16 lanes (one DPP row); every lane gets the max.
__device__ __forceinline__ float max16(float v) {
    v = max8(v);
    return fmaxf(v, dpp_f<kDppRowMirror>(v));
}

__device__ __forceinline__ int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0)); }

// signed 4 x int8 dot product accumulate (v_dot4_i32_i8)
__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Workgroup barrier for LDS hand-offs that leaves global loads in flight.  __syncthreads()
// is a release/acquire fence plus s_barrier, and the release makes every wave wait for all
// of its outstanding global loads (vmcnt(0)) -- loads that the barrier does not protect
// included, so every wave then waits for the slowest wave's data.  Here only the wave's own
// LDS accesses (lgkmcnt) are waited for; the asm's memory clobber keeps the compiler from
// moving memory accesses across it, and the compiler still waits for each load before the
// first use of its registers.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

}  // namespace mnemo
