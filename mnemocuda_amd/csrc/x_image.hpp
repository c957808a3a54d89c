// x_image.hpp -- the GEMV's image of the input vector x (decode GEMVs, gemv.hip; the
// router builds the same image of the normed x for the MoE gate/up launch, router.hip).
//
// Per 32-element sub-block: u = amax/32767 and q = rne(x/u), stored as its signed high byte
// d1 and unsigned low byte d2 (x ~= u * (256*d1 + d2), |x - xhat| <= amax/65534), with fp32
// sums of x per 32 and per 16 elements.
#pragma once

#include "mnemo_common.hpp"

namespace mnemo {

// LDS image of x for a padded length kp (multiple of 256):
//   int8 d1[kp + 128] | uint8 d2[kp + 128] | float u[kp/32] | float s32[kp/32] | float s16[kp/16]
// The digit planes are stored in 16-byte words, interleaved by 128-column chunk: column c
// lives in word ((c % 128) / 16) * (kp/128 + 1) + c / 128.  Lane ul reads chunk ul, so the
// 16-byte reads of one instruction hit consecutive words (no bank conflicts); the +1
// skew keeps the 4-byte writes of the preparation conflict-free as well.
struct XLds {
    int8_t *d1;
    int8_t *d2;
    float *u;
    float *s32;
    float *s16;
    int nch1;  // 128-column chunks + 1
    __device__ XLds(uint8_t *base, int kp)
        : d1((int8_t *)base), d2((int8_t *)(base + kp + 128)), u((float *)(base + 2 * kp + 256)),
          s32((float *)(base + 2 * kp + 256 + kp / 8)), s16((float *)(base + 2 * kp + 256 + kp / 4)),
          nch1(kp / 128 + 1) {}
    // byte offset of column c (c % 16 == 0 gives a 16-byte aligned word)
    __device__ __forceinline__ int off(int c) const {
        return ((((c & 127) >> 4) * nch1 + (c >> 7)) << 4) + (c & 15);
    }
};

__host__ __device__ constexpr size_t xlds_bytes(int kp) { return (size_t)2 * kp + 256 + kp / 2; }

__device__ __forceinline__ float silu_mul(float g, float u) {
    // silu(g) * u, the reference's expression (kernels.cu:686-687)
    return g / (1.0f + expf(-g)) * u;
}

template <int XPT>  // float4 of x per thread: kp <= 4 * XPT * (threads building the image)
struct XRegs {
    float4 v[XPT];
};

__device__ __forceinline__ uint32_t umax_dpp8(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppXor1, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppXor2, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppRowHalfMirror, 0xF, 0xF, false));
    return v;
}

// The digit planes and sums of the elements held by tid (one of NT threads); no barrier.
template <int XPT, int XM, int NT>
__device__ __forceinline__ void build_x(const XRegs<XPT> &R, const XRegs<XPT> &R2, int n, int kp, const XLds &X,
                                        int tid) {
    const int lane = lane_id();
    constexpr float kMagic = 12582912.0f;  // 1.5 * 2^23: adding it rounds to an integer (RNE)
    const bool ragged = (n & 3) != 0;      // uniform (the host rejects ragged n for XM == 2)

#pragma unroll
    for (int i = 0; i < XPT; i++) {
        // computed unconditionally (a load used only under a branch would be sunk into it,
        // behind the weight loads); only the stores are guarded
        const int e4 = tid + i * NT;
        const bool store = 4 * e4 < kp;  // uniform per 8-lane group: kp is a multiple of 256
        const int e = 4 * e4;
        float v[4] = {R.v[i].x, R.v[i].y, R.v[i].z, R.v[i].w};
        if (XM != 0) {
            const float g[4] = {R2.v[i].x, R2.v[i].y, R2.v[i].z, R2.v[i].w};
#pragma unroll
            for (int j = 0; j < 4; j++) v[j] = XM == 1 ? silu_mul(v[j], g[j]) : v[j] * g[j];
        }
        if (ragged) {
            // element e+j sits at v[j + sh], sh = e - min(e, n-4) (non-zero only in the last
            // partial group); elements >= n are zero
            const int sh = e - min(e, n - 4);
            float t[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int k = min(j + sh, 3);
                float a = v[3];
                a = k == 2 ? v[2] : a;
                a = k == 1 ? v[1] : a;
                a = k == 0 ? v[0] : a;
                t[j] = e + j < n ? a : 0.0f;
            }
#pragma unroll
            for (int j = 0; j < 4; j++) v[j] = t[j];
        } else if (n != kp) {  // uniform: columns n .. kp-1 of the last super-block are zero
            const uint32_t keep = e < n ? ~0u : 0u;
#pragma unroll
            for (int j = 0; j < 4; j++) v[j] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v[j]) & keep);
        }
        // max |v| over the 8 lanes of the sub-block (|v| as float max3 with abs modifiers:
        // two instructions; non-negative floats order like their bits for the DPP max)
        const float a4 = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
        const float amax = __builtin_bit_cast(float, umax_dpp8(__builtin_bit_cast(uint32_t, a4)));
        const float u = amax * (1.0f / 32767.0f);
        const float inv = amax > 0.0f ? 32767.0f * __builtin_amdgcn_rcpf(amax) : 0.0f;
        // q = rne(v * inv): |v * inv| <= 32767 (1 + 2^-22), so |q| <= 32767.  The low half of
        // (t + magic) is q in two's complement: byte 1 is the signed digit d1 = q >> 8, byte 0
        // the unsigned digit d2 = q & 255, and q = 256 d1 + d2.
        uint32_t b1[4];
        float s4 = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            b1[j] = __builtin_bit_cast(uint32_t, fmaf(v[j], inv, kMagic));
            s4 += v[j];
        }
        // gather bytes: selector byte k picks byte sel_k of {src0 (4..7), src1 (0..3)}
        const uint32_t w1 = __builtin_amdgcn_perm(b1[1], b1[0], 0x0C0C0501u) |
                            __builtin_amdgcn_perm(b1[3], b1[2], 0x05010C0Cu);
        const uint32_t w2 = __builtin_amdgcn_perm(b1[1], b1[0], 0x0C0C0400u) |
                            __builtin_amdgcn_perm(b1[3], b1[2], 0x04000C0Cu);
        const float s16 = sum4(s4);                             // 4 lanes x 4 = 16 elements
        const float s32 = s16 + dpp_f<kDppRowHalfMirror>(s16);  // 8 lanes = 32 elements
        if (store) {
            const int o = X.off(e);
            *(uint32_t *)(X.d1 + o) = w1;
            *(uint32_t *)(X.d2 + o) = w2;
            if ((lane & 7) == 0) {
                X.u[e >> 5] = u;
                X.s32[e >> 5] = s32;
            }
            if ((lane & 3) == 0) X.s16[e >> 4] = s16;
        }
    }
}

}  // namespace mnemo
