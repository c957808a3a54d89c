// gemv.hip -- dequant-fused Q4_K / Q6_K matrix-vector products for decode (gfx950).
//
// One kernel serves every GEMV entry point of the reference (MnemoCUDA kernels.cu:66
// matvec_q4k, :149 _add, :205 _qkv, :278 _dual, :358 _scaled_add, :427 matvec_q6k):
// up to three weight matrices that share one input vector x are processed as one
// concatenated row space, each with its own GGUF type and epilogue
// (store | store + residual | y += scale * acc).
//
// Design (CDNA4, wave64):
//  * x is re-expressed per 32-element sub-block as a 16-bit integer in two bytes,
//      x ~= u * (256*d1 + d2),  u = amax/32767,  |x - xhat| <= amax/65534,
//    d1 the signed high byte and d2 the unsigned low byte of rne(x/u),
//    held in LDS together with fp32 sums of x per 32 and per 16 elements.  Each
//    workgroup (512 threads, two per CU) builds this image once for all of its rows.
//    Weight nibbles / 6-bit values (unsigned) are multiplied with v_dot4_i32_i8 (high
//    bytes) and v_dot4_u32_u8 (low bytes), 4 MACs per instruction, and the integer
//    partial of each sub-block is rescaled
//    in fp32:
//      Q4_K: w = d*sc*q - dmin*m   ->  acc += d*sc*u*I - dmin*m*sum32(x)
//      Q6_K: w = d*sc*(q-32)       ->  acc += d*sc*(u*I - 32*sum16(x))
//  * A lane owns one half super-block of a row (128 weights: 64 B of Q4_K nibbles plus the
//    16 B header, or 64 B ql + 32 B qh + 8 scale bytes + d of Q6_K), loaded with 16-byte
//    global loads; a row spans LPR = pow2ceil(K/128) <= 64 lanes, short rows put
//    P = 64/LPR rows in one wave pass.  The row sum is a DPP reduction.
//  * The x loads go out first, then the weight loads of the wave's first two passes, so
//    the x image is built while the weights are in flight.  Every load sits on a
//    branch-free path (addresses clamped, results masked) so that the compiler's waits
//    count exactly the loads a value depends on.
#include <climits>

#include "mnemo_common.hpp"
#include "mnemo_internal.hpp"
#include "x_image.hpp"

namespace mnemo {
// This file is compiled once per workgroup size (MNEMO_GEMV_THREADS) into the namespace
// MNEMO_GEMV_NS; gemv_launch.hip picks the variant per launch.
#ifndef MNEMO_GEMV_NS
#define MNEMO_GEMV_NS g512
#endif
namespace MNEMO_GEMV_NS {

#ifndef MNEMO_GEMV_THREADS
#define MNEMO_GEMV_THREADS 512
#endif
constexpr int kGemvThreads = MNEMO_GEMV_THREADS;
static_assert(kGemvThreads >= 256 && kGemvThreads <= 1024 && kGemvThreads % 64 == 0, "x image staging assumes 256..1024 threads");
// float4 of x per thread for rows of up to kp_max columns
constexpr int xpt_for(int kp_max) { return (kp_max + 4 * kGemvThreads - 1) / (4 * kGemvThreads); }

// ------------------------------------------------------------------ x preparation
// (the image layout, XLds, and build_x are in x_image.hpp: the router builds the same image)

// One 16-byte load per 4 elements from e clamped to n-4 (x may be unaligned; the host
// rejects n < 4), so the instruction sequence is fixed.
// XM: 0 x as given; 1 silu(x) * x2 (SwiGLU inputs); 2 rms_norm(x) * x2 (x2 = norm weight)
// NT threads share the image (the workgroup, or one wave); tid is the caller's index among them.
template <int XPT, int XM, int NT = kGemvThreads>
__device__ __forceinline__ void load_x(const float *__restrict__ x0, const float *__restrict__ x1, int n,
                                       XRegs<XPT> &R, XRegs<XPT> &R2, int tid = threadIdx.x) {
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        const int e = 4 * (tid + i * NT);
        const int ec = min(e, n - 4);
        __builtin_memcpy(&R.v[i], x0 + ec, 16);
        if (XM != 0) __builtin_memcpy(&R2.v[i], x1 + ec, 16);
    }
}

// Builds the workgroup's LDS image; every thread of the block must call this (it ends in a
// barrier).  Elements at or past n (loaded from clamped addresses) are zeroed, after the
// weight loads have been issued, so that waiting for x does not wait for the weights.
// With XM == 2 the image holds the digits of x * g; the norm scale 1 / sqrt(mean(x^2) + eps)
// is uniform over x, so it multiplies the finished dot products instead (returned here).
// The waves' sums of squares go to LDS with the image and are summed after its barrier, in
// a fixed order, so the norm costs no barrier of its own.
template <int XPT, int XM>
__device__ __forceinline__ float finish_x(const XRegs<XPT> &R, const XRegs<XPT> &R2, int n, int kp, XLds X,
                                          float eps) {
    __shared__ float part[XM == 2 ? kGemvThreads / 64 : 1];
    if (XM == 2) {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            if (4 * (threadIdx.x + i * kGemvThreads) < n) {
                ss = fmaf(R.v[i].x, R.v[i].x, ss);
                ss = fmaf(R.v[i].y, R.v[i].y, ss);
                ss = fmaf(R.v[i].z, R.v[i].z, ss);
                ss = fmaf(R.v[i].w, R.v[i].w, ss);
            }
        }
        ss = sum64_lane63(ss);
        if (lane_id() == 63) part[threadIdx.x >> 6] = ss;
    }
    build_x<XPT, XM, kGemvThreads>(R, R2, n, kp, X, threadIdx.x);
    lds_barrier();  // the image only: each wave's dot products wait for its own weights
    if (XM != 2) return 1.0f;
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < kGemvThreads / 64; w++) tot += part[w];
    return __builtin_amdgcn_rsqf(tot / (float)n + eps);  // rsqrtf, as the reference (kernels.cu:718)
}

// ------------------------------------------------------------------ weight units
// Raw bytes of one half super-block (128 weights), loaded ahead of use.
//   Q4_K: h = header (d, dmin, 12 scale bytes), q[0..3] = the 64 nibble bytes of the half
//   Q6_K: h = the 16 scale bytes, q[0..3] = 64 ql bytes, qh[0..1] = 32 qh bytes, dd = f16 d
struct RawH {
    uint4 h;
    uint4 q[4];
    uint4 qh[2];
    uint32_t dd;
};

// Q4_K half hf of super-block blk: qs bytes [64hf, +64), sub-blocks 4hf .. 4hf+3
// (kernels.cu:114-136: qs pair g holds sub-block 2g in low, 2g+1 in high nibbles).
__device__ __forceinline__ void load_q4k(const uint8_t *__restrict__ blk, int hf, RawH &r) {
    r.h = ld16(blk);
#pragma unroll
    for (int i = 0; i < 4; i++) r.q[i] = ld16(blk + 16 + 64 * hf + 16 * i);
}

// Q6_K half hf: ql bytes [64hf, +64), qh bytes [128 + 32hf, +32), the 16 scale bytes at
// 192 (the half uses 8hf .. 8hf+7), d at 208 (kernels.cu:427-491;
// validate_dequant.py:253-319).
__device__ __forceinline__ void load_q6k(const uint8_t *__restrict__ blk, int hf, RawH &r) {
    ld16_a2<4>(blk + 64 * hf, r.q);
    ld16_a2<2>(blk + 128 + 32 * hf, r.qh);
    r.h = ld16_a2(blk + 192);
    uint16_t dd;
    __builtin_memcpy(&dd, blk + 208, 2);
    r.dd = dd;
}

__device__ __forceinline__ int dot16(const uint32_t (&q)[4], const int4 &d, int acc) {
    acc = sdot4((int)q[0], d.x, acc);
    acc = sdot4((int)q[1], d.y, acc);
    acc = sdot4((int)q[2], d.z, acc);
    acc = sdot4((int)q[3], d.w, acc);
    return acc;
}
// the same with the unsigned low-byte digits (the weights are unsigned as well)
__device__ __forceinline__ int dot16u(const uint32_t (&q)[4], const int4 &d, int acc) {
    acc = (int)__builtin_amdgcn_udot4(q[0], (uint32_t)d.x, (uint32_t)acc, false);
    acc = (int)__builtin_amdgcn_udot4(q[1], (uint32_t)d.y, (uint32_t)acc, false);
    acc = (int)__builtin_amdgcn_udot4(q[2], (uint32_t)d.z, (uint32_t)acc, false);
    acc = (int)__builtin_amdgcn_udot4(q[3], (uint32_t)d.w, (uint32_t)acc, false);
    return acc;
}

// Sum over the 128 weights of a Q4_K half super-block whose first column is c.
// Sub-block t of the half: nibble t%2 of qs dwords 8(t/2) .. +7.
__device__ __forceinline__ float q4k_dot(const RawH &r, int hf, int c, const XLds &X) {
    int I[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int oa = X.off(c + 32 * t), ob = X.off(c + 32 * t + 16);
        const int4 d1a = *(const int4 *)(X.d1 + oa), d1b = *(const int4 *)(X.d1 + ob);
        const int4 d2a = *(const int4 *)(X.d2 + oa), d2b = *(const int4 *)(X.d2 + ob);
        const uint4 qa = r.q[2 * (t >> 1)], qb = r.q[2 * (t >> 1) + 1];
        const int sh = 4 * (t & 1);
        const uint32_t na[4] = {(qa.x >> sh) & 0x0F0F0F0Fu, (qa.y >> sh) & 0x0F0F0F0Fu,
                                (qa.z >> sh) & 0x0F0F0F0Fu, (qa.w >> sh) & 0x0F0F0F0Fu};
        const uint32_t nb[4] = {(qb.x >> sh) & 0x0F0F0F0Fu, (qb.y >> sh) & 0x0F0F0F0Fu,
                                (qb.z >> sh) & 0x0F0F0F0Fu, (qb.w >> sh) & 0x0F0F0F0Fu};
        const int a1 = dot16(nb, d1b, dot16(na, d1a, 0));
        const int a2 = dot16u(nb, d2b, dot16u(na, d2a, 0));
        I[t] = 256 * a1 + a2;
        // one sub-block's digit reads at a time: hoisting all of them costs ~64 VGPRs and
        // occupancy.  The sched_barrier alone does not hold: the compiler sinks the
        // arithmetic below later reads; the empty asm with the sub-block's result as an
        // operand and a memory clobber pins both (62 instead of 96 VGPRs).
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" : "+v"(I[t])::"memory");
    }
    // four 6-bit scales and mins per dword: the packed form of get_scale_min_k4
    // (kernels.cu:45-53), the same unpacking as gemm_q4k.cu:53-56
    const uint32_t S0 = r.h.y, S1 = r.h.z, S2 = r.h.w;
    const uint32_t sc = hf ? ((S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u)) : (S0 & 0x3F3F3F3Fu);
    const uint32_t mm = hf ? (((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u)) : (S1 & 0x3F3F3F3Fu);
    const float4 u = *(const float4 *)(X.u + (c >> 5));
    const float4 sx = *(const float4 *)(X.s32 + (c >> 5));
    const float d = h2f(r.h.x & 0xFFFFu), dmin = h2f(r.h.x >> 16);
    float a = (float)(sc & 0xFF) * (u.x * (float)I[0]);
    a = fmaf((float)((sc >> 8) & 0xFF), u.y * (float)I[1], a);
    a = fmaf((float)((sc >> 16) & 0xFF), u.z * (float)I[2], a);
    a = fmaf((float)(sc >> 24), u.w * (float)I[3], a);
    float m = (float)(mm & 0xFF) * sx.x;
    m = fmaf((float)((mm >> 8) & 0xFF), sx.y, m);
    m = fmaf((float)((mm >> 16) & 0xFF), sx.z, m);
    m = fmaf((float)(mm >> 24), sx.w, m);
    return fmaf(d, a, -dmin * m);
}

// Sum over the 128 weights of a Q6_K half super-block (values 32g + l of the half,
// g = 0..3) whose first column is c.
__device__ __forceinline__ float q6k_dot(const RawH &r, int hf, int c, const XLds &X) {
    const uint32_t H[8] = {r.qh[0].x, r.qh[0].y, r.qh[0].z, r.qh[0].w, r.qh[1].x, r.qh[1].y, r.qh[1].z, r.qh[1].w};
    const float4 u = *(const float4 *)(X.u + (c >> 5));
    const float4 s16a = *(const float4 *)(X.s16 + (c >> 4));
    const float4 s16b = *(const float4 *)(X.s16 + (c >> 4) + 4);
    const float uu[4] = {u.x, u.y, u.z, u.w};
    const float ss[8] = {s16a.x, s16a.y, s16a.z, s16a.w, s16b.x, s16b.y, s16b.z, s16b.w};
    float acc = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        // group g: low nibbles of ql bytes 32(g&1) .. +31 (high nibbles for g >= 2), top
        // two bits at 2g of qh bytes 0..31, moved to bits 4-5 of each byte
        const uint4 la = r.q[2 * (g & 1)], lb = r.q[2 * (g & 1) + 1];
        const uint32_t L[8] = {la.x, la.y, la.z, la.w, lb.x, lb.y, lb.z, lb.w};
        uint32_t q[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t lo = (g >= 2 ? (L[k] >> 4) : L[k]) & 0x0F0F0F0Fu;
            const uint32_t hi = (2 * g <= 4 ? (H[k] << (4 - 2 * g)) : (H[k] >> (2 * g - 4))) & 0x30303030u;
            q[k] = lo | hi;
        }
        const int oa = X.off(c + 32 * g), ob = X.off(c + 32 * g + 16);
        const int4 d1a = *(const int4 *)(X.d1 + oa), d1b = *(const int4 *)(X.d1 + ob);
        const int4 d2a = *(const int4 *)(X.d2 + oa), d2b = *(const int4 *)(X.d2 + ob);
        const uint32_t qa[4] = {q[0], q[1], q[2], q[3]}, qb[4] = {q[4], q[5], q[6], q[7]};
        const int i0 = 256 * dot16(qa, d1a, 0) + dot16u(qa, d2a, 0);
        const int i1 = 256 * dot16(qb, d1b, 0) + dot16u(qb, d2b, 0);
        // scale bytes 8hf + 2g, 8hf + 2g + 1 (the 16-value groups of group g)
        const uint32_t sw = hf ? (g < 2 ? r.h.z : r.h.w) : (g < 2 ? r.h.x : r.h.y);
        const int sc0 = (int8_t)(sw >> (16 * (g & 1)));
        const int sc1 = (int8_t)(sw >> (16 * (g & 1) + 8));
        acc = fmaf((float)sc0, fmaf(uu[g], (float)i0, -32.0f * ss[2 * g]), acc);
        acc = fmaf((float)sc1, fmaf(uu[g], (float)i1, -32.0f * ss[2 * g + 1]), acc);
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" : "+v"(acc)::"memory");  // as in q4k_dot (76 instead of 112 VGPRs)
    }
    return h2f(r.dd) * acc;
}

// ------------------------------------------------------------------ the kernel
template <int LPR>
__device__ __forceinline__ float reduce_rows(float v) {
    if constexpr (LPR == 64) return sum64_lane63(v);
    else if constexpr (LPR == 32) return sum32_lane31(v);
    else if constexpr (LPR == 16) return sum16(v);
    else if constexpr (LPR == 8) {
        v = sum4(v);
        return v + dpp_f<kDppRowHalfMirror>(v);
    } else if constexpr (LPR == 4) return sum4(v);
    else return v + dpp_f<kDppXor1>(v);
}

// One wave pass: P = 64/LPR rows, each lane holding UPL half super-blocks of its row.
template <int UPL>
struct Pass {
    RawH q[UPL];
    int lrow;  // row of this lane within its matrix (clamped)
    bool valid;
};

// Matrices start at multiples of P rows in the concatenated row space (launch_gemv pads),
// so a pass never straddles two matrices and its matrix index is wave-uniform.
__device__ __forceinline__ int pass_matrix(const GemvArgs &args, int base) {
    return (base >= args.off[1]) + (base >= args.off[2]);
}

// The matrix of the pass starting at row `base` (wave-uniform) and its first row in the
// row space.
__device__ __forceinline__ GemvMat pass_mat(const GemvArgs &args, int base, int &row0) {
    if (!args.experts) {
        const int mi = pass_matrix(args, base);
        row0 = args.off[mi];
        return args.m[mi];
    }
    const GemvExperts &E = args.ex;
    const bool pair = E.act && E.nm == 2;  // row space [slot][row][gate, up]
    const int sm = pair ? 2 * (base / (2 * E.rows)) : base / E.rows;  // slot * nm + matrix
    const int s = sm / E.nm, m = sm - s * E.nm;
    row0 = sm * E.rows;
    int e = E.idx[s];
    const bool ok = e >= 0 && e < E.n_experts;  // a dropped slot computes expert 0 with weight 0
    e = ok ? e : 0;
    GemvMat M;
    M.w = E.table + (size_t)e * E.stride + E.off[m];
    M.rows = E.rows;
    M.type = E.type;
    M.res = nullptr;
    M.pair = pair;
    M.mstride = (long long)E.off[1] - (long long)E.off[0];
    if (pair) {
        M.y = E.y + (size_t)s * E.rows;
        M.mode = kEpiSwiGLU;
        M.scale = 0.0f;
    } else if (E.nm == 2) {
        M.y = E.y + (size_t)sm * E.rows;
        M.mode = kEpiStore;
        M.scale = 0.0f;
    } else {
        M.part = E.part + (size_t)s * E.rows;
        M.tag = (unsigned int)(*E.gen >> 32);
        M.mode = kEpiScaledStore;
        M.scale = ok ? E.wt[s] : 0.0f;
    }
    return M;
}

// TM: the type of this pass's matrix -- 1 Q4_K, 2 Q6_K.
template <int LPR, int UPL, int TM>
__device__ __forceinline__ void load_pass(const GemvMat &M, int row0, int base, int bpr, Pass<UPL> &ps) {
    const int lane = lane_id();
    const int ul = lane % LPR;
    const int uph = bpr * 2;  // half super-blocks per row
    const int i = lane / LPR;
    const int lrow = M.pair ? ((base - row0) >> 1) + (i >> 1) : base - row0 + i;
    // branch-free: a row past the end of its matrix re-loads the last row, dropped later
    ps.valid = lrow < M.rows;
    ps.lrow = min(lrow, M.rows - 1);
    const int bb = TM == 1 ? kQ4KBytes : kQ6KBytes;
    const uint8_t *wrow = (const uint8_t *)M.w + (M.pair ? (i & 1) * M.mstride : 0) + (size_t)ps.lrow * bpr * bb;
#pragma unroll
    for (int j = 0; j < UPL; j++) {
        const int u = min(ul + j * LPR, uph - 1);
        const uint8_t *blk = wrow + (size_t)(u >> 1) * bb;
        if (TM == 1) load_q4k(blk, u & 1, ps.q[j]);
        else load_q6k(blk, u & 1, ps.q[j]);
    }
}

// The row sums of a pass, valid in lane LPR - 1 of each row's lanes.
template <int LPR, int UPL, int TM>
__device__ __forceinline__ float pass_dot(int bpr, const Pass<UPL> &ps, const XLds &X) {
    const int lane = lane_id();
    const int ul = lane % LPR;
    const int uph = bpr * 2;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < UPL; j++) {
        const int u = ul + j * LPR;
        const int uc = min(u, uph - 1);
        float v;
        if (TM == 1) v = q4k_dot(ps.q[j], uc & 1, uc * 128, X);
        else v = q6k_dot(ps.q[j], uc & 1, uc * 128, X);
        acc += u < uph ? v : 0.0f;
        __builtin_amdgcn_sched_barrier(0);  // one unit's digit reads at a time
    }
    return reduce_rows<LPR>(acc);
}

template <int LPR, int UPL, int TM>
__device__ __forceinline__ void finish_pass(const GemvMat &M, int bpr, const Pass<UPL> &ps, const XLds &X,
                                            float oscale) {
    const float acc = pass_dot<LPR, UPL, TM>(bpr, ps, X) * oscale;
    if (M.mode == kEpiSwiGLU) {
        // the gate row's sum sits LPR lanes below the up row's
        const int lane = lane_id();
        const float g = __shfl(acc, lane - LPR);
        if (lane % LPR == LPR - 1 && ((lane / LPR) & 1) && ps.valid) M.y[ps.lrow] = silu_mul(g, acc);
        return;
    }
    if (lane_id() % LPR == LPR - 1 && ps.valid) {
        if (M.mode == kEpiStore) M.y[ps.lrow] = acc;
        else if (M.mode == kEpiResidual) M.y[ps.lrow] = acc + M.res[ps.lrow];
        else if (M.mode == kEpiScaledAdd) M.y[ps.lrow] += M.scale * acc;
        else  // expert partials: tagged 64-bit slots (see experts_combine)
            __hip_atomic_store(M.part + ps.lrow, ((unsigned long long)M.tag << 32) | __float_as_uint(M.scale * acc),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Expert-mode down launch: after a workgroup has stored its rows' partials, the last of
// the `slots` workgroups that cover the same row tile (one per slot) adds the slot sum,
// in slot order, into out -- deterministic, and no separate combine launch.
// Visibility across the XCDs' separate L2s without fences (an agent-scope fence writes back
// and invalidates a whole L2 per workgroup; it cost ~48 us per MoE layer): every partial is
// one 64-bit atomic slot {tag, value} whose tag is this call's number (the high half of the
// router's arrival counter, which the router of the same call moved on), the tile counter
// only elects the last workgroup, and that workgroup reads each slot until it carries the
// call's tag.  The slot stores were issued before their workgroups counted in, so every
// wait ends; no ordering between two locations is assumed.
constexpr int kPartialWait = 1 << 22;  // bound on one slot's wait (s_sleep rounds)

template <int RPB>
__device__ __forceinline__ void experts_combine(const GemvExperts &E) {
    __shared__ int is_last;
    __syncthreads();  // every wave of the workgroup has issued its partial stores
    const int tile = (int)blockIdx.x % E.ntiles;
    if (threadIdx.x == 0) {
        const int old = __hip_atomic_fetch_add(&E.tile_cnt[tile], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        is_last = old == E.slots - 1;
        if (is_last) __hip_atomic_store(&E.tile_cnt[tile], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!is_last) return;
    const unsigned int tag = (unsigned int)(*E.gen >> 32);
    for (int r = threadIdx.x; r < RPB; r += kGemvThreads) {
        const int row = tile * RPB + r;
        float sum = 0.0f;
        for (int s = 0; s < E.slots; s++) {
            const unsigned long long *slot = E.part + (size_t)s * E.rows + row;
            unsigned long long v = __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            for (int t = 0; (unsigned int)(v >> 32) != tag && t < kPartialWait; t++) {
                __builtin_amdgcn_s_sleep(1);
                v = __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            // a slot still without this call's tag after the bound (a broken ordering, never
            // seen) makes the row NaN instead of adding an earlier call's value
            sum += (unsigned int)(v >> 32) == tag ? __uint_as_float((unsigned int)v) : __builtin_nanf("");
        }
        E.out[row] += sum;
    }
}

// One wave pass per wave, loaded before the x image is built.  The grid covers the row
// space exactly once (no loop), so the loads of every wave are issued back to back.
template <int LPR, int UPL, int XPT, int XM, int TM>
__device__ __forceinline__ void gemv_body(const GemvArgs &args, uint8_t *smem) {
    const int kp = (args.n_cols + 255) & ~255;
    const int bpr = kp / 256;
    XLds X(smem, kp);
    constexpr int P = 64 / LPR;
    constexpr int wpb = kGemvThreads / 64;
    constexpr int rows_per_block = wpb * P;
    const int wave = blockIdx.x * wpb + (threadIdx.x >> 6);
    const int base = __builtin_amdgcn_readfirstlane(wave * P);  // wave-uniform
    const int last = args.total_rows - P;
    const bool down = args.experts && args.ex.nm == 1;  // uniform
    const float *x0 = args.x, *x1 = args.x2;
    if (down) {  // x of this workgroup's slot (rows is a multiple of the workgroup's rows)
        const int s = (int)blockIdx.x * rows_per_block / args.ex.rows;
        x0 = args.ex.xs + (size_t)(args.ex.act ? s : 2 * s) * args.n_cols;
        x1 = x0 + args.n_cols;
    }

    XRegs<XPT> xr, xr2;
    load_x<XPT, XM>(x0, x1, args.n_cols, xr, xr2);
    // a wave past the end loads the last pass again (dropped) so every wave issues the
    // same loads
    int row0;
    const int bc = min(base, last);
    const GemvMat M = pass_mat(args, bc, row0);
    Pass<UPL> ps;
    load_pass<LPR, UPL, TM>(M, row0, bc, bpr, ps);
    // the x image gates every wave of the workgroup at the barrier, while a wave's dot
    // products gate only its own rows: the image is built at raised wave priority, so a
    // SIMD shared with other workgroups' dot products finishes it first (~0.4 us of the
    // fused QKV launch)
    __builtin_amdgcn_s_setprio(3);
    const float oscale = finish_x<XPT, XM>(xr, xr2, args.n_cols, kp, X, args.eps);
    __builtin_amdgcn_s_setprio(0);
    if (base < args.total_rows) finish_pass<LPR, UPL, TM>(M, bpr, ps, X, oscale);
    if (args.experts && args.ex.nm == 2 && blockIdx.x == 0) {
        // clear the tile counters of the down launch that follows on the stream
        for (int t = threadIdx.x; t < args.ex.ntiles; t += kGemvThreads) args.ex.tile_cnt[t] = 0;
    }
    if (down) experts_combine<rows_per_block>(args.ex);
}

#if MNEMO_GEMV_THREADS == 512
// Expert-mode down projection with the slots side by side (slots <= 8, n_cols <= 2048): a
// workgroup covers one tile of P = 64/LPR rows for every slot at once, wave w computing
// slot w's expert with an x image of its own (the SwiGLU of the slot's gate and up rows,
// built by the wave alone).  The slot results meet in LDS and are added in slot order into
// out -- the arithmetic of the partial-buffer path (same digits, same products, same
// order), without the partial stores, the arrival counter and the waits they need, and with
// one workgroup per row tile (256 for 4096 rows at LPR 4: one round on the chip).
constexpr int kSlotWaves = kGemvThreads / 64;
template <int LPR, int UPL, int XPW, int XM, int TM>
__global__ void __launch_bounds__(kGemvThreads) gemv_down_slots_kernel(GemvArgs args) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int P = 64 / LPR;
    __shared__ float red[kSlotWaves][P];
    const GemvExperts &E = args.ex;
    const int n = args.n_cols;
    const int kp = (n + 255) & ~255;
    const int bpr = kp / 256;
    const int w = threadIdx.x >> 6, lane = lane_id();
    const int s = min(w, E.slots - 1);  // waves past the slots repeat the last one, weight 0
    const float *x0 = E.xs + (size_t)(2 * s) * n, *x1 = x0 + n;
    if (XM == 0) x0 = E.xs + (size_t)s * n;  // the SwiGLU output of the gate/up launch
    XRegs<XPW> xr, xr2;
    load_x<XPW, XM, 64>(x0, x1, n, xr, xr2, lane);
    int e = E.idx[s];
    const bool ok = e >= 0 && e < E.n_experts;  // a dropped slot computes expert 0 with weight 0
    e = ok ? e : 0;
    GemvMat M;
    M.w = E.table + (size_t)e * E.stride + E.off[0];
    M.rows = E.rows;
    M.pair = 0;
    M.mstride = 0;
    const int base = (int)blockIdx.x * P;
    // the image before the weight loads: a wave's 33 loads fill the memory queue and stall
    // its instruction issue until they are accepted, so an image built after them starts
    // only then (and the barrier waits for the slowest wave's issue); built first, it
    // costs the weight loads ~0.4 us of delay and the dot products start at once when the
    // loads are in (16.0 -> 14.7 us for 8 experts of 4096 x 1536 Q6_K)
    const XLds X(smem + (size_t)w * xlds_bytes(kp), kp);
    build_x<XPW, XM, 64>(xr, xr2, n, kp, X, lane);
    lds_barrier();
    Pass<UPL> ps;
    load_pass<LPR, UPL, TM>(M, 0, base, bpr, ps);
    const float wt = ok && w < E.slots ? E.wt[s] : 0.0f;
    const float acc = pass_dot<LPR, UPL, TM>(bpr, ps, X);
    if (lane % LPR == LPR - 1) red[w][lane / LPR] = wt * acc;
    __syncthreads();
    const int row = base + (int)threadIdx.x;
    if (threadIdx.x < P && row < E.rows) {
        float sum = 0.0f;
        for (int k = 0; k < E.slots; k++) sum += red[k][threadIdx.x];
        E.out[row] += sum;
    }
}

// The same for Q6_K rows of 1536 values (the expert down projection of 1536-wide experts),
// with the weights staged.  A 210-byte block starts at every even byte offset, so the
// half-super-block loads of the kernel above are 16-byte loads from 4-byte aligned
// addresses (ld16_a2), which stream at under half the rate of aligned ones here.  Instead
// wave w reads its slot's 16-row tile (16 x 1260 contiguous bytes, 16-byte aligned) as
// chunk 64 j + lane of the tile (aligned 16-byte loads, consecutive lanes on consecutive
// chunks), all 20 loads issued at once, and passes the tile through LDS in two parts: the
// first 128 half super-blocks (rows 0..9 and the first 8 of row 10, 13,440 bytes), then the
// other 64.  Lane l takes half super-blocks l and 64 + l of the first part and 128 + l of
// the second, reading each from LDS with the same 2-byte realignment as ld16_a2 and running
// the kernel's dot code; the 12 partial sums of a row are added in order from LDS.
constexpr int kStageRowBytes = 6 * kQ6KBytes;                  // 1260
constexpr int kStageTile = 16 * kStageRowBytes;                // 20160
constexpr int kStagePartA = 64 * kQ6KBytes;                    // 13440: 128 half super-blocks
constexpr int kStageChunks = kStageTile / 16;                  // 1260
constexpr int kStageChunksA = kStagePartA / 16;                // 840
constexpr int kStageLoads = (kStageChunks + 63) / 64;          // 20 per lane
constexpr int kStageBuf = kStagePartA + 16;                    // + a dummy 16-byte slot
constexpr size_t kStageLds = (size_t)kSlotWaves * (kStageBuf + xlds_bytes(1536) + 192 * 4);

// N 16-byte words from a 2-byte aligned LDS address (the LDS form of ld16_a2)
template <int N>
__device__ __forceinline__ void lds16_a2(const uint8_t *p, uint4 (&out)[N]) {
    const uint32_t sh = (uint32_t)(uintptr_t)p & 2u;
    const uint32_t *a = (const uint32_t *)(p - sh);
    uint32_t w[4 * N + 1];
#pragma unroll
    for (int i = 0; i < 4 * N + 1; i++) w[i] = a[i];
#pragma unroll
    for (int i = 0; i < N; i++) {
        out[i].x = __builtin_amdgcn_alignbyte(w[4 * i + 1], w[4 * i], sh);
        out[i].y = __builtin_amdgcn_alignbyte(w[4 * i + 2], w[4 * i + 1], sh);
        out[i].z = __builtin_amdgcn_alignbyte(w[4 * i + 3], w[4 * i + 2], sh);
        out[i].w = __builtin_amdgcn_alignbyte(w[4 * i + 4], w[4 * i + 3], sh);
    }
}

// Half super-block u (0..191) of the tile, staged at buf + its tile offset - base.
__device__ __forceinline__ float stage_unit_dot(const uint8_t *buf, int base, int u, const XLds &X) {
    const int row = u / 12, k = u - 12 * row, hf = k & 1;
    const uint8_t *blk = buf + row * kStageRowBytes + (k >> 1) * kQ6KBytes - base;
    RawH r;
    lds16_a2<4>(blk + 64 * hf, r.q);
    lds16_a2<2>(blk + 128 + 32 * hf, r.qh);
    uint4 h[1];
    lds16_a2<1>(blk + 192, h);
    r.h = h[0];
    r.dd = *(const uint16_t *)(blk + 208);
    return q6k_dot(r, hf, k * 128, X);
}

template <int XM>
__global__ void __launch_bounds__(kGemvThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
gemv_down_stage_kernel(GemvArgs args) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int XPW = 6;  // 1536 values: 6 float4 per lane
    __shared__ float red[kSlotWaves][16];
    const GemvExperts &E = args.ex;
    const int n = args.n_cols;
    const int w = threadIdx.x >> 6, lane = lane_id();
    uint8_t *buf = smem + (size_t)w * kStageBuf;
    const XLds X(smem + (size_t)kSlotWaves * kStageBuf + (size_t)w * xlds_bytes(1536), 1536);
    float *part = (float *)(smem + (size_t)kSlotWaves * (kStageBuf + xlds_bytes(1536))) + w * 192;
    if (w < E.slots) {  // wave-uniform: waves past the slots load nothing
        const int s = w;
        const float *x0 = E.xs + (size_t)(2 * s) * n, *x1 = x0 + n;
        if (XM == 0) x0 = E.xs + (size_t)s * n;  // the SwiGLU output of the gate/up launch
        XRegs<XPW> xr, xr2;
        load_x<XPW, XM, 64>(x0, x1, n, xr, xr2, lane);
        int e = E.idx[s];
        const bool ok = e >= 0 && e < E.n_experts;  // a dropped slot computes expert 0 with weight 0
        e = ok ? e : 0;
        const float wt = ok ? E.wt[s] : 0.0f;
        const uint8_t *tile = E.table + (size_t)e * E.stride + E.off[0] + (size_t)blockIdx.x * kStageTile;
        // The loads of part A, the image, then the loads of part B: all 20 loads before the
        // image stall the issue of its instructions until the memory queue drains (13.9 us
        // against 12.5 us for the 8-slot 4096 x 1536 launch), all of them after it start the
        // tile late (12.9 us).  An LLVM vector type: an array of the HIP uint4 class is
        // copied with memcpy and stays in scratch memory.
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        constexpr int kLoadsA = (kStageChunksA + 63) / 64;  // 14
        u32x4 v[kStageLoads];
#pragma unroll
        for (int j = 0; j < kLoadsA; j++) v[j] = ((const u32x4 *)tile)[min(64 * j + lane, kStageChunks - 1)];
        __builtin_amdgcn_sched_barrier(0);
        build_x<XPW, XM, 64>(xr, xr2, n, 1536, X, lane);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = kLoadsA; j < kStageLoads; j++)
            v[j] = ((const u32x4 *)tile)[min(64 * j + lane, kStageChunks - 1)];
        // Every lane of a load stores (chunks of the other part into a dummy slot past the
        // buffer): a load read only under a lane condition is sunk into it by the compiler,
        // behind the waits of the loads before it.
#pragma unroll
        for (int j = 0; j < kStageLoads; j++) {
            const int c = 64 * j + lane;
            if (64 * j < kStageChunksA) *(u32x4 *)(buf + (c < kStageChunksA ? 16 * c : kStagePartA)) = v[j];
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave's image and part A are in LDS
        part[lane] = stage_unit_dot(buf, 0, lane, X);
        __builtin_amdgcn_sched_barrier(0);  // one unit's digit reads at a time
        part[64 + lane] = stage_unit_dot(buf, 0, 64 + lane, X);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // part A read before it is overwritten
#pragma unroll
        for (int j = 0; j < kStageLoads; j++) {
            const int c = 64 * j + lane - kStageChunksA;
            if (64 * j + 63 >= kStageChunksA)
                *(u32x4 *)(buf + (c >= 0 && c < kStageChunks - kStageChunksA ? 16 * c : kStagePartA)) = v[j];
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        part[128 + lane] = stage_unit_dot(buf, kStagePartA, 128 + lane, X);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane < 16) {  // row lane: its 12 half super-blocks in order
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < 12; k++) acc += part[12 * lane + k];
            red[w][lane] = wt * acc;
        }
    }
    __syncthreads();
    const int row = (int)blockIdx.x * 16 + (int)threadIdx.x;
    if (threadIdx.x < 16) {
        float sum = 0.0f;
        for (int k = 0; k < E.slots; k++) sum += red[k][threadIdx.x];
        E.out[row] += sum;
    }
}

// Paired gate/up launch of the decode MoE block for rows of 4096 values (Q4_K), staged like
// the down kernel above: a 4-wave workgroup owns 16 rows of one slot (wave w: rows
// 4w .. 4w+3 of the gate and of the up matrix) and builds one x image (with the RMS norm,
// XM 2) for all of them.  A wave reads its 4 gate rows (9,216 contiguous bytes, 9 aligned
// 16-byte loads per lane, consecutive lanes on consecutive chunks), then its 4 up rows,
// passes each part through a wave-private LDS area and runs the unchanged q4k_dot on half
// super-blocks l and 64 + l of the part (rows l / 32 and 2 + l / 32).  768 workgroups for
// 8 slots x 1536 rows, three per CU: one round.  Half the image builds and x reads of the
// whole-row launch, and whole cache lines per load instruction.
constexpr int kGuRowBytes = 16 * kQ4KBytes;        // 2304: 4096 values
constexpr int kGuPart = 4 * kGuRowBytes;           // 9216: 4 rows
constexpr int kGuLoads = kGuPart / 16 / 64;        // 9 per lane and part
constexpr int kGuThreads = 256;
constexpr size_t kGuLds = (size_t)(kGuThreads / 64) * kGuPart + xlds_bytes(4096);
static_assert(kGuPart % 1024 == 0, "a part is whole 64-lane loads");

template <int XM>
__global__ void __launch_bounds__(kGuThreads) gemv_gateup_stage_kernel(GemvArgs args) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int XPT = 4096 / (4 * kGuThreads);  // 4 float4 of x per thread
    __shared__ float part_ss[kGuThreads / 64];
    const GemvExperts &E = args.ex;
    const int w = threadIdx.x >> 6, lane = lane_id();
    const int tiles = E.rows / 16;
    const int s = (int)blockIdx.x / tiles, r0 = ((int)blockIdx.x - s * tiles) * 16 + 4 * w;
    uint8_t *buf = smem + (size_t)w * kGuPart;
    const XLds X(smem + (size_t)(kGuThreads / 64) * kGuPart, 4096);
    XRegs<XPT> xr, xr2;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    // XM 3: the router's image of x * g, 16-byte words copied into LDS (every thread loads:
    // clamped, stored only where inside the image)
    constexpr int kImgWords = (int)(xlds_bytes(4096) / 16);
    constexpr int kImgPer = (kImgWords + kGuThreads - 1) / kGuThreads;
    u32x4 im[XM == 3 ? kImgPer : 1];
    if (XM == 3) {
#pragma unroll
        for (int i = 0; i < kImgPer; i++)
            im[i] = ((const u32x4 *)args.ximg)[min((int)threadIdx.x + kGuThreads * i, kImgWords - 1)];
    } else {
        load_x<XPT, XM == 2 ? 2 : 0, kGuThreads>(args.x, args.x2, 4096, xr, xr2, threadIdx.x);
    }
    int e = E.idx[s];
    e = e >= 0 && e < E.n_experts ? e : 0;  // a dropped slot computes expert 0 (weight 0 in the down)
    const uint8_t *mat = E.table + (size_t)e * E.stride;
    const u32x4 *gsrc = (const u32x4 *)(mat + E.off[0] + (size_t)r0 * kGuRowBytes);
    const u32x4 *usrc = (const u32x4 *)(mat + E.off[1] + (size_t)r0 * kGuRowBytes);
    u32x4 vg[kGuLoads], vu[kGuLoads];
#pragma unroll
    for (int j = 0; j < kGuLoads; j++) vg[j] = gsrc[64 * j + lane];
    __builtin_amdgcn_sched_barrier(0);
    // the image (every thread builds 16 values; the barrier ends it)
    float ss = 0.0f;
    if (XM == 2) {
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            ss = fmaf(xr.v[i].x, xr.v[i].x, ss);
            ss = fmaf(xr.v[i].y, xr.v[i].y, ss);
            ss = fmaf(xr.v[i].z, xr.v[i].z, ss);
            ss = fmaf(xr.v[i].w, xr.v[i].w, ss);
        }
        ss = sum64_lane63(ss);
        if (lane == 63) part_ss[w] = ss;
    }
    if (XM == 3) {
        uint8_t *ximg = smem + (size_t)(kGuThreads / 64) * kGuPart;
#pragma unroll
        for (int i = 0; i < kImgPer; i++) {
            const int c = (int)threadIdx.x + kGuThreads * i;
            if (c < kImgWords) *(u32x4 *)(ximg + 16 * c) = im[i];
        }
    } else {
        build_x<XPT, XM == 2 ? 2 : 0, kGuThreads>(xr, xr2, 4096, 4096, X, threadIdx.x);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < kGuLoads; j++) vu[j] = usrc[64 * j + lane];
    lds_barrier();  // the image (the waves' weights stay in flight)
    float oscale = 1.0f;
    if (XM == 3) oscale = *args.xscale;
    if (XM == 2) {
        float tot = 0.0f;
#pragma unroll
        for (int k = 0; k < kGuThreads / 64; k++) tot += part_ss[k];
        oscale = __builtin_amdgcn_rsqf(tot / 4096.0f + args.eps);  // rsqrtf, as the reference (kernels.cu:718)
    }
    float acc[2][2];  // [gate, up][unit l, unit 64 + l]
#pragma unroll
    for (int m = 0; m < 2; m++) {
        const u32x4 *v = m == 0 ? vg : vu;
#pragma unroll
        for (int j = 0; j < kGuLoads; j++) *(u32x4 *)(buf + 16 * (64 * j + lane)) = v[j];
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's part is in LDS
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int u = 64 * k + lane, row = u >> 5, hu = u & 31;
            const uint8_t *blk = buf + row * kGuRowBytes + (hu >> 1) * kQ4KBytes;
            RawH r;
            r.h = *(const uint4 *)blk;
#pragma unroll
            for (int i = 0; i < 4; i++) r.q[i] = *(const uint4 *)(blk + 16 + 64 * (hu & 1) + 16 * i);
            acc[m][k] = sum32_lane31(q4k_dot(r, hu & 1, hu * 128, X));
            __builtin_amdgcn_sched_barrier(0);  // one unit's digit reads at a time
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the part is read before it is overwritten
    }
    if ((lane & 31) == 31) {
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int row = r0 + 2 * k + (lane >> 5);
            E.y[(size_t)s * E.rows + row] = silu_mul(acc[0][k] * oscale, acc[1][k] * oscale);
        }
    }
    if (blockIdx.x == 0)  // clear the tile counters of the down launch that follows on the stream
        for (int t = threadIdx.x; t < E.ntiles; t += kGuThreads) E.tile_cnt[t] = 0;
}

template <int UPL, int XPW>
static void launch_down_slots(const GemvArgs &a, int tm, hipStream_t stream) {
    constexpr int LPR = 4, P = 64 / LPR;
    const int kp = (a.n_cols + 255) & ~255;
    const int blocks = (a.ex.rows + P - 1) / P;
    const size_t lds = (size_t)kSlotWaves * xlds_bytes(kp);
    const dim3 g(blocks), b(kGemvThreads);
    if (a.ex.act) {
        if (tm == 1) hipLaunchKernelGGL((gemv_down_slots_kernel<LPR, UPL, XPW, 0, 1>), g, b, lds, stream, a);
        else hipLaunchKernelGGL((gemv_down_slots_kernel<LPR, UPL, XPW, 0, 2>), g, b, lds, stream, a);
    } else {
        if (tm == 1) hipLaunchKernelGGL((gemv_down_slots_kernel<LPR, UPL, XPW, 1, 1>), g, b, lds, stream, a);
        else hipLaunchKernelGGL((gemv_down_slots_kernel<LPR, UPL, XPW, 1, 2>), g, b, lds, stream, a);
    }
}
#endif

#if MNEMO_GEMV_THREADS == 512
// Split-columns form of the static GEMV.  A workgroup owns 64 / LPR rows; its W waves split
// the columns, wave w taking the 128 * LPR columns [w * 128 LPR, (w + 1) * 128 LPR) of those
// rows (one half super-block per lane, LPR lanes per row).  Each wave builds the x image of its
// own columns only and reads it back alone (no workgroup barrier before the dot products);
// the LPR lanes of a row read LPR different 16-byte words and the rows of the wave the same
// ones (an LDS broadcast).  The waves' row sums meet in LDS once, at the end, and are added in
// wave order.  TM: the workgroup's type, 1 Q4_K or 2 Q6_K.
template <int LPR, int W, int XM, int TM>
__device__ __forceinline__ void gemv_split_body(const GemvArgs &args, uint8_t (*img)[xlds_bytes(128 * LPR)],
                                                float (*red)[64 / LPR], float *ssw) {
    constexpr int R = 64 / LPR;
    constexpr int CW = 128 * LPR;
    constexpr int XPW = CW / 256;  // float4 of x per lane
    const int w = threadIdx.x >> 6, lane = lane_id();
    const int n = args.n_cols;
    const int kp = (n + 255) & ~255;
    const int uph = kp / 128;        // half super-blocks per row
    const int c0 = w * CW;           // this wave's first column
    const int nw = min(CW, n - c0);  // its columns (>= 4: n % 4 == 0 and c0 < n)
    XRegs<XPW> xr, xr2;
    load_x<XPW, XM, 64>(args.x + c0, args.x2 ? args.x2 + c0 : nullptr, nw, xr, xr2, lane);

    // the weights: row base + lane / LPR, half super-block w * LPR + lane % LPR
    const int base = (int)blockIdx.x * R;
    int row0;
    const GemvMat M = pass_mat(args, base, row0);
    const int i = lane / LPR, ul = lane % LPR;
    const int bb = TM == 1 ? kQ4KBytes : kQ6KBytes;
    const int u = w * LPR + ul;
    const int uc = min(u, uph - 1);
    RawH raw;
    {
        const int lrow = min(base - row0 + i, M.rows - 1);
        const uint8_t *blk = (const uint8_t *)M.w + ((size_t)lrow * (kp / 256) + (uc >> 1)) * bb;
        if (TM == 1) load_q4k(blk, uc & 1, raw);
        else load_q6k(blk, uc & 1, raw);
    }

    const XLds X(img[w], CW);
    build_x<XPW, XM, 64>(xr, xr2, nw, CW, X, lane);
    float ss = 0.0f;
    if (XM == 2) {
#pragma unroll
        for (int j = 0; j < XPW; j++) {
            if (4 * (lane + 64 * j) < nw) {
                ss = fmaf(xr.v[j].x, xr.v[j].x, ss);
                ss = fmaf(xr.v[j].y, xr.v[j].y, ss);
                ss = fmaf(xr.v[j].z, xr.v[j].z, ss);
                ss = fmaf(xr.v[j].w, xr.v[j].w, ss);
            }
        }
    }
    if (XM == 2) {
        ss = sum64_lane63(ss);
        if (lane == 63) ssw[w] = ss;
    }
    // the wave reads only what it wrote: its own LDS stores done is enough
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    float v = TM == 1 ? q4k_dot(raw, uc & 1, ul * 128, X) : q6k_dot(raw, uc & 1, ul * 128, X);
    v = u < uph ? v : 0.0f;
    v = reduce_rows<LPR>(v);
    if (ul == LPR - 1) red[w][i] = v;
    __syncthreads();
    if ((int)threadIdx.x < R) {
        const int r = threadIdx.x;
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < W; k++) acc += red[k][r];
        if (XM == 2) {
            float tot = 0.0f;
#pragma unroll
            for (int k = 0; k < W; k++) tot += ssw[k];
            acc *= __builtin_amdgcn_rsqf(tot / (float)n + args.eps);  // rsqrtf, as the reference (kernels.cu:718)
        }
        const int lr = base - row0 + r;
        if (lr < M.rows) {
            if (M.mode == kEpiStore) M.y[lr] = acc;
            else if (M.mode == kEpiResidual) M.y[lr] = acc + M.res[lr];
            else M.y[lr] += M.scale * acc;
        }
    }
}

// TM: types present in the launch, 1 Q4_K only, 2 Q6_K only, 3 both (each matrix then starts
// at a multiple of the workgroup's rows, so the type is uniform per workgroup).
template <int LPR, int W, int XM, int TM>
__global__ void __launch_bounds__(64 * W) gemv_split_kernel(GemvArgs args) {
    constexpr int R = 64 / LPR;
    __shared__ __align__(16) uint8_t img[W][xlds_bytes(128 * LPR)];
    __shared__ float red[W][R];
    __shared__ float ssw[W];
    if constexpr (TM == 3) {
        const int mi = pass_matrix(args, (int)blockIdx.x * R);
        if (args.m[mi].type == kTypeQ4K) gemv_split_body<LPR, W, XM, 1>(args, img, red, ssw);
        else gemv_split_body<LPR, W, XM, 2>(args, img, red, ssw);
    } else {
        gemv_split_body<LPR, W, XM, TM>(args, img, red, ssw);
    }
}

template <int LPR, int W, int TM>
static void launch_split_tm(const GemvArgs &a, int blocks, hipStream_t stream) {
    const dim3 g(blocks), b(64 * W);
    if (a.xmode == 1) hipLaunchKernelGGL((gemv_split_kernel<LPR, W, 1, TM>), g, b, 0, stream, a);
    else if (a.xmode == 2) hipLaunchKernelGGL((gemv_split_kernel<LPR, W, 2, TM>), g, b, 0, stream, a);
    else hipLaunchKernelGGL((gemv_split_kernel<LPR, W, 0, TM>), g, b, 0, stream, a);
}

// One Q6_K matrix of 4096-value rows (the lm_head), staged: a 4-wave workgroup owns 16 rows
// and builds one x image; wave w reads its 4 rows (13,440 contiguous, 16-byte aligned bytes:
// 14 aligned lane-contiguous loads per lane, the chunks past the rows going to a dummy
// slot), passes them through LDS and runs the unchanged q6k_dot on half super-blocks l and
// 64 + l (rows l / 32 and 2 + l / 32), read with the 2-byte realignment of lds16_a2.
constexpr int kQsRowBytes = 16 * kQ6KBytes;          // 3360: 4096 values
constexpr int kQsPart = 4 * kQsRowBytes;             // 13440: a wave's 4 rows
constexpr int kQsChunks = kQsPart / 16;              // 840
constexpr int kQsLoads = (kQsChunks + 63) / 64;      // 14
constexpr int kQsBuf = kQsPart + 16;                 // + a dummy 16-byte slot
constexpr int kQsThreads = 256;
constexpr size_t kQsLds = (size_t)(kQsThreads / 64) * kQsBuf + xlds_bytes(4096);

__global__ void __launch_bounds__(kQsThreads) gemv_q6stage_kernel(GemvArgs args) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int XPT = 4096 / (4 * kQsThreads);  // 4 float4 of x per thread
    const int w = threadIdx.x >> 6, lane = lane_id();
    const GemvMat &M = args.m[0];
    const int r0 = (int)blockIdx.x * 16 + 4 * w;
    uint8_t *buf = smem + (size_t)w * kQsBuf;
    const XLds X(smem + (size_t)(kQsThreads / 64) * kQsBuf, 4096);
    XRegs<XPT> xr, xr2;
    load_x<XPT, 0, kQsThreads>(args.x, nullptr, 4096, xr, xr2, threadIdx.x);
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 *src = (const u32x4 *)((const uint8_t *)M.w + (size_t)r0 * kQsRowBytes);
    u32x4 v[kQsLoads];
#pragma unroll
    for (int j = 0; j < kQsLoads; j++) v[j] = src[min(64 * j + lane, kQsChunks - 1)];
    __builtin_amdgcn_sched_barrier(0);
    build_x<XPT, 0, kQsThreads>(xr, xr2, 4096, 4096, X, threadIdx.x);
    lds_barrier();  // the image only: each wave's rows wait for its own loads
    // every lane of a load stores (a load read only under a lane condition is sunk into it)
#pragma unroll
    for (int j = 0; j < kQsLoads; j++) {
        const int c = 64 * j + lane;
        *(u32x4 *)(buf + (c < kQsChunks ? 16 * c : kQsPart)) = v[j];
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    float acc[2];
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int u = 64 * k + lane, row = u >> 5, hu = u & 31, hf = hu & 1;
        const uint8_t *blk = buf + row * kQsRowBytes + (hu >> 1) * kQ6KBytes;
        RawH r;
        lds16_a2<4>(blk + 64 * hf, r.q);
        lds16_a2<2>(blk + 128 + 32 * hf, r.qh);
        uint4 h[1];
        lds16_a2<1>(blk + 192, h);
        r.h = h[0];
        r.dd = *(const uint16_t *)(blk + 208);
        acc[k] = sum32_lane31(q6k_dot(r, hf, hu * 128, X));
        __builtin_amdgcn_sched_barrier(0);  // one unit's digit reads at a time
    }
    if ((lane & 31) == 31) {
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int row = r0 + 2 * k + (lane >> 5);
            if (M.mode == kEpiStore) M.y[row] = acc[k];
            else if (M.mode == kEpiResidual) M.y[row] = acc[k] + M.res[row];
            else M.y[row] += M.scale * acc[k];
        }
    }
}

// Returns kErrBadArg (nothing launched, no error recorded) for launches it does not take.
int launch_gemv_q6stage_impl(GemvArgs a, hipStream_t stream) {
    if (a.experts || a.nmat != 1 || a.xmode != 0 || a.n_cols != 4096) return kErrBadArg;
    const GemvMat &M = a.m[0];
    if (M.type != kTypeQ6K || M.rows <= 0 || M.rows % 16 || (uintptr_t)M.w % 16 ||
        (M.mode != kEpiStore && M.mode != kEpiResidual && M.mode != kEpiScaledAdd))
        return kErrBadArg;
    hipLaunchKernelGGL(gemv_q6stage_kernel, dim3(M.rows / 16), dim3(kQsThreads), kQsLds, stream, a);
    return check_launch("gemv (staged Q6_K 4096-value rows)");
}

// LPR 8: 1024 columns per wave, 4 or 8 waves per workgroup (rows of 3076..4096 or
// 7172..8192 columns).  Returns kErrBadArg (nothing launched, no error recorded) for launches
// it does not take.
int launch_gemv_split_impl(GemvArgs a, hipStream_t stream) {
    constexpr int LPR = 8, R = 64 / LPR;
    if (a.experts || a.n_cols < 4 || a.n_cols % 4 || a.n_cols > kMaxGemvCols) return kErrBadArg;
    const int kp = (a.n_cols + 255) & ~255;
    const int waves = (kp + 128 * LPR - 1) / (128 * LPR);
    if ((waves != 4 && waves != 8) || kp <= (waves - 1) * 128 * LPR) return kErrBadArg;
    int tm = 0;
    for (int i = 0; i < a.nmat; i++) {
        if (a.m[i].mode != kEpiStore && a.m[i].mode != kEpiResidual && a.m[i].mode != kEpiScaledAdd) return kErrBadArg;
        tm |= a.m[i].type == kTypeQ4K ? 1 : 2;
    }
    int off = 0;
    for (int i = 0; i < a.nmat; i++) {
        a.off[i] = off;
        off += (a.m[i].rows + R - 1) / R * R;  // a workgroup never spans two matrices
    }
    for (int i = a.nmat; i < 3; i++) a.off[i] = INT_MAX;
    a.total_rows = off;
    const int blocks = off / R;
    if (waves == 4) {
        if (tm == 1) launch_split_tm<LPR, 4, 1>(a, blocks, stream);
        else if (tm == 2) launch_split_tm<LPR, 4, 2>(a, blocks, stream);
        else launch_split_tm<LPR, 4, 3>(a, blocks, stream);
    } else {
        if (tm == 1) launch_split_tm<LPR, 8, 1>(a, blocks, stream);
        else if (tm == 2) launch_split_tm<LPR, 8, 2>(a, blocks, stream);
        else launch_split_tm<LPR, 8, 3>(a, blocks, stream);
    }
    return check_launch("gemv split");
}
#endif

// TM: types present in the launch -- 1 Q4_K only, 2 Q6_K only, 3 both.  With both, every
// matrix starts at a multiple of the rows of one workgroup, so the type is uniform per
// workgroup and each workgroup runs the single-type code (the barrier of the x image
// sits in both branches; each wave reaches exactly one).
template <int LPR, int UPL, int XPT, int XM, int TM>
__global__ void __launch_bounds__(kGemvThreads) gemv_kernel(GemvArgs args) {
    extern __shared__ __align__(16) uint8_t smem[];
    if constexpr (TM == 3) {
        constexpr int rows_per_block = (kGemvThreads / 64) * (64 / LPR);
        const int mi = pass_matrix(args, (int)blockIdx.x * rows_per_block);
        if (args.m[mi].type == kTypeQ4K) gemv_body<LPR, UPL, XPT, XM, 1>(args, smem);
        else gemv_body<LPR, UPL, XPT, XM, 2>(args, smem);
    } else {
        gemv_body<LPR, UPL, XPT, XM, TM>(args, smem);
    }
}

template <int LPR, int UPL, int XPT, int TM>
static void launch_tm(const GemvArgs &a, int blocks, size_t lds, hipStream_t stream) {
    if (a.xmode == 1)
        hipLaunchKernelGGL((gemv_kernel<LPR, UPL, XPT, 1, TM>), dim3(blocks), dim3(kGemvThreads), lds, stream, a);
    else if (a.xmode == 2)
        hipLaunchKernelGGL((gemv_kernel<LPR, UPL, XPT, 2, TM>), dim3(blocks), dim3(kGemvThreads), lds, stream, a);
    else
        hipLaunchKernelGGL((gemv_kernel<LPR, UPL, XPT, 0, TM>), dim3(blocks), dim3(kGemvThreads), lds, stream, a);
}

template <int LPR, int UPL, int XPT>
static void launch(const GemvArgs &a, int tm, int blocks, size_t lds, hipStream_t stream) {
    if (tm == 1) launch_tm<LPR, UPL, XPT, 1>(a, blocks, lds, stream);
    else if (tm == 2) launch_tm<LPR, UPL, XPT, 2>(a, blocks, lds, stream);
    else launch_tm<LPR, UPL, XPT, 3>(a, blocks, lds, stream);
}

static int device_cus() {
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

int launch_gemv_impl(GemvArgs a, hipStream_t stream) {
    if (a.n_cols < 4 || a.n_cols > kMaxGemvCols) return kErrBadArg;
    if (a.xmode == 2 && (a.n_cols % 4 || !a.x2)) return set_error(kErrBadArg, "gemv rms-norm input: n_cols %% 4 and a weight");
    const int kp = (a.n_cols + 255) & ~255;
    // half super-blocks per row -> lanes per row (pow2, <= 64) and rows per wave pass
    const int uph = kp / 128;
    int lpr = 2;
    while (lpr < uph && lpr < 64) lpr <<= 1;
    constexpr int wpb = kGemvThreads / 64;
    int tm = 0;
    for (int i = 0; i < a.nmat; i++) tm |= a.m[i].type == kTypeQ4K ? 1 : 2;
    // Row space: each matrix starts at a multiple of P rows so that no wave pass spans two
    // matrices; with mixed types at a multiple of a workgroup's rows (the type is then
    // uniform per workgroup).  One pass per wave: the loads of a wave are issued back to
    // back and the hardware queues the workgroups beyond what fits on the chip.
    auto layout = [&](int lanes_per_row) {
        const int P = 64 / lanes_per_row;
        const int align = tm == 3 ? wpb * P : P;
        int off = 0;
        for (int i = 0; i < a.nmat; i++) {
            a.off[i] = off;
            off += (a.m[i].rows + align - 1) / align * align;
        }
        for (int i = a.nmat; i < 3; i++) a.off[i] = INT_MAX;
        a.total_rows = off;
        return off / P;
    };
    const int passes = layout(lpr);
    // More waves than fit on the chip at once (16 per CU) leave a second, mostly idle
    // generation of workgroups; the alternatives measured slower: two row passes per wave,
    // two half super-blocks per lane (register pressure halves the waves per CU) and
    // 640..1024-thread workgroups.
    const int blocks = (passes + wpb - 1) / wpb;
    const size_t lds = xlds_bytes(kp);
    // XPT = float4 of x per thread = kp / (4 * kGemvThreads), rounded up
    constexpr int T4 = 4 * kGemvThreads;
    constexpr int X4K = (4096 + T4 - 1) / T4, X8K = (8192 + T4 - 1) / T4, X16K = (16384 + T4 - 1) / T4;
    switch (lpr) {
    case 2: launch<2, 1, xpt_for(256)>(a, tm, blocks, lds, stream); break;
    case 4: launch<4, 1, xpt_for(512)>(a, tm, blocks, lds, stream); break;
    case 8: launch<8, 1, xpt_for(1024)>(a, tm, blocks, lds, stream); break;
    case 16: launch<16, 1, xpt_for(2048)>(a, tm, blocks, lds, stream); break;
    case 32: launch<32, 1, X4K>(a, tm, blocks, lds, stream); break;
    default:
        if (kp <= 8192) launch<64, 1, X8K>(a, tm, blocks, lds, stream);
        else launch<64, 2, X16K>(a, tm, blocks, lds, stream);
    }
    return check_launch("gemv");
}

// Expert mode: lpr from n_cols as for the static launch; the rows of one matrix must be a
// multiple of a workgroup's rows so that a workgroup never spans two slots (its x image
// and its row tile belong to one slot).
int launch_gemv_experts_impl(GemvArgs a, hipStream_t stream) {
    if (a.n_cols < 4 || a.n_cols > kMaxGemvCols) return kErrBadArg;
    const int kp = (a.n_cols + 255) & ~255;
    const int uph = kp / 128;
#ifndef MNEMO_DOWN_SLOTS
#define MNEMO_DOWN_SLOTS 1
#endif
#if MNEMO_GEMV_THREADS == 512
    if (MNEMO_DOWN_SLOTS && a.ex.nm == 1 && a.ex.slots <= kSlotWaves && kp <= 2048 && a.ex.rows > 0) {
        a.experts = 1;
        a.nmat = 0;
        a.xmode = a.ex.act ? 0 : 1;
        a.total_rows = a.ex.rows;
        const int tm = a.ex.type == kTypeQ4K ? 1 : 2;
        // LPR 4: a row's uph half super-blocks over 4 lanes, UPL = uph / 4 each
        // Q6_K 1536-value rows in whole 16-row tiles, 16-byte aligned: the staged kernel
        if (tm == 2 && a.n_cols == 1536 && a.ex.rows % 16 == 0 &&
            ((uintptr_t)a.ex.table % 16 | a.ex.stride % 16 | a.ex.off[0] % 16) == 0) {
            const dim3 g(a.ex.rows / 16), b(kGemvThreads);
            if (a.ex.act) hipLaunchKernelGGL((gemv_down_stage_kernel<0>), g, b, kStageLds, stream, a);
            else hipLaunchKernelGGL((gemv_down_stage_kernel<1>), g, b, kStageLds, stream, a);
            return check_launch("gemv_experts down (staged)");
        }
        if (uph <= 4) launch_down_slots<1, 2>(a, tm, stream);
        else if (uph <= 8) launch_down_slots<2, 4>(a, tm, stream);
        else if (uph <= 12) launch_down_slots<3, 6>(a, tm, stream);
        else launch_down_slots<4, 8>(a, tm, stream);
        return check_launch("gemv_experts down");
    }
#endif
#if MNEMO_GEMV_THREADS == 512
    // paired gate/up of 4096-value Q4_K rows in whole 16-row tiles, 16-byte aligned: staged
    if (a.ex.nm == 2 && a.ex.act && a.ex.type == kTypeQ4K && a.n_cols == 4096 && a.ex.rows % 16 == 0 &&
        a.ex.rows > 0 && ((uintptr_t)a.ex.table % 16 | a.ex.stride % 16 | a.ex.off[0] % 16 | a.ex.off[1] % 16) == 0) {
        a.experts = 1;
        a.nmat = 0;
        const dim3 g(a.ex.slots * (a.ex.rows / 16)), b(kGuThreads);
        if (a.ximg) hipLaunchKernelGGL((gemv_gateup_stage_kernel<3>), g, b, kGuLds, stream, a);
        else if (a.x2) hipLaunchKernelGGL((gemv_gateup_stage_kernel<2>), g, b, kGuLds, stream, a);
        else hipLaunchKernelGGL((gemv_gateup_stage_kernel<0>), g, b, kGuLds, stream, a);
        return check_launch("gemv_experts gate/up (staged)");
    }
#endif
    int lpr = 2;
    while (lpr < uph && lpr < 64) lpr <<= 1;
    const int P = 64 / lpr;
    constexpr int wpb = kGemvThreads / 64;
    const int rpb = wpb * P;
    GemvExperts &E = a.ex;
    const bool pair = E.act && E.nm == 2;  // gate and up rows side by side in a pass
    if (pair && P < 2) return set_error(kErrBadArg, "expert GEMV: paired gate/up needs n_cols <= 4096");
    if ((pair ? 2 * E.rows : E.rows) % rpb != 0)
        return set_error(kErrBadArg, "expert GEMV: rows %d not a multiple of %d", E.rows, pair ? rpb / 2 : rpb);
    a.experts = 1;
    a.nmat = 0;
    // down: SwiGLU of the slot (or its precomputed product); gate/up: x, or its RMS norm
    a.xmode = E.nm == 1 ? (E.act ? 0 : 1) : (a.x2 ? 2 : 0);
    if (a.xmode == 2 && a.n_cols % 4) return set_error(kErrBadArg, "expert GEMV rms-norm input: n_cols %% 4");
    a.total_rows = E.slots * E.nm * E.rows;
    if (E.nm == 1) E.ntiles = E.rows / rpb;
    const int tm = E.type == kTypeQ4K ? 1 : 2;
    const int blocks = a.total_rows / rpb;
    const size_t lds = xlds_bytes(kp);
    constexpr int T4 = 4 * kGemvThreads;
    constexpr int X4K = (4096 + T4 - 1) / T4, X8K = (8192 + T4 - 1) / T4, X16K = (16384 + T4 - 1) / T4;
    switch (lpr) {
    case 2: launch<2, 1, xpt_for(256)>(a, tm, blocks, lds, stream); break;
    case 4: launch<4, 1, xpt_for(512)>(a, tm, blocks, lds, stream); break;
    case 8: launch<8, 1, xpt_for(1024)>(a, tm, blocks, lds, stream); break;
    case 16: launch<16, 1, xpt_for(2048)>(a, tm, blocks, lds, stream); break;
    case 32: launch<32, 1, X4K>(a, tm, blocks, lds, stream); break;
    default:
        if (kp <= 8192) launch<64, 1, X8K>(a, tm, blocks, lds, stream);
        else launch<64, 2, X16K>(a, tm, blocks, lds, stream);
    }
    return check_launch("gemv_experts");
}

}  // namespace MNEMO_GEMV_NS
}  // namespace mnemo
