// attn.hip -- the decode attention chain around the projections (MnemoCUDA forward.c:687-786,
// graph form forward.c:1290-1420): RMS norms, the per-head pass (QK norm, RoPE, KV-cache
// store) and attention over the cache.
//
//  * rms_norm_row     (kernels.cu:692-749): one workgroup of 1024 threads per vector, fixed-
//                     order reduction; optional copy of the input (the residual save).
//  * head pass        (kernels.cu:754-781, 1196-1219, 818-852, 1320-1377): one wave per head;
//                     lane j holds the RoPE pairs (j + 64t, j + 64t + hd/2), so the norm is a
//                     wave reduction and the rotation needs no exchange.  Q heads, K heads and
//                     V heads of one token go through one launch: norm -> RoPE -> store to the
//                     cache (f16, or int8 with a per-head absmax scale).  The position can come
//                     from device memory, so a captured graph replays for every token without
//                     the reference's per-token kernel-node parameter updates
//                     (forward.c:638-666).
//  * attention        (kernels.cu:1382-1481, 1550-1660): one workgroup per query head over
//                     tiles of positions with an online softmax, as the reference's entry
//                     points define it (no workspace); the GQA-batched split-position kernel
//                     lives in attn_decode.hip.
//
// RoPE: frequencies 1.0f / powf(theta, (float)(2j) / (float)hd) are computed on the host
// with the C library's powf, as the reference does (kernels.cu:1256-1266), and travel in the
// kernel arguments; angles pos * freq in fp32 as the reference forms them; sin/cos are the
// accurate sincosf (the reference uses the __sincosf approximation, whose error grows with
// the angle).
#include <math.h>

#include "mnemo_common.hpp"
#include "mnemo_internal.hpp"

namespace mnemo {

constexpr int kNormThreads = 1024;


// ------------------------------------------------------------------ RMS norm of one vector
// out may alias in (each element is read and written by the same thread after the
// reduction); res, when given, aliases neither.  Vector path (n % 4 == 0, n <= 16384,
// 16-byte aligned): every thread's float4s are loaded once, up front, and kept in
// registers; the general path reads in twice.
constexpr int kNormV4 = 4;

__global__ void __launch_bounds__(kNormThreads) rms_norm_row_kernel(const float *in, const float *__restrict__ w,
                                                                   float *out, float *__restrict__ res, int n,
                                                                   float eps, int vec4) {
    __shared__ float part[kNormThreads / 64];
    const int tid = threadIdx.x;
    float ss = 0.0f;
    float4 xv[kNormV4];
    const int n4 = n / 4;
    if (vec4) {
#pragma unroll
        for (int u = 0; u < kNormV4; u++) {
            const int i = min(tid + u * kNormThreads, n4 - 1);  // clamped: branch-free loads
            xv[u] = ((const float4 *)in)[i];
        }
#pragma unroll
        for (int u = 0; u < kNormV4; u++) {
            if (tid + u * kNormThreads < n4) {
                ss = fmaf(xv[u].x, xv[u].x, ss);
                ss = fmaf(xv[u].y, xv[u].y, ss);
                ss = fmaf(xv[u].z, xv[u].z, ss);
                ss = fmaf(xv[u].w, xv[u].w, ss);
                if (res) ((float4 *)res)[tid + u * kNormThreads] = xv[u];
            }
        }
    } else {
        for (int i = tid; i < n; i += kNormThreads) {
            const float v = in[i];
            ss = fmaf(v, v, ss);
            if (res) res[i] = v;
        }
    }
    ss = sum64_lane63(ss);
    if (lane_id() == 63) part[tid >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < kNormThreads / 64; i++) tot += part[i];  // same order in every thread
    const float scale = __builtin_amdgcn_rsqf(tot / (float)n + eps);  // rsqrtf, as the reference (kernels.cu:718)
    if (vec4) {
#pragma unroll
        for (int u = 0; u < kNormV4; u++) {
            const int i = tid + u * kNormThreads;
            if (i < n4) {
                const float4 wv = ((const float4 *)w)[i];
                float4 o;
                o.x = xv[u].x * scale * wv.x;
                o.y = xv[u].y * scale * wv.y;
                o.z = xv[u].z * scale * wv.z;
                o.w = xv[u].w * scale * wv.w;
                ((float4 *)out)[i] = o;
            }
        }
    } else {
        for (int i = tid; i < n; i += kNormThreads) out[i] = in[i] * scale * w[i];
    }
}

int launch_rms_norm(const float *in, const float *w, float *out, float *res, int n, float eps, hipStream_t s) {
    if (!in || !w || !out || n <= 0) return set_error(kErrBadArg, "rms_norm: bad arguments");
    if (res == in) res = nullptr;  // saving the input onto itself: nothing to write
    if (res && (res == out || res == w)) return set_error(kErrBadArg, "rms_norm: residual aliases out or weight");
    const int vec4 = n % 4 == 0 && n <= 4 * kNormV4 * kNormThreads &&
                     (((uintptr_t)in | (uintptr_t)w | (uintptr_t)out | (uintptr_t)res) % 16) == 0;
    hipLaunchKernelGGL(rms_norm_row_kernel, dim3(1), dim3(kNormThreads), 0, s, in, w, out, res, n, eps, vec4);
    return check_launch("rms_norm");
}

__global__ void residual_add_kernel(const float *__restrict__ a, const float *__restrict__ b, float *out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = a[i] + b[i];
}

int launch_residual_add(const float *a, const float *b, float *out, int n, hipStream_t s) {
    if (!a || !b || !out || n <= 0) return set_error(kErrBadArg, "residual_add: bad arguments");
    hipLaunchKernelGGL(residual_add_kernel, dim3((n + 255) / 256), dim3(256), 0, s, a, b, out, n);
    return check_launch("residual_add");
}

__global__ void f32_to_f16_dual_kernel(const float *__restrict__ a, const float *__restrict__ b,
                                       _Float16 *__restrict__ oa, _Float16 *__restrict__ ob, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        oa[i] = (_Float16)a[i];  // round to nearest even, as __float2half
        ob[i] = (_Float16)b[i];
    }
}

int launch_f32_to_f16_dual(const float *a, const float *b, void *oa, void *ob, int n, hipStream_t s) {
    if (!a || !b || !oa || !ob || n <= 0) return set_error(kErrBadArg, "f32_to_f16_dual: bad arguments");
    hipLaunchKernelGGL(f32_to_f16_dual_kernel, dim3((n + 255) / 256), dim3(256), 0, s, a, b, (_Float16 *)oa,
                       (_Float16 *)ob, n);
    return check_launch("f32_to_f16_dual");
}

void *f16_dual_kernel_ptr() { return reinterpret_cast<void *>(&f32_to_f16_dual_kernel); }

// ------------------------------------------------------------------ RoPE entry point
// cuda_rope launches this kernel.  Its first seven parameters are those of the reference's
// rope_kernel in the same order (kernels.cu:818-822: q, k, head_dim, pos, theta, n_heads_q,
// n_heads_k), because the reference patches parameter 3 (pos) of the captured node before each
// graph replay (forward.c:635-640).  The frequencies 1 / powf(theta, 2j / head_dim) come by value
// after them, computed on the host as the reference does (kernels.cu:1259-1266; it keeps them in
// constant memory).  One thread per rotated pair; the rotation is head_pass_kernel's, bit for bit.
struct RopeFreqs {
    float f[kMaxRopeFreqs];
};

__global__ void __launch_bounds__(256) rope_kernel(float *__restrict__ q, float *__restrict__ k, int head_dim, int pos,
                                                   float theta, int n_heads_q, int n_heads_k, RopeFreqs fr) {
    (void)theta;  // folded into fr
    const int half = head_dim / 2;
    const int tid = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (tid >= (n_heads_q + n_heads_k) * half) return;
    const int head = tid / half, j = tid - head * half;
    float *v = head < n_heads_q ? q + (size_t)head * head_dim : k + (size_t)(head - n_heads_q) * head_dim;
    float sn, cs;
    sincosf((float)pos * fr.f[j], &sn, &cs);
    const float v0 = v[j], v1 = v[j + half];
    v[j] = fmaf(v0, cs, -(v1 * sn));
    v[j + half] = fmaf(v0, sn, v1 * cs);
}

void *rope_kernel_ptr() { return reinterpret_cast<void *>(&rope_kernel); }

int launch_rope(float *q, float *k, int head_dim, int pos, float theta, int nq, int nk, hipStream_t s) {
    if (head_dim <= 0 || (head_dim & 1) || head_dim / 2 > kMaxRopeFreqs || nq < 0 || nk < 0 || nq + nk <= 0 ||
        (nq && !q) || (nk && !k))
        return set_error(kErrBadArg, "rope: need an even head_dim <= %d, heads > 0 and q / k", 2 * kMaxRopeFreqs);
    RopeFreqs fr = {};
    for (int j = 0; j < head_dim / 2; j++) fr.f[j] = 1.0f / powf(theta, (float)(2 * j) / (float)head_dim);
    const int total = (nq + nk) * (head_dim / 2);
    hipLaunchKernelGGL(rope_kernel, dim3((total + 255) / 256), dim3(256), 0, s, q, k, head_dim, pos, theta, nq, nk,
                       fr);
    return check_launch("rope");
}

// ------------------------------------------------------------------ per-head pass
constexpr int kHeadPairs = 4;  // RoPE pairs per lane: head_dim <= 512

__global__ void __launch_bounds__(256) head_pass_kernel(HeadPassArgs a) {
    const int head = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    const int lane = lane_id();
    const int half = a.hd / 2;
    const int nqk = a.nq + a.nk;
    if (head >= nqk + a.nv) return;  // wave-uniform
    const bool is_q = head < a.nq, is_k = !is_q && head < nqk;
    const int h = is_q ? head : (is_k ? head - a.nq : head - nqk);
    const float *src = is_q ? a.q + (size_t)h * a.hd : (is_k ? a.k + (size_t)h * a.hd : a.v + (size_t)h * a.hd);
    // q / k heads are written back only when the pass changes them (a store-only pass reads k)
    const bool writes = (a.flags & (kHeadNorm | kHeadRope)) != 0;
    float *dst = !writes ? nullptr : (is_q ? a.qo + (size_t)h * a.hd : (is_k ? a.ko + (size_t)h * a.hd : nullptr));
    float x0[kHeadPairs], x1[kHeadPairs];
#pragma unroll
    for (int t = 0; t < kHeadPairs; t++) {
        const int j = lane + 64 * t;
        const bool ok = j < half;
        x0[t] = ok ? src[j] : 0.0f;
        x1[t] = ok ? src[j + half] : 0.0f;
    }
    const float *nw = is_q ? a.qw : (is_k ? a.kw : nullptr);
    if ((a.flags & kHeadNorm) && nw) {
        float ss = 0.0f;
#pragma unroll
        for (int t = 0; t < kHeadPairs; t++) ss = fmaf(x0[t], x0[t], fmaf(x1[t], x1[t], ss));
        // the hardware reciprocal square root, as the reference's rsqrtf (kernels.cu:777);
        // the fused decode attention repeats this exact expression
        const float scale = __builtin_amdgcn_rsqf(wave_sum_all(ss) / (float)a.hd + a.eps);
#pragma unroll
        for (int t = 0; t < kHeadPairs; t++) {
            const int j = lane + 64 * t;
            if (j < half) {
                x0[t] = x0[t] * scale * nw[j];
                x1[t] = x1[t] * scale * nw[j + half];
            }
        }
    }
    const int pos = a.pos_dev ? *a.pos_dev : a.pos;
    if ((a.flags & kHeadRope) && (is_q || is_k)) {
#pragma unroll
        for (int t = 0; t < kHeadPairs; t++) {
            const int j = lane + 64 * t;
            if (j < half) {
                const float ang = (float)pos * a.freq[j];
                float sn, cs;
                sincosf(ang, &sn, &cs);
                const float v0 = x0[t], v1 = x1[t];
                // explicit fmas: the fused decode attention repeats this rotation bit for bit
                x0[t] = fmaf(v0, cs, -(v1 * sn));
                x1[t] = fmaf(v0, sn, v1 * cs);
            }
        }
    }
    if (dst) {
#pragma unroll
        for (int t = 0; t < kHeadPairs; t++) {
            const int j = lane + 64 * t;
            if (j < half) {
                dst[j] = x0[t];
                dst[j + half] = x1[t];
            }
        }
    }
    if ((a.flags & kHeadStore) && !is_q) {
        // the cache takes the fp32 values rounded once more (no fma folded into the conversion)
#pragma unroll
        for (int t = 0; t < kHeadPairs; t++) asm volatile("" : "+v"(x0[t]), "+v"(x1[t]));
        // K rows [pos][nk][hd]; V rows likewise, or blocked: element (pos, h, d) at
        // ((pos/64 * nk + h) * hd + d) * 64 + pos % 64 (attention_decode reads it directly)
        const bool blocked = !is_k && a.v_layout == 1;
        const size_t base = blocked ? (((size_t)(pos / 64) * a.nk + h) * a.hd) * 64 + pos % 64
                                    : ((size_t)pos * a.nk + h) * a.hd;
        const int es = blocked ? 64 : 1;  // element stride along the head dim
        void *cache = is_k ? a.kc : a.vc;
        if (a.kv_type == kKvF16) {
            _Float16 *c = (_Float16 *)cache + base;
#pragma unroll
            for (int t = 0; t < kHeadPairs; t++) {
                const int j = lane + 64 * t;
                if (j < half) {
                    c[(size_t)j * es] = (_Float16)x0[t];
                    c[(size_t)(j + half) * es] = (_Float16)x1[t];
                }
            }
        } else {
            float m = 0.0f;
#pragma unroll
            for (int t = 0; t < kHeadPairs; t++) m = fmaxf(m, fmaxf(fabsf(x0[t]), fabsf(x1[t])));
            m = wave_max_all(m);
            const float inv = m > 0.0f ? 127.0f / m : 0.0f;
            int8_t *c = (int8_t *)cache + base;
#pragma unroll
            for (int t = 0; t < kHeadPairs; t++) {
                const int j = lane + 64 * t;
                if (j < half) {
                    c[(size_t)j * es] = (int8_t)fminf(fmaxf(rintf(x0[t] * inv), -127.0f), 127.0f);
                    c[(size_t)(j + half) * es] = (int8_t)fminf(fmaxf(rintf(x1[t] * inv), -127.0f), 127.0f);
                }
            }
            float *sc = is_k ? a.ksc : a.vsc;
            if (lane == 0) sc[(size_t)pos * a.nk + h] = m > 0.0f ? m / 127.0f : 0.0f;
        }
    }
}

int launch_head_pass(HeadPassArgs a, hipStream_t s) {
    const int heads = a.nq + a.nk + a.nv;
    if (a.flags & kHeadRope) {
        if (a.hd / 2 > kMaxRopeFreqs) return set_error(kErrBadArg, "rope: head_dim > %d", 2 * kMaxRopeFreqs);
        for (int j = 0; j < a.hd / 2; j++) a.freq[j] = 1.0f / powf(a.theta, (float)(2 * j) / (float)a.hd);
    }
    if (a.hd <= 0 || (a.hd & 1) || a.hd > 2 * 64 * kHeadPairs || heads <= 0 || a.nq < 0 || a.nk < 0 || a.nv < 0)
        return set_error(kErrBadArg, "head pass: need an even head_dim <= %d and heads > 0", 2 * 64 * kHeadPairs);
    if ((a.nq && !a.q) || (a.nk && !a.k) || (a.nv && !a.v))
        return set_error(kErrBadArg, "head pass: missing q / k / v");
    if (!a.qo) a.qo = a.q;
    if (!a.ko) a.ko = a.k;
    if ((a.flags & kHeadStore) && (((a.nk && !a.kc) || (a.nv && !a.vc)) ||
                                   (a.kv_type == kKvInt8 && ((a.nk && !a.ksc) || (a.nv && !a.vsc)))))
        return set_error(kErrBadArg, "head pass: missing cache pointers");
    if ((a.flags & kHeadStore) && a.nv && a.nk && a.nv != a.nk)
        return set_error(kErrBadArg, "head pass: K and V must have the same number of heads");
    if ((a.flags & kHeadStore) && !a.nk) a.nk = a.nv;  // V-only store: the cache row has nv heads
    hipLaunchKernelGGL(head_pass_kernel, dim3((heads + 3) / 4), dim3(256), 0, s, a);
    return check_launch("head pass");
}

// ------------------------------------------------------------------ attention (entry-point form)
// One 1024-thread workgroup per query head, split-K inside the workgroup: wave w takes the
// positions [w*C, (w+1)*C) of the sequence.  In a wave, G = hd/8 lanes hold 8 dims each of a
// position (16-byte f16 loads) and the wave covers 64/G positions per step (one per lane
// group, "slot"); every slot keeps its own online softmax (running max m, sum l and the
// 8-dim slice of acc), so the loop has no barrier and no cross-slot exchange.  The slots of a
// wave are merged with shuffles and the 16 waves through LDS at the end (the merge of two
// partial softmaxes: m = max, l and acc rescaled by exp(m_i - m)).  The reference runs one
// 256-thread block per head and walks the whole sequence in tiles
// (src/kernels.cu:1382-1481, 1550-1673); the result is the same softmax(q.K^T * scale).V.
constexpr int kAttnThreads = 1024;
constexpr int kAttnWaves = kAttnThreads / 64;
constexpr int kAttnUnroll = 4;  // positions per slot per step (loads in flight)

template <int KV>
__device__ __forceinline__ void load8(const void *cache, size_t off, const float *scales, size_t si, float (&k)[8]) {
    if (KV == kKvF16) {
        uint4 raw;
        __builtin_memcpy(&raw, (const _Float16 *)cache + off, 16);
        const _Float16 *hv = (const _Float16 *)&raw;
#pragma unroll
        for (int i = 0; i < 8; i++) k[i] = (float)hv[i];
    } else {
        uint2 raw;
        __builtin_memcpy(&raw, (const int8_t *)cache + off, 8);
        const int8_t *iv = (const int8_t *)&raw;
        const float sc = scales[si];
#pragma unroll
        for (int i = 0; i < 8; i++) k[i] = (float)iv[i] * sc;
    }
}

template <int KV, int HD>
__global__ void __launch_bounds__(kAttnThreads) attention_kernel(AttnArgs a) {
    constexpr int G = HD / 8;   // lanes per position
    constexpr int S = 64 / G;   // slots (positions per wave step)
    __shared__ float wm[kAttnWaves], wl[kAttnWaves];
    __shared__ float wacc[kAttnWaves][HD];
    const int head = blockIdx.x, kvh = head / a.gqa, tid = threadIdx.x, lane = lane_id();
    const int wave = tid >> 6, gi = lane % G, slot = lane / G;
    const int seq = (a.seq_dev ? *a.seq_dev : 0) + a.seq;
    const size_t stride = (size_t)a.nkv * HD;
    float q[8];
#pragma unroll
    for (int e = 0; e < 8; e++) q[e] = a.q[(size_t)head * HD + 8 * gi + e] * a.scale;
    const int chunk = (seq + kAttnWaves - 1) / kAttnWaves;
    const int p0 = wave * chunk, p1 = min(seq, p0 + chunk);
    float m = -INFINITY, l = 0.0f, acc[8] = {};
    for (int pb = p0; pb < p1; pb += S * kAttnUnroll) {
        float s[kAttnUnroll], v[kAttnUnroll][8];
#pragma unroll
        for (int u = 0; u < kAttnUnroll; u++) {
            const int p = pb + u * S + slot;
            const int pc = min(p, p1 - 1);  // past the chunk: the last position again, masked below
            float k[8];
            load8<KV>(a.kc, (size_t)pc * stride + (size_t)kvh * HD + 8 * gi, a.ksc, (size_t)pc * a.nkv + kvh, k);
            load8<KV>(a.vc, (size_t)pc * stride + (size_t)kvh * HD + 8 * gi, a.vsc, (size_t)pc * a.nkv + kvh, v[u]);
            float d = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) d = fmaf(q[e], k[e], d);
#pragma unroll
            for (int o = G / 2; o > 0; o >>= 1) d += __shfl_xor(d, o);
            s[u] = p < p1 ? d : -INFINITY;
        }
        float mt = m;
#pragma unroll
        for (int u = 0; u < kAttnUnroll; u++) mt = fmaxf(mt, s[u]);
        if (mt == -INFINITY) continue;  // nothing valid in this slot yet (uniform per slot)
        const float r = expf(m - mt);   // m = -inf: 0
        l *= r;
#pragma unroll
        for (int e = 0; e < 8; e++) acc[e] *= r;
#pragma unroll
        for (int u = 0; u < kAttnUnroll; u++) {
            const float w = expf(s[u] - mt);
            l += w;
#pragma unroll
            for (int e = 0; e < 8; e++) acc[e] = fmaf(w, v[u][e], acc[e]);
        }
        m = mt;
    }
    // merge the slots of the wave (lanes gi + G * slot)
#pragma unroll
    for (int o = G; o < 64; o <<= 1) {
        const float mo = __shfl_xor(m, o), lo = __shfl_xor(l, o);
        const float mn = fmaxf(m, mo);
        const float ra = mn == -INFINITY ? 0.0f : expf(m - mn), rb = mn == -INFINITY ? 0.0f : expf(mo - mn);
        l = l * ra + lo * rb;
#pragma unroll
        for (int e = 0; e < 8; e++) acc[e] = acc[e] * ra + __shfl_xor(acc[e], o) * rb;
        m = mn;
    }
    if (slot == 0) {
#pragma unroll
        for (int e = 0; e < 8; e++) wacc[wave][8 * gi + e] = acc[e];
        if (gi == 0) {
            wm[wave] = m;
            wl[wave] = l;
        }
    }
    __syncthreads();
    // merge the waves: thread d < HD owns output dim d
    if (tid < HD) {
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < kAttnWaves; w++) mx = fmaxf(mx, wm[w]);
        float lt = 0.0f, o = 0.0f;
#pragma unroll
        for (int w = 0; w < kAttnWaves; w++) {
            const float r = wm[w] == -INFINITY ? 0.0f : expf(wm[w] - mx);
            lt = fmaf(wl[w], r, lt);
            o = fmaf(wacc[w][tid], r, o);
        }
        a.out[(size_t)head * HD + tid] = seq > 0 && lt > 0.0f ? o / lt : 0.0f;
    }
}

int launch_attention(AttnArgs a, int kv_type, hipStream_t s) {
    if (!a.q || !a.kc || !a.vc || !a.out || a.nh <= 0 || a.nkv <= 0 || a.gqa <= 0 || a.nh != a.nkv * a.gqa)
        return set_error(kErrBadArg, "attention: bad pointers or head counts (n_heads must be n_kv_heads * gqa)");
    if (!(a.hd == 64 || a.hd == 128 || a.hd == 256))
        return set_error(kErrBadArg, "attention: head_dim %d not supported (64, 128, 256)", a.hd);
    if (a.seq < 0) return set_error(kErrBadArg, "attention: seq_len < 0");
    if (kv_type == kKvInt8 && (!a.ksc || !a.vsc)) return set_error(kErrBadArg, "attention: int8 cache needs scales");
#define MNEMO_ATTN(HD_)                                                                                  \
    do {                                                                                                 \
        if (kv_type == kKvF16) hipLaunchKernelGGL((attention_kernel<kKvF16, HD_>), dim3(a.nh), dim3(kAttnThreads), 0, s, a); \
        else hipLaunchKernelGGL((attention_kernel<kKvInt8, HD_>), dim3(a.nh), dim3(kAttnThreads), 0, s, a); \
    } while (0)
    if (a.hd == 64) MNEMO_ATTN(64);
    else if (a.hd == 128) MNEMO_ATTN(128);
    else MNEMO_ATTN(256);
#undef MNEMO_ATTN
    return check_launch("attention");
}

}  // namespace mnemo
