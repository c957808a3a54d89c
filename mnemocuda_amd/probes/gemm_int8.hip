// gemm_int8.hip -- the Q4_K x Q8_1 prefill GEMM on gfx950 int8 matrix cores, measured
// beside the library's exact-f16 kernel (a measurement program for the design notes; not
// part of the library).
//
// Same tiling, loaders, pipeline, running scales and epilogue as gemm_q8_1_kernel in
// csrc/gemm.hip; what differs is the operand form of a 32-value sub-block:
//   library:  A = sc * q as exact f16 integers, B = q8 as f16, one v_mfma_f32_16x16x32_f16
//             accumulating into acc * rho (one multiply per output and sub-block);
//   here:     A = q (4-bit) and B = q8 as int8 bytes (no conversion: the quants are copied),
//             v_mfma_i32_16x16x32_i8 into a fresh int32 tile t, then
//             acc = fma(acc, rho, sc * float(t)) per output (convert, multiply, fma).
// Both give the reference's integer sub-block sums (gemm_q4k.cu:103-112); the outputs agree
// to fp32 rounding.  Q4_K only, one K split, M and N multiples of 128.
//
// Build: hipcc -O3 -std=c++17 --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops
//        -I mnemocuda_amd/csrc mnemocuda_amd/probes/gemm_int8.hip -o gemm_int8
// Prints, for M = 8192 weight rows, K = 4096, N = 512 tokens (the benchmark's prefill GEMM; one
// K split in both kernels): the time per launch of both kernels (HIP events, 40 launches
// over 8 copies of the weights) and the relative L2 difference between their outputs.
#include "gemm.hip"

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

namespace mnemo {
int set_error(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vfprintf(stderr, fmt, ap);
    va_end(ap);
    fputc('\n', stderr);
    return code;
}
int check_launch(const char *what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        fprintf(stderr, "launch %s: %s\n", what, hipGetErrorString(e));
        return kErrLaunch;
    }
    return kOk;
}

namespace int8probe {
typedef int i4v __attribute__((ext_vector_type(4)));

// One LDS stage: byte tiles of 64 K per row (8-byte units XOR-swizzled by row), the token
// ratios, the row ratios and the 6-bit scales of the step's two sub-blocks per row.
struct Stage8 {
    uint8_t a[kBM * kKS];
    uint8_t b[kBN * kKS];
    float rho[2][kBN];
    float sig[kBM];
    float sc[2][kBM];
    uint8_t pad[4096];  // three stages hold the 64 KB that the parity reduction reuses
};
static_assert(3 * sizeof(Stage8) >= sizeof(float) * (kWaves / 2) * 64 * kWTok, "reduction area");
__device__ __forceinline__ int off8(int row, int k8) { return row * kKS + ((k8 ^ (row & 7)) << 3); }

__device__ __forceinline__ void store_w(const RawW &r, int ks, int p, Stage8 &st, int row, LoaderState &ls,
                                        bool live) {
    const int c = kVP * p;
    const int j = 2 * (ks & 3) + (c >> 5);
    uint32_t sc, m;
    q4k_scale_min(r.h.y, r.h.z, r.h.w, j, sc, m);
    const float d = h2f(r.h.x & 0xFFFFu);
    if (d == 0.0f) sc = 0;
    const int sh = 4 * (c >> 5);
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; k++) o[k] = (r.a.w[k] >> sh) & 0x0F0F0F0Fu;
    *(uint2 *)(st.a + off8(row, c >> 3)) = make_uint2(o[0], o[1]);
    *(uint2 *)(st.a + off8(row, (c >> 3) + 1)) = make_uint2(o[2], o[3]);
    if ((c & 31) == 0) st.sc[c >> 5][row] = (float)sc;
    if (p == 0 && (ks & 3) == 0 && live) {
        const float dn = d != 0.0f ? d : ls.deff;
        st.sig[row] = ls.deff * __builtin_amdgcn_rcpf(dn);
        ls.deff = dn;
    }
}

__device__ __forceinline__ void store_a8(const RawA &r, int p, Stage8 &st, int row, LoaderState &ls, bool live) {
    const float d8 = h2f(r.ds & 0xFFFFu);
    const bool zero = d8 == 0.0f;
    const int c = kVP * p;
    *(uint2 *)(st.b + off8(row, c >> 3)) = make_uint2(zero ? 0u : r.q.w[0], zero ? 0u : r.q.w[1]);
    *(uint2 *)(st.b + off8(row, (c >> 3) + 1)) = make_uint2(zero ? 0u : r.q.w[2], zero ? 0u : r.q.w[3]);
    if ((c & 31) == 0 && live) {
        const float dn = zero ? ls.d8eff : d8;
        st.rho[c >> 5][row] = ls.d8eff * __builtin_amdgcn_rcpf(dn);
        ls.d8eff = dn;
    }
}

struct Frags8 {
    long a[4], b[kNB];
    f4 sc[4];
    float rho[kNB];
};

__device__ __forceinline__ void read_frags8(const Stage8 &st, int wi, int wj, int kh, int lane, Frags8 &f) {
    const int k8 = 4 * kh + (lane >> 4);
#pragma unroll
    for (int t = 0; t < 4; t++) {
        f.a[t] = *(const long *)(st.a + off8(wi + 16 * t + (lane & 15), k8));
        f.sc[t] = *(const f4 *)(st.sc[kh] + wi + 16 * t + 4 * (lane >> 4));
    }
#pragma unroll
    for (int t = 0; t < kNB; t++) {
        const int rb = wj + 16 * t + (lane & 15);
        f.b[t] = *(const long *)(st.b + off8(rb, k8));
        f.rho[t] = st.rho[kh][rb];
    }
}

__device__ __forceinline__ void mfma_step8(const Frags8 &f, const Stage8 &st, int wi, int lane, f4 (&acc)[4][kNB],
                                           bool sb_start) {
    if (sb_start) {
#pragma unroll
        for (int a = 0; a < 4; a++) {
            const f4 sg = *(const f4 *)(st.sig + wi + 16 * a + 4 * (lane >> 4));
#pragma unroll
            for (int b = 0; b < kNB; b++) acc[a][b] *= sg;
        }
    }
#pragma unroll
    for (int b = 0; b < kNB; b++)
#pragma unroll
        for (int a = 0; a < 4; a++) {
            const i4v t = __builtin_amdgcn_mfma_i32_16x16x32_i8(f.a[a], f.b[b], i4v{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int e = 0; e < 4; e++) acc[a][b][e] = fmaf(acc[a][b][e], f.rho[b], f.sc[a][e] * (float)t[e]);
        }
}

__global__ void __launch_bounds__(kThreads) gemm_q4k_int8_kernel(GemmArgs g) {
    __shared__ __align__(16) Stage8 lds[3];
    __shared__ float dlast[kBM], d8last[2][kBN];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int K = g.K;
    const int wi = (wave & 1) * 64, wj = ((wave >> 1) % kWC) * kWTok, kh = wave / (2 * kWC);
    const size_t wrow_bytes = (size_t)(K / 256) * kQ4KBytes;
    const int sb0 = 0, sb1 = K / 256;
    const int ks0 = 0, ks1 = 4 * sb1, last = ks1 - 1;
    const int i0 = blockIdx.x * kBM, j0 = blockIdx.y * kBN;
    const int lr = tid / kParts, lp = tid % kParts;
    const uint8_t *wrow = g.W + (size_t)min(i0 + lr, g.M - 1) * wrow_bytes;
    const uint8_t *arow = (const uint8_t *)g.A + (size_t)min(j0 + lr, g.N - 1) * (K / 128) * kQ81Bytes;
    LoaderState ls{1.0f, 1.0f};
    f4 acc[4][kNB];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < kNB; b++) acc[a][b] = f4{0.f, 0.f, 0.f, 0.f};

    RawW rw[kPF];
    RawA ra[kPF];
#pragma unroll
    for (int p = 0; p < kPF; p++) load_step<kTypeQ4K>(wrow, arow, min(ks0 + p, last), lp, rw[p], ra[p]);
    store_w(rw[0], ks0, lp, lds[0], lr, ls, true);
    store_a8(ra[0], lp, lds[0], lr, ls, true);
    store_w(rw[1], ks0 + 1, lp, lds[1], lr, ls, ks0 + 1 < ks1);
    store_a8(ra[1], lp, lds[1], lr, ls, ks0 + 1 < ks1);
    lds_barrier();
    Frags8 fr;
    read_frags8(lds[0], wi, wj, kh, lane, fr);
    for (int kb = ks0; kb < ks1; kb += kUnroll) {
#pragma unroll
        for (int p = 0; p < kUnroll; p++) {
            const int ks = kb + p;
            if (ks < ks1) {
                const int r = p % kPF, b = p % 3;
                load_step<kTypeQ4K>(wrow, arow, min(ks + kPF, last), lp, rw[r], ra[r]);
                mfma_step8(fr, lds[b], wi, lane, acc, p % 4 == 0);
                read_frags8(lds[(b + 1) % 3], wi, wj, kh, lane, fr);
                store_w(rw[(r + 2) % kPF], ks + 2, lp, lds[(b + 2) % 3], lr, ls, ks + 2 < ks1);
                store_a8(ra[(r + 2) % kPF], lp, lds[(b + 2) % 3], lr, ls, ks + 2 < ks1);
                lds_barrier();
            }
        }
    }
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
    // the min term, as in the library kernel
    const int q = lane >> 4;
    const int nwin = (sb1 - sb0 + 3) / 4;
    for (int w = kh; w < nwin; w += 2) {
        const int sb = sb0 + 4 * w + q;
        const bool valid = sb < sb1;
        uint4 hdr[4], blk[kNB][2];
#pragma unroll
        for (int a = 0; a < 4; a++) {
            const uint8_t *rp = g.W + (size_t)min(i0 + wi + 16 * a + (lane & 15), g.M - 1) * wrow_bytes;
            hdr[a] = valid ? ld16(rp + (size_t)sb * kQ4KBytes) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int b = 0; b < kNB; b++) {
            const uint8_t *ap =
                (const uint8_t *)g.A + (size_t)min(j0 + wj + 16 * b + (lane & 15), g.N - 1) * (K / 128) * kQ81Bytes;
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
    // the two parities meet through the idle stages
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
        for (int b = 0; b < kNB; b++) {
#pragma unroll
            for (int e = 0; e < 4; e++) acc[a][b][e] += red[((a * kNB + b) * 4 + e) * 64 + lane];
            const int j = j0 + wj + 16 * b + (lane & 15);
            const int ib = i0 + wi + 16 * a + 4 * (lane >> 4);
            *(f4 *)(g.out + (size_t)j * g.out_ld + ib) = acc[a][b];
        }
}
}  // namespace int8probe
}  // namespace mnemo

static uint16_t f16_bits(float f) {
    const _Float16 h = (_Float16)f;
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}

int main() {
    using namespace mnemo;
    const int K = 4096, N = 512, NW = 8, reps = 40;
    std::mt19937 rng(1);
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return 1;
    for (int M : {8192}) {
        const size_t wbytes = (size_t)M * (K / 256) * kQ4KBytes, abytes = (size_t)N * (K / 128) * kQ81Bytes;
        std::vector<uint8_t> w(wbytes), a(abytes);
        for (auto &v : w) v = (uint8_t)rng();
        for (auto &v : a) v = (uint8_t)rng();
        std::uniform_real_distribution<float> ud(0.005f, 0.02f);
        for (size_t b = 0; b < wbytes / kQ4KBytes; b++) {
            const uint16_t d = f16_bits(ud(rng)), dm = f16_bits(ud(rng));
            std::memcpy(&w[b * kQ4KBytes], &d, 2);
            std::memcpy(&w[b * kQ4KBytes + 2], &dm, 2);
        }
        for (size_t b = 0; b < abytes / kQ81Bytes; b++)
            for (int s = 0; s < 4; s++) {
                const uint16_t d = f16_bits(ud(rng)), ds = f16_bits(ud(rng) * 10.0f);
                std::memcpy(&a[b * kQ81Bytes + 4 * s], &d, 2);
                std::memcpy(&a[b * kQ81Bytes + 4 * s + 2], &ds, 2);
            }
        std::vector<uint8_t *> dw(NW);
        uint8_t *da = nullptr;
        float *o16 = nullptr, *o8 = nullptr;
        for (auto &p : dw)
            if (hipMalloc(&p, wbytes) != hipSuccess || hipMemcpy(p, w.data(), wbytes, hipMemcpyHostToDevice) != hipSuccess)
                return 1;
        if (hipMalloc(&da, abytes) != hipSuccess || hipMemcpy(da, a.data(), abytes, hipMemcpyHostToDevice) != hipSuccess ||
            hipMalloc(&o16, (size_t)M * N * 4) != hipSuccess || hipMalloc(&o8, (size_t)M * N * 4) != hipSuccess)
            return 1;
        auto int8_launch = [&](const uint8_t *wd, float *out) {
            GemmArgs g{};
            g.W = wd;
            g.A = da;
            g.out = out;
            g.M = M;
            g.K = K;
            g.N = N;
            g.splits = 1;
            g.out_ld = M;
            hipLaunchKernelGGL(int8probe::gemm_q4k_int8_kernel, dim3(M / kBM, N / kBN), dim3(kThreads), 0, 0, g);
            return check_launch("int8 probe");
        };
        if (launch_gemm_q8_1(kTypeQ4K, dw[0], da, o16, M, K, N, 0) || int8_launch(dw[0], o8) ||
            hipDeviceSynchronize() != hipSuccess)
            return 1;
        std::vector<float> r16((size_t)M * N), r8((size_t)M * N);
        if (hipMemcpy(r16.data(), o16, r16.size() * 4, hipMemcpyDeviceToHost) != hipSuccess ||
            hipMemcpy(r8.data(), o8, r8.size() * 4, hipMemcpyDeviceToHost) != hipSuccess)
            return 1;
        double num = 0, den = 0;
        for (size_t i = 0; i < r16.size(); i++) {
            num += ((double)r8[i] - r16[i]) * ((double)r8[i] - r16[i]);
            den += (double)r16[i] * r16[i];
        }
        float t[2];
        for (int v = 0; v < 2; v++) {
            for (int i = 0; i < NW; i++) v ? int8_launch(dw[i], o8) : launch_gemm_q8_1(kTypeQ4K, dw[i], da, o16, M, K, N, 0);
            if (hipEventRecord(e0) != hipSuccess) return 1;
            for (int i = 0; i < reps; i++)
                v ? int8_launch(dw[i % NW], o8) : launch_gemm_q8_1(kTypeQ4K, dw[i % NW], da, o16, M, K, N, 0);
            if (hipEventRecord(e1) != hipSuccess || hipEventSynchronize(e1) != hipSuccess) return 1;
            float ms = 0.0f;
            if (hipEventElapsedTime(&ms, e0, e1) != hipSuccess) return 1;
            t[v] = ms * 1e3f / reps;
        }
        const double ops = 2.0 * M * N * K;
        printf("M=%d K=%d N=%d  exact-f16 MFMA: %.2f us (%.1f TOPS)  int8 MFMA: %.2f us (%.1f TOPS)  "
               "relative L2 difference %.2e\n",
               M, K, N, t[0], ops / t[0] / 1e6, t[1], ops / t[1] / 1e6, std::sqrt(num / den));
        for (auto p : dw) (void)hipFree(p);
        (void)hipFree(da);
        (void)hipFree(o16);
        (void)hipFree(o8);
    }
    return 0;
}
