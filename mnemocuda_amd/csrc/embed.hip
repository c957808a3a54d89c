// embed.hip -- token embedding lookup from the resident table (MnemoCUDA forward.c:1145-1280,
// GPU path kernels.cu:1901-1951, wrapper kernels.cu:2192-2198).
//
// One workgroup of 256 threads dequantises one row of the table into the hidden vector;
// thread t owns 16 consecutive values of each 4096-value stretch.  The values are the
// canonical GGUF decode (value v of a Q4_K block: byte qs[32 (v/64) + v%32], low nibble
// for v%64 < 32), which is what the reference's matvec kernels and its CPU embedding
// fallback (forward.c:1189-1229) compute; the reference's GPU embedding kernel indexes the
// nibbles as qs[(j/2) % 64] and disagrees with both, so it is not followed.  Arithmetic as
// the oracle: (d*sc)*q - dmin*m in fp32 (each product exact), Q6_K (d*sc)*(q-32).
// mnemo_embedding_lookup reads the token id from device memory, so the sampled token of
// one decode step feeds the next step's embedding inside one captured graph.
#include "mnemo_common.hpp"
#include "mnemo_internal.hpp"

namespace mnemo {

constexpr int kEmbThreads = 256;

__device__ __forceinline__ void scale_min(const uint8_t *s, int j, int &sc, int &m) {
    if (j < 4) {
        sc = s[j] & 63;
        m = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

__global__ void __launch_bounds__(kEmbThreads) embed_kernel(const uint8_t *__restrict__ table, int type,
                                                            const int *__restrict__ tok_dev, int tok, int n_vocab,
                                                            float *__restrict__ out, int hidden, size_t row_bytes) {
    int t = tok_dev ? *tok_dev : tok;
    t = min(max(t, 0), n_vocab - 1);  // an id outside the table reads its nearest row
    const uint8_t *row = table + (size_t)t * row_bytes;
    for (int v0 = 16 * threadIdx.x; v0 < hidden; v0 += 16 * kEmbThreads) {
        const int b = v0 / 256, j = v0 % 256;  // 16 values inside one block
        if (type == kTypeF32) {
#pragma unroll
            for (int i = 0; i < 16; i++)
                if (v0 + i < hidden) out[v0 + i] = ((const float *)row)[v0 + i];
        } else if (type == kTypeQ4K) {
            const uint8_t *blk = row + (size_t)b * kQ4KBytes;
            uint16_t dh, mh;
            __builtin_memcpy(&dh, blk, 2);
            __builtin_memcpy(&mh, blk + 2, 2);
            const float d = h2f(dh), dmin = h2f(mh);
            int sc, m;
            scale_min(blk + 4, j / 32, sc, m);
            const float d1 = d * (float)sc, m1 = dmin * (float)m;
            const int g = j / 64, hi = (j % 64) >= 32, l0 = j % 32;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint8_t q = blk[16 + 32 * g + l0 + i];
                if (v0 + i < hidden) out[v0 + i] = d1 * (float)(hi ? q >> 4 : q & 15) - m1;
            }
        } else {
            const uint8_t *blk = row + (size_t)b * kQ6KBytes;
            uint16_t dh;
            __builtin_memcpy(&dh, blk + 208, 2);
            const float s = h2f(dh) * (float)(int8_t)blk[192 + j / 16];
            const int h = j / 128, u = j % 128, grp = u / 32, l0 = u % 32;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int l = l0 + i;
                const int lo4 = (blk[64 * h + 32 * (grp & 1) + l] >> (grp >= 2 ? 4 : 0)) & 15;
                const int hi2 = (blk[128 + 32 * h + l] >> (2 * grp)) & 3;
                if (v0 + i < hidden) out[v0 + i] = s * (float)(((hi2 << 4) | lo4) - 32);
            }
        }
    }
}

int launch_embedding(const void *table, int type, const int *tok_dev, int tok, int n_vocab, float *out, int hidden,
                     size_t row_bytes, hipStream_t s) {
    if (!table || !out || hidden <= 0 || n_vocab <= 0 || (!tok_dev && (tok < 0 || tok >= n_vocab)))
        return set_error(kErrBadArg, "embedding: bad arguments (token %d of %d)", tok, n_vocab);
    if (type != kTypeF32 && type != kTypeQ4K && type != kTypeQ6K)
        return set_error(kErrUnsupportedType, "embedding: type %d (F32, Q4_K, Q6_K)", type);
    hipLaunchKernelGGL(embed_kernel, dim3(1), dim3(kEmbThreads), 0, s, (const uint8_t *)table, type, tok_dev, tok,
                       n_vocab, out, hidden, row_bytes);
    return check_launch("embedding");
}

}  // namespace mnemo
