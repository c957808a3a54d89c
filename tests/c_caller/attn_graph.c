/*
 * attn_graph.c -- the reference engine's attention-graph path, in plain C against the
 * library's C-ABI: build_attention_graphs (MnemoCUDA src/forward.c:1290-1420) captures one
 * layer's attention chain in a graph, finds the RoPE, f16 KV-store and attention nodes by the
 * function pointers cuda_get_*_kernel_ptr return, and forward_layer (forward.c:633-668)
 * patches them before every replay: RoPE parameter 3 = pos, KV-store parameters 2 and 3 =
 * the cache rows of pos, attention parameter 6 = pos + 1.
 *
 * The chain per token (forward.c:1333-1383): rms_norm_residual(hidden) -> q4k_qkv ->
 * rms_norm_qk -> rope -> f32_to_f16_dual (K, V rows of pos) -> attention_f16kv -> q4k_add
 * (O + residual -> hidden).  The cache rows before P0 hold seeded f16 values (a long prompt),
 * so the decoded tokens attend over P0 + 1 .. P0 + NTOK positions -- more 64-position chunks
 * than the attention kernel has workgroups per KV head, which makes workgroups take several.
 *
 * The same NTOK tokens run twice on fresh caches: through the patched graph and eagerly.
 * Written to the output file (little endian): int32 H, NH, NKV, HD, P0, NTOK, CTX, then the
 * inputs Wq, Wk, Wv (Q4_K), Wo (Q4_K), attn_norm[H], q_norm[HD], k_norm[HD], hidden_in[NTOK][H],
 * the f16 caches K, V [CTX][NKV][HD] before the run, then for each mode (graph, eager): per
 * token q[NH*HD] and k[NKV*HD] after the norm and RoPE, v[NKV*HD], attn_out[NH*HD],
 * hidden_out[H]; then the final caches K, V.  tests/test_gpu_attn_graph.py checks them.
 * Exit status 0 on success, 1 on a HIP or library error, 2 when a node is not found.
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/mnemo_kernels.h"

#define H 512
#define NH 8
#define NKV 2
#define HD 128
#define P0 9000 /* positions already in the cache */
#define NTOK 24
#define CTX (P0 + NTOK + 8)
#define THETA 1000000.0f
#define EPS 1e-6f
#define Q4B(cols) ((size_t)((cols) / 256) * 144)

static uint64_t lcg = 0x2545F4914F6CDD1Dull;
static uint32_t next32(void) {
    lcg = lcg * 6364136223846793005ull + 1442695040888963407ull;
    return (uint32_t)(lcg >> 32);
}
static float uniform(void) { return (float)(next32() >> 8) * (1.0f / 16777216.0f); }
static uint16_t small_f16(void) { return (uint16_t)(0x1C00 | (next32() & 0x3FF)); }
static void fill_q4k(uint8_t *w, size_t rows, int cols) {
    for (size_t b = 0; b < rows * (size_t)(cols / 256); b++) {
        uint8_t *blk = w + b * 144;
        uint16_t d = small_f16(), dmin = small_f16();
        memcpy(blk, &d, 2);
        memcpy(blk + 2, &dmin, 2);
        for (int i = 4; i < 144; i++) blk[i] = (uint8_t)next32();
    }
}
static uint16_t kv_f16(void) { return (uint16_t)((next32() & 0x8000u) | (0x3000u + next32() % 0x0C00u)); }

#define CK(x)                                                                          \
    do {                                                                               \
        hipError_t e_ = (x);                                                           \
        if (e_ != hipSuccess) {                                                        \
            fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
            return 1;                                                                  \
        }                                                                              \
    } while (0)

static void *upload(const void *h, size_t n) {
    void *d = NULL;
    if (hipMalloc(&d, n) != hipSuccess || hipMemcpy(d, h, n, hipMemcpyHostToDevice) != hipSuccess) return NULL;
    return d;
}

/* device state of the layer, as the engine's GPUState holds it */
static void *d_wq, *d_wk, *d_wv, *d_wo;
static float *d_anorm, *d_qn, *d_kn, *d_hidden, *d_normed, *d_residual, *d_q, *d_k, *d_v, *d_attn;
static void *d_kv_k, *d_kv_v;
static hipStream_t cs;

/* forward.c:1336-1383 with the host values of this token (the eager path and the capture) */
static void layer_calls(int pos, void *kdst, void *vdst, int seq_len) {
    cuda_rms_norm_residual(d_hidden, d_anorm, d_normed, d_residual, H, EPS, cs);
    cuda_matvec_q4k_qkv(d_wq, d_wk, d_wv, d_normed, d_q, d_k, d_v, NH * HD, NKV * HD, H, cs);
    cuda_rms_norm_qk(d_q, d_k, d_qn, d_kn, HD, NH, NKV, EPS, cs);
    cuda_rope(d_q, d_k, HD, pos, THETA, NH, NKV, cs);
    cuda_f32_to_f16_dual(d_k, d_v, kdst, vdst, NKV * HD, cs);
    cuda_attention_f16kv(d_q, d_kv_k, d_kv_v, d_attn, NH, HD, NKV, seq_len, NH / NKV,
                         1.0f / sqrtf((float)HD), cs);
    cuda_matvec_q4k_add(d_wo, d_attn, d_residual, d_hidden, H, NH * HD, cs);
}

static int dump_token(FILE *f) {
    static float q[NH * HD], k[NKV * HD], v[NKV * HD], att[NH * HD], hid[H];
    CK(hipStreamSynchronize(cs));
    CK(hipMemcpy(q, d_q, sizeof q, hipMemcpyDeviceToHost));
    CK(hipMemcpy(k, d_k, sizeof k, hipMemcpyDeviceToHost));
    CK(hipMemcpy(v, d_v, sizeof v, hipMemcpyDeviceToHost));
    CK(hipMemcpy(att, d_attn, sizeof att, hipMemcpyDeviceToHost));
    CK(hipMemcpy(hid, d_hidden, sizeof hid, hipMemcpyDeviceToHost));
    fwrite(q, 1, sizeof q, f);
    fwrite(k, 1, sizeof k, f);
    fwrite(v, 1, sizeof v, f);
    fwrite(att, 1, sizeof att, f);
    fwrite(hid, 1, sizeof hid, f);
    return 0;
}

int main(int argc, char **argv) {
    if (argc != 2) {
        fprintf(stderr, "usage: %s out.bin\n", argv[0]);
        return 1;
    }
    FILE *f = fopen(argv[1], "wb");
    if (!f) return 1;
    CK(hipSetDevice(0));
    cuda_kernels_init();
    if (mnemo_last_error()) return 1;
    CK(hipStreamCreate(&cs));

    const size_t nq = Q4B(H) * NH * HD, nk = Q4B(H) * NKV * HD, no = Q4B(NH * HD) * H;
    const size_t ncache = (size_t)CTX * NKV * HD;
    uint8_t *wq = malloc(nq), *wk = malloc(nk), *wv = malloc(nk), *wo = malloc(no);
    float *anorm = malloc(H * 4), *qn = malloc(HD * 4), *kn = malloc(HD * 4), *hin = malloc((size_t)NTOK * H * 4);
    uint16_t *kc0 = calloc(ncache, 2), *vc0 = calloc(ncache, 2), *cache = malloc(ncache * 2);
    if (!wq || !wk || !wv || !wo || !anorm || !qn || !kn || !hin || !kc0 || !vc0 || !cache) return 1;
    fill_q4k(wq, NH * HD, H);
    fill_q4k(wk, NKV * HD, H);
    fill_q4k(wv, NKV * HD, H);
    fill_q4k(wo, H, NH * HD);
    for (int i = 0; i < H; i++) anorm[i] = 0.5f + uniform();
    for (int i = 0; i < HD; i++) qn[i] = 0.5f + uniform();
    for (int i = 0; i < HD; i++) kn[i] = 0.5f + uniform();
    for (int i = 0; i < NTOK * H; i++) hin[i] = 2.0f * uniform() - 1.0f;
    for (size_t i = 0; i < (size_t)P0 * NKV * HD; i++) {
        kc0[i] = kv_f16();
        vc0[i] = kv_f16();
    }
    const int hdr[7] = {H, NH, NKV, HD, P0, NTOK, CTX};
    fwrite(hdr, 4, 7, f);
    fwrite(wq, 1, nq, f);
    fwrite(wk, 1, nk, f);
    fwrite(wv, 1, nk, f);
    fwrite(wo, 1, no, f);
    fwrite(anorm, 4, H, f);
    fwrite(qn, 4, HD, f);
    fwrite(kn, 4, HD, f);
    fwrite(hin, 4, (size_t)NTOK * H, f);
    fwrite(kc0, 2, ncache, f);
    fwrite(vc0, 2, ncache, f);

    d_wq = upload(wq, nq);
    d_wk = upload(wk, nk);
    d_wv = upload(wv, nk);
    d_wo = upload(wo, no);
    d_anorm = upload(anorm, H * 4);
    d_qn = upload(qn, HD * 4);
    d_kn = upload(kn, HD * 4);
    if (!d_wq || !d_wk || !d_wv || !d_wo || !d_anorm || !d_qn || !d_kn) return 1;
    CK(hipMalloc((void **)&d_hidden, H * 4));
    CK(hipMalloc((void **)&d_normed, H * 4));
    CK(hipMalloc((void **)&d_residual, H * 4));
    CK(hipMalloc((void **)&d_q, NH * HD * 4));
    CK(hipMalloc((void **)&d_k, NKV * HD * 4));
    CK(hipMalloc((void **)&d_v, NKV * HD * 4));
    CK(hipMalloc((void **)&d_attn, NH * HD * 4));
    CK(hipMalloc(&d_kv_k, ncache * 2));
    CK(hipMalloc(&d_kv_v, ncache * 2));

    void *rope_fn = cuda_get_rope_kernel_ptr();
    void *f16d_fn = cuda_get_f16dual_kernel_ptr();
    void *attn_fn = cuda_get_attn_f16kv_kernel_ptr();
    const size_t row = (size_t)NKV * HD * 2; /* bytes of one cache row */

    for (int mode = 0; mode < 2; mode++) { /* 0: patched graph, 1: eager */
        CK(hipMemcpy(d_kv_k, kc0, ncache * 2, hipMemcpyHostToDevice));
        CK(hipMemcpy(d_kv_v, vc0, ncache * 2, hipMemcpyHostToDevice));
        hipGraph_t graph = NULL;
        hipGraphExec_t exec = NULL;
        hipGraphNode_t rope_node = NULL, kvst_node = NULL, attn_node = NULL;
        hipKernelNodeParams rope_p, kvst_p, attn_p;
        /* parameter counts of the three kernels: rope (q, k, head_dim, pos, theta, n_q, n_k,
         * freqs), KV store (a, b, oa, ob, n), attention (q, kv_k, kv_v, out, head_dim, n_kv,
         * seq_len, gqa, scale, workspace, nsplit, k_scales, v_scales) */
        void *rope_args[8], *kvst_args[5], *attn_args[13];
        /* the values the patched parameters point at (forward.c's attn_*_buf) */
        int pos_buf = 0, seqlen_buf = 1;
        void *kdst_buf = d_kv_k, *vdst_buf = d_kv_v;
        if (mode == 0) {
            /* build_attention_graphs: capture with pos 0, the row-0 destinations, seq_len 1 */
            CK(hipStreamBeginCapture(cs, hipStreamCaptureModeGlobal));
            layer_calls(pos_buf, kdst_buf, vdst_buf, seqlen_buf);
            CK(hipStreamEndCapture(cs, &graph));
            if (mnemo_last_error()) return 1;
            size_t n_nodes = 0;
            CK(hipGraphGetNodes(graph, NULL, &n_nodes));
            hipGraphNode_t *nodes = malloc(n_nodes * sizeof *nodes);
            CK(hipGraphGetNodes(graph, nodes, &n_nodes));
            for (size_t i = 0; i < n_nodes; i++) {
                hipGraphNodeType type;
                CK(hipGraphNodeGetType(nodes[i], &type));
                if (type != hipGraphNodeTypeKernel) continue;
                hipKernelNodeParams kp;
                memset(&kp, 0, sizeof kp);
                CK(hipGraphKernelNodeGetParams(nodes[i], &kp));
                if (kp.func == rope_fn) {
                    rope_node = nodes[i];
                    rope_p = kp;
                } else if (kp.func == f16d_fn) {
                    kvst_node = nodes[i];
                    kvst_p = kp;
                } else if (kp.func == attn_fn) {
                    attn_node = nodes[i];
                    attn_p = kp;
                }
            }
            free(nodes);
            if (!rope_node || !kvst_node || !attn_node) {
                fprintf(stderr, "node not found: rope %p kv-store %p attention %p\n", (void *)rope_node,
                        (void *)kvst_node, (void *)attn_node);
                return 2;
            }
            CK(hipGraphInstantiate(&exec, graph, NULL, NULL, 0));
            /* The parameter arrays that hipGraphKernelNodeGetParams returns belong to the graph
             * node (which frees their elements when the graph is destroyed), so the patches
             * go into private copies of the pointer arrays, and the graph stays alive while the
             * unpatched elements are read.  (The reference writes into the node's own array
             * after destroying the graph, forward.c:1415 and :637-666.) */
            memcpy(rope_args, rope_p.kernelParams, sizeof rope_args);
            memcpy(kvst_args, kvst_p.kernelParams, sizeof kvst_args);
            memcpy(attn_args, attn_p.kernelParams, sizeof attn_args);
            rope_p.kernelParams = rope_args;
            kvst_p.kernelParams = kvst_args;
            attn_p.kernelParams = attn_args;
        }
        for (int t = 0; t < NTOK; t++) {
            const int pos = P0 + t;
            CK(hipMemcpyAsync(d_hidden, hin + (size_t)t * H, H * 4, hipMemcpyHostToDevice, cs));
            void *kdst = (char *)d_kv_k + (size_t)pos * row, *vdst = (char *)d_kv_v + (size_t)pos * row;
            if (mode == 0) {
                /* forward.c:635-666 */
                pos_buf = pos;
                rope_p.kernelParams[3] = &pos_buf;
                CK(hipGraphExecKernelNodeSetParams(exec, rope_node, &rope_p));
                kdst_buf = kdst;
                vdst_buf = vdst;
                kvst_p.kernelParams[2] = &kdst_buf;
                kvst_p.kernelParams[3] = &vdst_buf;
                CK(hipGraphExecKernelNodeSetParams(exec, kvst_node, &kvst_p));
                seqlen_buf = pos + 1;
                attn_p.kernelParams[6] = &seqlen_buf;
                CK(hipGraphExecKernelNodeSetParams(exec, attn_node, &attn_p));
                CK(hipGraphLaunch(exec, cs));
            } else {
                layer_calls(pos, kdst, vdst, pos + 1);
            }
            if (mnemo_last_error()) return 1;
            if (dump_token(f)) return 1;
        }
        if (exec) CK(hipGraphExecDestroy(exec));
        if (graph) CK(hipGraphDestroy(graph));
    }
    CK(hipMemcpy(cache, d_kv_k, ncache * 2, hipMemcpyDeviceToHost));
    fwrite(cache, 2, ncache, f);
    CK(hipMemcpy(cache, d_kv_v, ncache * 2, hipMemcpyDeviceToHost));
    fwrite(cache, 2, ncache, f);
    fclose(f);
    printf("attention graph: %d tokens patched and replayed from position %d\n", NTOK, P0);
    return 0;
}
