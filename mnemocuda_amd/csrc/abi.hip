// abi.hip -- extern "C" entry points declared in include/mnemo_kernels.h.
//
// Each wrapper validates its arguments, fills a launch descriptor and returns; errors are
// printed (as the reference's KERNEL_LAUNCH_CHECK does, kernels.cu:1062-1067) and kept
// per host thread for mnemo_last_error().
#include <climits>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "mnemo_common.hpp"
#include "mnemo_internal.hpp"
#include "../../include/mnemo_kernels.h"

namespace mnemo {

static thread_local int g_err = kOk;
static thread_local char g_msg[256];

int set_error(int code, const char *fmt, ...) {
    g_err = code;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_msg, sizeof g_msg, fmt, ap);
    va_end(ap);
    fprintf(stderr, "[mnemo] %s\n", g_msg);
    return code;
}

int check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(kErrLaunch, "kernel launch error in %s: %s", what, hipGetErrorString(e));
    return kOk;
}

int launch_matvec_f32(const float *w, const float *x, float *y, int n_rows, int n_cols, hipStream_t s);
int launch_topk_softmax(const float *scores, int *idx, float *wts, int n, int k, hipStream_t s);
int launch_swiglu(const float *g, const float *u, float *out, int n, hipStream_t s);
int launch_scaled_add(float *out, const float *x, float sc, int n, hipStream_t s);
int launch_quantize_q8_1(const float *src, void *dst, int K, int N, hipStream_t s);
int launch_gemm_q8_1(int type, const void *w, const void *act, float *out, int M, int K, int N, hipStream_t s);
size_t moe_prefill_workspace_bytes(int T, int hidden, int eff, int E, int k);
int launch_sample_token(const float *logits, int V, float temperature, float top_p, unsigned long long seed,
                        int *out, hipStream_t stream);
int launch_sample_token_ws(const float *logits, int V, float temperature, float top_p, unsigned long long seed,
                           void *ws, size_t ws_bytes, int *out, hipStream_t stream);
size_t sample_workspace_bytes();
size_t moe_decode_workspace_bytes(int hidden, int eff, int E, int k);
int moe_decode_scratch_init();
int launch_moe_decode_noalloc(const float *router_w, const void *experts, size_t expert_stride, size_t gate_off,
                              size_t up_off, size_t down_off, int down_type, const float *x, const float *norm_w,
                              float eps, int hidden, int eff, int E, int k, float *out, int *idx_out, float *w_out,
                              hipStream_t s);
int launch_moe_decode(const float *router_w, const void *experts, size_t expert_stride, size_t gate_off,
                      size_t up_off, size_t down_off, int down_type, const float *x, const float *norm_w, float eps,
                      int hidden, int eff, int E, int k, void *ws, size_t ws_bytes, float *out, int *idx_out,
                      float *w_out, hipStream_t s);
int launch_moe_prefill(const void *experts, size_t expert_stride, size_t gate_off, size_t up_off, size_t down_off,
                       int down_type, const float *x, const int *topk_idx, const float *topk_w, int T, int hidden,
                       int eff, int E, int k, void *ws, size_t ws_bytes, float *out, hipStream_t s);

static bool type_ok(int t) { return t == kTypeQ4K || t == kTypeQ6K; }

// Builds a GEMV launch over up to three matrices sharing x (all with n_cols columns).
struct GemvBuilder {
    GemvArgs a;
    GemvBuilder(const float *x, int n_cols) {
        memset(&a, 0, sizeof a);
        a.x = x;
        a.n_cols = n_cols;
        a.off[0] = 0;
        a.off[1] = a.off[2] = INT_MAX;
    }
    void add(const void *w, int type, float *y, int rows, int mode, const float *res = nullptr,
             float scale = 0.0f) {
        GemvMat &m = a.m[a.nmat];
        m.w = w; m.type = type; m.y = y; m.rows = rows; m.mode = mode; m.res = res; m.scale = scale;
        a.off[a.nmat] = a.total_rows;
        a.total_rows += rows;
        a.nmat++;
    }
    int run(const char *what, hipStream_t s) {
        if (!a.x || a.n_cols < 4 || a.n_cols > kMaxGemvCols)
            return set_error(kErrBadArg, "%s: need x != NULL and 4 <= n_cols <= %d", what, kMaxGemvCols);
        for (int i = 0; i < a.nmat; i++) {
            const GemvMat &m = a.m[i];
            if (!m.w || !m.y || m.rows <= 0 || (m.mode == kEpiResidual && !m.res))
                return set_error(kErrBadArg, "%s: bad pointer or row count for matrix %d", what, i);
            if (!type_ok(m.type)) return set_error(kErrUnsupportedType, "%s: unsupported GGUF type %d", what, m.type);
        }
        for (int i = a.nmat; i < 3; i++) a.off[i] = INT_MAX;
        return launch_gemv(a, s);
    }
};

}  // namespace mnemo

using namespace mnemo;

extern "C" {

int mnemo_last_error(void) {
    int e = g_err;
    g_err = kOk;
    return e;
}
const char *mnemo_last_error_string(void) { return g_msg; }
const char *mnemo_version(void) { return "mnemo-mi355x 0.1 gfx950"; }

int mnemo_record_error(int code, const char *msg) { return set_error(code, "%s", msg ? msg : "error"); }

void cuda_kernels_init(void) {
    int dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) {
        set_error(kErrLaunch, "cuda_kernels_init: no HIP device");
        return;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        set_error(kErrLaunch, "cuda_kernels_init: built for gfx950, device is %s", prop.gcnArchName);
        return;
    }
    moe_decode_scratch_init();  // this device's copy of the no-allocation decode scratch
    attn_rows_ws_init();        // partials of the split-chunk path of cuda_attention_*
}

void cuda_matvec_q4k(const void *w, const float *x, float *y, int n_rows, int n_cols, hipStream_t s) {
    GemvBuilder b(x, n_cols);
    b.add(w, kTypeQ4K, y, n_rows, kEpiStore);
    b.run("cuda_matvec_q4k", s);
}

void cuda_matvec_q4k_add(const void *w, const float *x, const float *res, float *y, int n_rows, int n_cols,
                         hipStream_t s) {
    GemvBuilder b(x, n_cols);
    b.add(w, kTypeQ4K, y, n_rows, kEpiResidual, res);
    b.run("cuda_matvec_q4k_add", s);
}

void cuda_matvec_q4k_qkv(const void *wq, const void *wk, const void *wv, const float *x, float *oq, float *ok,
                         float *ov, int q_rows, int kv_rows, int n_cols, hipStream_t s) {
    GemvBuilder b(x, n_cols);
    b.add(wq, kTypeQ4K, oq, q_rows, kEpiStore);
    b.add(wk, kTypeQ4K, ok, kv_rows, kEpiStore);
    b.add(wv, kTypeQ4K, ov, kv_rows, kEpiStore);
    b.run("cuda_matvec_q4k_qkv", s);
}

void cuda_matvec_q4k_dual(const void *wa, const void *wb, const float *x, float *ya, float *yb, int n_rows,
                          int n_cols, hipStream_t s) {
    GemvBuilder b(x, n_cols);
    b.add(wa, kTypeQ4K, ya, n_rows, kEpiStore);
    b.add(wb, kTypeQ4K, yb, n_rows, kEpiStore);
    b.run("cuda_matvec_q4k_dual", s);
}

void cuda_matvec_q4k_scaled_add(const void *w, const float *x, float *y, int n_rows, int n_cols, float scale,
                                hipStream_t s) {
    GemvBuilder b(x, n_cols);
    b.add(w, kTypeQ4K, y, n_rows, kEpiScaledAdd, nullptr, scale);
    b.run("cuda_matvec_q4k_scaled_add", s);
}

void cuda_matvec_q6k(const void *w, const float *x, float *y, int n_rows, int n_cols, hipStream_t s) {
    GemvBuilder b(x, n_cols);
    b.add(w, kTypeQ6K, y, n_rows, kEpiStore);
    b.run("cuda_matvec_q6k", s);
}

void mnemo_matvec_q6k_scaled_add(const void *w, const float *x, float *y, int n_rows, int n_cols, float scale,
                                 hipStream_t s) {
    GemvBuilder b(x, n_cols);
    b.add(w, kTypeQ6K, y, n_rows, kEpiScaledAdd, nullptr, scale);
    b.run("mnemo_matvec_q6k_scaled_add", s);
}

void mnemo_matvec_dual(const void *wa, int ta, const void *wb, int tb, const float *x, float *ya, float *yb,
                       int n_rows, int n_cols, hipStream_t s) {
    GemvBuilder b(x, n_cols);
    b.add(wa, ta, ya, n_rows, kEpiStore);
    b.add(wb, tb, yb, n_rows, kEpiStore);
    b.run("mnemo_matvec_dual", s);
}

void mnemo_matvec_qkv(const void *wq, int tq, const void *wk, int tk, const void *wv, int tv, const float *x,
                      float *oq, float *ok, float *ov, int q_rows, int kv_rows, int n_cols, hipStream_t s) {
    GemvBuilder b(x, n_cols);
    b.add(wq, tq, oq, q_rows, kEpiStore);
    b.add(wk, tk, ok, kv_rows, kEpiStore);
    b.add(wv, tv, ov, kv_rows, kEpiStore);
    b.run("mnemo_matvec_qkv", s);
}

void mnemo_matvec_qkv_rmsnorm(const void *wq, int tq, const void *wk, int tk, const void *wv, int tv,
                              const float *x, const float *norm_w, float eps, float *oq, float *ok, float *ov,
                              int q_rows, int kv_rows, int n_cols, hipStream_t s) {
    if (!norm_w) {
        set_error(kErrBadArg, "mnemo_matvec_qkv_rmsnorm: norm_w == NULL");
        return;
    }
    GemvBuilder b(x, n_cols);
    b.a.x2 = norm_w;
    b.a.xmode = 2;
    b.a.eps = eps;
    b.add(wq, tq, oq, q_rows, kEpiStore);
    b.add(wk, tk, ok, kv_rows, kEpiStore);
    b.add(wv, tv, ov, kv_rows, kEpiStore);
    b.run("mnemo_matvec_qkv_rmsnorm", s);
}

void mnemo_matvec_swiglu_scaled_add(const void *w, int type, const float *gate, const float *up, float *y,
                                    int n_rows, int n_cols, float scale, hipStream_t s) {
    GemvBuilder b(gate, n_cols);
    b.a.x2 = up;
    b.a.xmode = 1;
    if (!up) {
        set_error(kErrBadArg, "mnemo_matvec_swiglu_scaled_add: up == NULL");
        return;
    }
    b.add(w, type, y, n_rows, kEpiScaledAdd, nullptr, scale);
    b.run("mnemo_matvec_swiglu_scaled_add", s);
}

void cuda_matvec_f32(const float *w, const float *x, float *y, int n_rows, int n_cols, hipStream_t s) {
    launch_matvec_f32(w, x, y, n_rows, n_cols, s);
}

void cuda_topk_softmax(const float *scores, int *idx, float *wts, int n_experts, int k, hipStream_t s) {
    launch_topk_softmax(scores, idx, wts, n_experts, k, s);
}

void cuda_swiglu(const float *g, const float *u, float *out, int n, hipStream_t s) { launch_swiglu(g, u, out, n, s); }

void cuda_scaled_add(float *out, const float *x, float scale, int n, hipStream_t s) {
    launch_scaled_add(out, x, scale, n, s);
}

void cuda_quantize_mmq_q8_1(const float *src, void *dst, int K, int N, hipStream_t s) {
    launch_quantize_q8_1(src, dst, K, N, s);
}

void cuda_gemm_q4k(const void *w, const void *act, float *out, int M, int K, int N, hipStream_t s) {
    launch_gemm_q8_1(kTypeQ4K, w, act, out, M, K, N, s);
}

void mnemo_gemm_q6k(const void *w, const void *act, float *out, int M, int K, int N, hipStream_t s) {
    launch_gemm_q8_1(kTypeQ6K, w, act, out, M, K, N, s);
}

void cuda_sample_token(const float *logits, int vocab_size, float temperature, float top_p,
                       unsigned long long rng_state, int *d_result, hipStream_t s) {
    launch_sample_token(logits, vocab_size, temperature, top_p, rng_state, d_result, s);
}

size_t mnemo_sample_workspace_bytes(void) { return sample_workspace_bytes(); }

int mnemo_sample_token_ws(const float *logits, int vocab_size, float temperature, float top_p,
                          unsigned long long rng_state, void *workspace, size_t workspace_bytes, int *d_result,
                          hipStream_t s) {
    return launch_sample_token_ws(logits, vocab_size, temperature, top_p, rng_state, workspace, workspace_bytes,
                                  d_result, s);
}

// ---------------------------------------------------------------- attention chain
void cuda_rms_norm(const float *input, const float *weight, float *output, int n, float eps, hipStream_t s) {
    launch_rms_norm(input, weight, output, nullptr, n, eps, s);
}

void cuda_rms_norm_residual(const float *input, const float *weight, float *normed_output, float *residual_output,
                            int n, float eps, hipStream_t s) {
    if (!residual_output) {
        set_error(kErrBadArg, "rms_norm_residual: residual_output is NULL");
        return;
    }
    launch_rms_norm(input, weight, normed_output, residual_output, n, eps, s);
}

void cuda_rms_norm_batched(const float *input, const float *weight, float *output, int head_dim, int n_heads,
                           float eps, hipStream_t s) {
    HeadPassArgs a = {};
    a.q = (float *)input;
    a.qo = output;
    a.qw = weight;
    a.hd = head_dim;
    a.nq = n_heads;
    a.eps = eps;
    a.flags = kHeadNorm;
    if (!weight || !output) {
        set_error(kErrBadArg, "rms_norm_batched: NULL weight or output");
        return;
    }
    launch_head_pass(a, s);
}

void cuda_rms_norm_qk(float *q, float *k, const float *q_weight, const float *k_weight, int head_dim, int n_q,
                      int n_k, float eps, hipStream_t s) {
    HeadPassArgs a = {};
    a.q = q;
    a.k = k;
    a.qw = q_weight;
    a.kw = k_weight;
    a.hd = head_dim;
    a.nq = n_q;
    a.nk = n_k;
    a.eps = eps;
    a.flags = kHeadNorm;
    if (!q_weight || !k_weight) {
        set_error(kErrBadArg, "rms_norm_qk: NULL weights");
        return;
    }
    launch_head_pass(a, s);
}

void cuda_residual_add(const float *a, const float *b, float *out, int n, hipStream_t s) {
    launch_residual_add(a, b, out, n, s);
}

void cuda_rope(float *q, float *k, int head_dim, int pos, float theta, int n_heads_q, int n_heads_k, hipStream_t s) {
    launch_rope(q, k, head_dim, pos, theta, n_heads_q, n_heads_k, s);
}

// The kernels whose graph nodes the reference engine finds by function pointer and patches
// before every replay (kernels.cu:2243-2245; forward.c:1291-1297, 1395-1412, 633-668):
// parameter 3 of the RoPE node (pos), 2 and 3 of the f16 KV store (destinations), 6 of the
// attention node (seq_len).  Each is the kernel its entry point launches, with those parameters
// at those positions.
void *cuda_get_rope_kernel_ptr(void) { return rope_kernel_ptr(); }
void *cuda_get_f16dual_kernel_ptr(void) { return f16_dual_kernel_ptr(); }
void *cuda_get_attn_f16kv_kernel_ptr(void) { return attn_rows_kernel_ptr(); }

int mnemo_attention_reserve(int n_slots) {
    if (n_slots < 0) return set_error(kErrBadArg, "attention_reserve: n_slots < 0");
    const int rc = attn_rows_reserve(n_slots);
    if (rc != kOk) return set_error(rc, "attention_reserve: could not hold %d free slots", n_slots);
    return kOk;
}

size_t mnemo_attention_slot_bytes(void) { return attn_rows_slot_bytes(); }

void cuda_f32_to_f16_dual(const float *a, const float *b, void *oa, void *ob, int n, hipStream_t s) {
    launch_f32_to_f16_dual(a, b, oa, ob, n, s);
}

void cuda_f32_to_int8_kv_dual(const float *k, const float *v, void *out_k, void *out_v, float *k_scales,
                              float *v_scales, int head_dim, int n_kv_heads, hipStream_t s) {
    // the reference passes the cache rows and scale slots of the current position
    HeadPassArgs a = {};
    a.k = (float *)k;  // read only: a store-only pass writes nothing back
    a.v = v;
    a.hd = head_dim;
    a.nk = n_kv_heads;
    a.nv = n_kv_heads;
    a.kc = out_k;
    a.vc = out_v;
    a.ksc = k_scales;
    a.vsc = v_scales;
    a.kv_type = kKvInt8;
    a.flags = kHeadStore;
    launch_head_pass(a, s);
}

void cuda_attention_f16kv(const void *q, const void *kv_k, const void *kv_v, float *out, int n_heads_q, int head_dim,
                          int n_kv_heads, int seq_len, int gqa_ratio, float scale, hipStream_t s) {
    if (launch_attention_rows((const float *)q, kv_k, kv_v, nullptr, nullptr, kKvF16, out, n_heads_q, head_dim,
                              n_kv_heads, gqa_ratio, seq_len, scale, s) != kErrBadArg)
        return;
    AttnArgs a = {};
    a.q = (const float *)q;
    a.kc = kv_k;
    a.vc = kv_v;
    a.out = out;
    a.nh = n_heads_q;
    a.hd = head_dim;
    a.nkv = n_kv_heads;
    a.gqa = gqa_ratio;
    a.seq = seq_len;
    a.scale = scale;
    launch_attention(a, kKvF16, s);
}

void cuda_attention_int8kv(const float *q, const void *kv_k, const void *kv_v, const float *k_scales,
                           const float *v_scales, float *out, int n_heads_q, int head_dim, int n_kv_heads,
                           int seq_len, int gqa_ratio, float scale, hipStream_t s) {
    if (k_scales && v_scales &&
        launch_attention_rows(q, kv_k, kv_v, k_scales, v_scales, kKvInt8, out, n_heads_q, head_dim, n_kv_heads,
                              gqa_ratio, seq_len, scale, s) != kErrBadArg)
        return;
    AttnArgs a = {};
    a.q = q;
    a.kc = kv_k;
    a.vc = kv_v;
    a.ksc = k_scales;
    a.vsc = v_scales;
    a.out = out;
    a.nh = n_heads_q;
    a.hd = head_dim;
    a.nkv = n_kv_heads;
    a.gqa = gqa_ratio;
    a.seq = seq_len;
    a.scale = scale;
    launch_attention(a, kKvInt8, s);
}

int mnemo_attn_prep(float *q, float *k, const float *v, const float *q_norm_w, const float *k_norm_w, int head_dim,
                    int n_heads, int n_kv_heads, float eps, float theta, const int *pos_dev, void *k_cache,
                    void *v_cache, float *k_scales, float *v_scales, int kv_type, int v_layout, hipStream_t s) {
    if (!pos_dev) return set_error(kErrBadArg, "attn_prep: pos_dev is NULL");
    if (v_layout != 0 && v_layout != 1) return set_error(kErrBadArg, "attn_prep: v_layout %d", v_layout);
    if (kv_type != kKvF16 && kv_type != kKvInt8) return set_error(kErrBadArg, "attn_prep: kv_type %d", kv_type);
    if ((q_norm_w == nullptr) != (k_norm_w == nullptr))
        return set_error(kErrBadArg, "attn_prep: give both QK-norm weights or neither");
    HeadPassArgs a = {};
    a.q = q;
    a.k = k;
    a.v = v;
    a.qw = q_norm_w;
    a.kw = k_norm_w;
    a.hd = head_dim;
    a.nq = n_heads;
    a.nk = n_kv_heads;
    a.nv = n_kv_heads;
    a.eps = eps;
    a.theta = theta;
    a.pos_dev = pos_dev;
    a.kc = k_cache;
    a.vc = v_cache;
    a.ksc = k_scales;
    a.vsc = v_scales;
    a.kv_type = kv_type;
    a.v_layout = v_layout;
    a.flags = (q_norm_w ? kHeadNorm : 0) | kHeadRope | kHeadStore;
    return launch_head_pass(a, s);
}

int mnemo_attention(const float *q, const void *k_cache, const void *v_cache, const float *k_scales,
                    const float *v_scales, int kv_type, float *out, int n_heads, int head_dim, int n_kv_heads,
                    const int *pos_dev, float scale, hipStream_t s) {
    if (!pos_dev) return set_error(kErrBadArg, "attention: pos_dev is NULL");
    if (kv_type != kKvF16 && kv_type != kKvInt8) return set_error(kErrBadArg, "attention: kv_type %d", kv_type);
    if (n_kv_heads <= 0 || n_heads % n_kv_heads) return set_error(kErrBadArg, "attention: n_heads %% n_kv_heads");
    AttnArgs a = {};
    a.q = q;
    a.kc = k_cache;
    a.vc = v_cache;
    a.ksc = k_scales;
    a.vsc = v_scales;
    a.out = out;
    a.nh = n_heads;
    a.hd = head_dim;
    a.nkv = n_kv_heads;
    a.gqa = n_heads / n_kv_heads;
    a.seq = 1;
    a.seq_dev = pos_dev;
    a.scale = scale;
    return launch_attention(a, kv_type, s);
}

size_t mnemo_attention_decode_workspace_bytes(int n_kv_heads, int max_ctx) {
    return n_kv_heads > 0 && max_ctx > 0 ? attn_decode_workspace_bytes(n_kv_heads, max_ctx) : 0;
}

size_t mnemo_v_cache_bytes(int n_kv_heads, int head_dim, int max_ctx, int kv_type, int v_layout) {
    if (n_kv_heads <= 0 || head_dim <= 0 || max_ctx <= 0) return 0;
    const size_t rows = v_layout == 1 ? ((size_t)max_ctx + 63) / 64 * 64 : (size_t)max_ctx;
    return rows * n_kv_heads * head_dim * (kv_type == kKvInt8 ? 1 : 2);
}

int mnemo_attention_decode(const float *q, const void *k_cache, const void *v_cache, const float *k_scales,
                           const float *v_scales, int kv_type, int v_layout, float *out, int n_heads, int head_dim,
                           int n_kv_heads, int max_ctx, const int *pos_dev, float scale, void *workspace,
                           size_t workspace_bytes, hipStream_t s) {
    if (kv_type != kKvF16 && kv_type != kKvInt8) return set_error(kErrBadArg, "attention_decode: kv_type %d", kv_type);
    if (n_kv_heads <= 0 || n_heads % n_kv_heads) return set_error(kErrBadArg, "attention_decode: n_heads %% n_kv_heads");
    if ((uintptr_t)workspace % 16) return set_error(kErrBadArg, "attention_decode: workspace not 16-byte aligned");
    AttnDecodeArgs a = {};
    a.q = q;
    a.kc = k_cache;
    a.vc = v_cache;
    a.ksc = k_scales;
    a.vsc = v_scales;
    a.out = out;
    a.ws = (float *)workspace;
    a.ws_bytes = workspace_bytes;
    a.nh = n_heads;
    a.hd = head_dim;
    a.nkv = n_kv_heads;
    a.gqa = n_heads / n_kv_heads;
    a.max_ctx = max_ctx;
    a.pos_dev = pos_dev;
    a.scale = scale;
    a.v_layout = v_layout;
    return launch_attention_decode(a, kv_type, s);
}

int mnemo_attention_decode_prep(const float *q, const float *k, const float *v, const float *q_norm_w,
                                const float *k_norm_w, float eps, float theta, void *k_cache, void *v_cache,
                                float *k_scales, float *v_scales, int kv_type, int v_layout, float *out, int n_heads,
                                int head_dim, int n_kv_heads, int max_ctx, const int *pos_dev, float scale,
                                void *workspace, size_t workspace_bytes, hipStream_t s) {
    if (n_kv_heads <= 0 || n_heads % n_kv_heads)
        return set_error(kErrBadArg, "attention_decode_prep: n_heads %% n_kv_heads");
    if ((uintptr_t)workspace % 16) return set_error(kErrBadArg, "attention_decode_prep: workspace not 16-byte aligned");
    AttnDecodeArgs a = {};
    a.q = q;
    a.kc = k_cache;
    a.vc = v_cache;
    a.ksc = k_scales;
    a.vsc = v_scales;
    a.out = out;
    a.ws = (float *)workspace;
    a.ws_bytes = workspace_bytes;
    a.nh = n_heads;
    a.hd = head_dim;
    a.nkv = n_kv_heads;
    a.gqa = n_heads / n_kv_heads;
    a.max_ctx = max_ctx;
    a.pos_dev = pos_dev;
    a.scale = scale;
    a.v_layout = v_layout;
    a.kn = k;
    a.vn = v;
    a.qw = q_norm_w;
    a.kw = k_norm_w;
    a.eps = eps;
    a.kcw = k_cache;
    a.vcw = v_cache;
    a.kscw = k_scales;
    a.vscw = v_scales;
    return launch_attention_decode_prep(a, kv_type, theta, s);
}

// ---------------------------------------------------------------- embedding
void cuda_embedding_lookup_q4k(const void *embd_table, float *output, int token_id, int hidden_size, int row_bytes,
                               hipStream_t s) {
    // the reference passes no vocabulary size; its row bound is the caller's
    if (row_bytes <= 0 || (size_t)row_bytes < (size_t)((hidden_size + 255) / 256) * kQ4KBytes) {
        set_error(kErrBadArg, "embedding_lookup_q4k: row_bytes %d too small for %d values", row_bytes, hidden_size);
        return;
    }
    launch_embedding(embd_table, kTypeQ4K, nullptr, token_id, INT_MAX, output, hidden_size, (size_t)row_bytes, s);
}

int mnemo_embedding_lookup(const void *table, int type_id, const int *token_dev, int n_vocab, float *output,
                           int hidden_size, hipStream_t s) {
    size_t rb = 0;
    if (type_id == kTypeF32) rb = (size_t)hidden_size * 4;
    else if (type_id == kTypeQ4K) rb = (size_t)((hidden_size + 255) / 256) * kQ4KBytes;
    else if (type_id == kTypeQ6K) rb = (size_t)((hidden_size + 255) / 256) * kQ6KBytes;
    if (!token_dev) return set_error(kErrBadArg, "embedding_lookup: token_dev is NULL");
    return launch_embedding(table, type_id, token_dev, 0, n_vocab, output, hidden_size, rb, s);
}

size_t mnemo_moe_prefill_workspace_bytes(int n_tokens, int hidden, int eff, int n_experts, int k) {
    return moe_prefill_workspace_bytes(n_tokens, hidden, eff, n_experts, k);
}

int mnemo_moe_prefill(const void *experts, size_t expert_stride, size_t gate_off, size_t up_off, size_t down_off,
                      int down_type, const float *x, const int *topk_idx, const float *topk_w, int n_tokens,
                      int hidden, int eff, int n_experts, int k, void *workspace, size_t workspace_bytes, float *out,
                      hipStream_t s) {
    return launch_moe_prefill(experts, expert_stride, gate_off, up_off, down_off, down_type, x, topk_idx, topk_w,
                              n_tokens, hidden, eff, n_experts, k, workspace, workspace_bytes, out, s);
}

size_t mnemo_moe_decode_workspace_bytes(int hidden, int eff, int n_experts, int k) {
    return moe_decode_workspace_bytes(hidden, eff, n_experts, k);
}

int mnemo_moe_decode(const float *router_w, const void *experts, size_t expert_stride, size_t gate_off,
                     size_t up_off, size_t down_off, int down_type, const float *x, int hidden, int eff,
                     int n_experts, int k, void *workspace, size_t workspace_bytes, float *out, int *topk_idx,
                     float *topk_w, hipStream_t s) {
    return launch_moe_decode(router_w, experts, expert_stride, gate_off, up_off, down_off, down_type, x, nullptr, 0.0f,
                             hidden, eff, n_experts, k, workspace, workspace_bytes, out, topk_idx, topk_w, s);
}

int mnemo_moe_decode_rmsnorm(const float *router_w, const void *experts, size_t expert_stride, size_t gate_off,
                             size_t up_off, size_t down_off, int down_type, const float *x, const float *norm_w,
                             float eps, int hidden, int eff, int n_experts, int k, void *workspace,
                             size_t workspace_bytes, float *out, int *topk_idx, float *topk_w, hipStream_t s) {
    if (!norm_w) return set_error(kErrBadArg, "moe_decode_rmsnorm: norm_w is NULL");
    return launch_moe_decode(router_w, experts, expert_stride, gate_off, up_off, down_off, down_type, x, norm_w, eps,
                             hidden, eff, n_experts, k, workspace, workspace_bytes, out, topk_idx, topk_w, s);
}

int mnemo_moe_decode_rmsnorm_noalloc(const float *router_w, const void *experts, size_t expert_stride,
                                     size_t gate_off, size_t up_off, size_t down_off, int down_type, const float *x,
                                     const float *norm_w, float eps, int hidden, int eff, int n_experts, int k,
                                     float *out, int *topk_idx, float *topk_w, hipStream_t s) {
    if (!norm_w) return set_error(kErrBadArg, "moe_decode_rmsnorm_noalloc: norm_w is NULL");
    return launch_moe_decode_noalloc(router_w, experts, expert_stride, gate_off, up_off, down_off, down_type, x,
                                     norm_w, eps, hidden, eff, n_experts, k, out, topk_idx, topk_w, s);
}

}  // extern "C"
