// mnemo_internal.hpp -- host-side plumbing shared by the kernel files (not exported).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mnemo {

// Token rows per tile of a grouped (MoE prefill) GEMM launch, the unit of the tile list the
// routing writes (up to four 16-token MFMA columns of the grouped kernel).
constexpr int kGroupTile = 64;

// Activation rows staged for the grouped GEMM (gemm.hip, stage_f32_kernel): the Q8_1 values
// of each row as f16 integers [rows][K], the f16 ds of each 32-value sub-block [rows][K/32],
// the running-scale ratio of each sub-block [rows][K/32] and the row's last nonzero d8 [rows].
struct StagedAct {
    _Float16 *q8;
    float *rho;
    uint16_t *ds;
    float *dlast;
};

// Error codes reported through mnemo_last_error() (include/mnemo_kernels.h).
constexpr int kOk = 0;
constexpr int kErrBadArg = 1;
constexpr int kErrLaunch = 2;
constexpr int kErrUnsupportedType = 3;

constexpr int kMaxGemvCols = 16384;  // LDS image of x: 2.375 B per column
constexpr int kMaxGemvColsPad = 16384;
constexpr int kGemvMaxBlocks = 512;

enum GemvEpilogue : int { kEpiStore = 0, kEpiResidual = 1, kEpiScaledAdd = 2, kEpiScaledStore = 3, kEpiSwiGLU = 4 };

struct GemvMat {
    const void *w;     // GGUF blocks, row-major, ceil(n_cols/256) blocks per row
    float *y;          // output rows
    const float *res;  // residual (kEpiResidual)
    float scale;       // kEpiScaledAdd
    int rows;
    int type;  // 12 Q4_K | 14 Q6_K
    int mode;  // GemvEpilogue
    // pair != 0: the rows of a pass alternate between this matrix and the one mstride bytes
    // further (gate, up, gate, up, ...); lrow counts row pairs (kEpiSwiGLU)
    int pair;
    long long mstride;
    // kEpiScaledStore: the expert partials as tagged 64-bit slots {tag, fp32 bits}
    unsigned long long *part;
    unsigned int tag;
};

// Expert mode (GemvArgs::experts != 0): the matrices are chosen on the device from the
// routed expert ids.  Slot s (0 <= s < slots) uses expert idx[s]; its matrix m (0 <= m < nm)
// sits at table + idx[s] * stride + off[m].  The row space is [slot][matrix][rows].
//  nm == 2 (gate + up of every slot, one x): y[(2s + m) * rows + r]; also clears tile_cnt.
//  nm == 1 (down of every slot, x of slot s = silu(xs[2s]) * xs[2s + 1], n_cols each):
//          out += sum_s wt[s] * (W x) in slot order.  Up to 8 slots and 2048 columns: one
//          workgroup covers a row tile for all slots (gemv_down_slots_kernel); otherwise
//          partial[s * rows + r] = wt[s] * (W x) and the last workgroup to finish a row tile
//          adds the partials (tile_cnt counts the arrivals).
//  act != 0: gate row r and up row r sit side by side in one pass and the gate/up launch
//          writes y[s * rows + r] = silu(gate) * up; the down launch reads x of slot s at
//          xs[s * n_cols].
struct GemvExperts {
    const uint8_t *table;
    size_t stride;
    size_t off[2];
    const int *idx;
    const float *wt;
    const float *xs;
    float *y;
    float *out;
    // down launch with per-slot partials: the tagged partial slots [slots][rows] and the
    // 64-bit counter whose high half is this call's tag (the router's arrival counter)
    unsigned long long *part;
    const unsigned long long *gen;
    int *tile_cnt;
    int slots, nm, rows, type, n_experts;
    int act;
    int ntiles;  // nm == 2: counters to clear; nm == 1: row tiles per slot
};

struct GemvArgs {
    GemvMat m[3];
    int off[3];  // first concatenated row of each matrix (unused slots = INT32_MAX)
    int nmat;
    int total_rows;
    int n_cols;
    int xmode;  // 0: x;  1: silu(x) * x2;  2: rms_norm(x, eps) * x2
    float eps;
    const float *x;
    const float *x2;
    // expert gate/up with the RMS norm: the image of x * g (x_image.hpp layout) and 1 / rms,
    // built by the router launch before it (null: the launch builds them itself)
    const uint8_t *ximg;
    const float *xscale;
    int experts;  // 0: the static matrices m[]; 1: expert mode (ex)
    GemvExperts ex;
};

int launch_gemv(GemvArgs a, hipStream_t stream);
int launch_gemv_experts(GemvArgs a, hipStream_t stream);

// ---- attention chain (attn.hip, attn_decode.hip)
constexpr int kKvF16 = 0;
constexpr int kKvInt8 = 1;
constexpr int kHeadNorm = 1;   // RMS-normalise q and k heads with qw / kw
constexpr int kHeadRope = 2;   // rotate q and k heads
constexpr int kHeadStore = 4;  // store k and v heads at the cache row of pos

constexpr int kMaxRopeFreqs = 256;  // head_dim <= 512
struct HeadPassArgs {
    float *q, *k;          // nq / nk heads, read (and by default written back)
    const float *v;        // nv heads, only stored
    float *qo, *ko;        // outputs of the q / k heads (null: in place)
    const float *qw, *kw;  // norm weights [hd]
    int hd, nq, nk, nv;
    float eps, theta;
    int pos;               // cache row and RoPE position ...
    const int *pos_dev;    // ... or read from device memory when not null
    void *kc, *vc;         // caches [pos][nk][hd] (f16 or int8)
    float *ksc, *vsc;      // int8 scales [pos][nk]
    int kv_type;
    int flags;
    int v_layout;               // of the V cache store: 0 rows, 1 blocked (see AttnDecodeArgs)
    float freq[kMaxRopeFreqs];  // RoPE frequencies, filled by launch_head_pass
};

struct AttnArgs {
    const float *q;
    const void *kc, *vc;
    const float *ksc, *vsc;
    float *out;
    int nh, hd, nkv, gqa;
    int seq;             // sequence length = seq + (seq_dev ? *seq_dev : 0): with seq_dev the
    const int *seq_dev;  // current position in device memory and seq = 1
    float scale;
};

struct AttnDecodeArgs {
    const float *q;
    const void *kc, *vc;
    const float *ksc, *vsc;
    float *out;
    float *ws;
    size_t ws_bytes;
    int nh, hd, nkv, gqa;
    int max_ctx, max_chunks;
    int loop_split;      // decode launches: workgroups walk several chunks on long sequences (1 blocked V, 2 V rows)
    const int *pos_dev;  // sequence length = min(*pos_dev + 1, max_ctx)
    int seq_fixed;       // with pos_dev NULL: the sequence length (a host value)
    float scale;
    int v_layout;        // 0: V rows [pos][n_kv][hd]; 1: blocked [pos/64][n_kv][hd][pos%64]
    // the new token's preparation inside the launch (launch_attention_decode_prep): q is
    // raw, kn / vn are the raw K / V heads [nkv][hd] of position *pos_dev
    const float *kn, *vn;
    const float *qw, *kw;  // QK-norm weights [hd], or both NULL
    float eps;
    void *kcw, *vcw;       // the caches again, written at *pos_dev
    float *kscw, *vscw;
    float freq[64];        // RoPE frequencies of the head_dim-128 kernel
};
size_t attn_decode_workspace_bytes(int n_kv_heads, int max_ctx);
int launch_attention_decode(AttnDecodeArgs a, int kv_type, hipStream_t s);
int attn_rows_ws_init();
int attn_rows_reserve(int n);
size_t attn_rows_slot_bytes();
void *attn_rows_kernel_ptr();
void *rope_kernel_ptr();
void *f16_dual_kernel_ptr();
int launch_rope(float *q, float *k, int head_dim, int pos, float theta, int nq, int nk, hipStream_t s);
int launch_attention_rows(const float *q, const void *kc, const void *vc, const float *ksc, const float *vsc,
                          int kv_type, float *out, int nh, int hd, int nkv, int gqa, int seq, float scale,
                          hipStream_t s);
int launch_attention_decode_prep(AttnDecodeArgs a, int kv_type, float theta, hipStream_t s);

int launch_embedding(const void *table, int type, const int *tok_dev, int tok, int n_vocab, float *out, int hidden,
                     size_t row_bytes, hipStream_t s);
int launch_rms_norm(const float *in, const float *w, float *out, float *res, int n, float eps, hipStream_t s);
int launch_residual_add(const float *a, const float *b, float *out, int n, hipStream_t s);
int launch_f32_to_f16_dual(const float *a, const float *b, void *oa, void *ob, int n, hipStream_t s);
int launch_head_pass(HeadPassArgs a, hipStream_t s);
int launch_attention(AttnArgs a, int kv_type, hipStream_t s);

// Records (and prints, as the reference's KERNEL_LAUNCH_CHECK does, kernels.cu:1062-1067)
// the error of the last launch; returns a kErr code.
int check_launch(const char *what);
int set_error(int code, const char *fmt, ...);

}  // namespace mnemo
