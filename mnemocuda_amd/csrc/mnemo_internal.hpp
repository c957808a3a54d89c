// mnemo_internal.hpp -- host-side plumbing shared by the kernel files (not exported).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mnemo {

// Error codes reported through mnemo_last_error() (include/mnemo_kernels.h).
constexpr int kOk = 0;
constexpr int kErrBadArg = 1;
constexpr int kErrLaunch = 2;
constexpr int kErrUnsupportedType = 3;

constexpr int kMaxGemvCols = 16384;  // LDS image of x: 2.375 B per column
constexpr int kMaxGemvColsPad = 16384;
constexpr int kGemvMaxBlocks = 512;

enum GemvEpilogue : int { kEpiStore = 0, kEpiResidual = 1, kEpiScaledAdd = 2 };

struct GemvMat {
    const void *w;     // GGUF blocks, row-major, ceil(n_cols/256) blocks per row
    float *y;          // output rows
    const float *res;  // residual (kEpiResidual)
    float scale;       // kEpiScaledAdd
    int rows;
    int type;  // 12 Q4_K | 14 Q6_K
    int mode;  // GemvEpilogue
};

struct GemvArgs {
    GemvMat m[3];
    int off[3];  // first concatenated row of each matrix (unused slots = INT32_MAX)
    int nmat;
    int total_rows;
    int n_cols;
    int xmode;  // 0: x;  1: silu(x) * x2
    const float *x;
    const float *x2;
};

int launch_gemv(GemvArgs a, hipStream_t stream);

// Records (and prints, as the reference's KERNEL_LAUNCH_CHECK does, kernels.cu:1062-1067)
// the error of the last launch; returns a kErr code.
int check_launch(const char *what);
int set_error(int code, const char *fmt, ...);

}  // namespace mnemo
