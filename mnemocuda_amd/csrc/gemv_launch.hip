// gemv_launch.hip -- picks the GEMV workgroup size per launch.  gemv.hip is compiled for
// 512-thread (g512) and 256-thread (g256) workgroups.  Measured on MI355X: 512 threads are
// faster whenever the waves of a launch fit on the chip at once (16 per CU) or fill it many
// times over; when they exceed one chip-full by a little (the fused Q+K+V launch: 4,608
// waves against 4,096), the last workgroups form a second, mostly idle round, and
// 4-wave workgroups shorten it (9.7 -> 8.2 us for 8192 + 2 x 512 rows at 4096 columns).
#include <climits>

#include "mnemo_internal.hpp"

namespace mnemo {
namespace g512 {
int launch_gemv_impl(GemvArgs a, hipStream_t stream);
int launch_gemv_experts_impl(GemvArgs a, hipStream_t stream);
}  // namespace g512
namespace g256 {
int launch_gemv_impl(GemvArgs a, hipStream_t stream);
}  // namespace g256

static int device_cus_launch() {
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

int launch_gemv(GemvArgs a, hipStream_t stream) {
    if (a.n_cols < 4 || a.n_cols > kMaxGemvCols) return kErrBadArg;
    const int kp = (a.n_cols + 255) & ~255;
    int lpr = 2;
    while (lpr < kp / 128 && lpr < 64) lpr <<= 1;
    long rows = 0;
    for (int i = 0; i < a.nmat; i++) rows += a.m[i].rows;
    const long waves = rows / (64 / lpr);
    const long chip = 16L * device_cus_launch();
    if (waves > chip && waves <= chip + chip / 4) return g256::launch_gemv_impl(a, stream);
    return g512::launch_gemv_impl(a, stream);
}

int launch_gemv_experts(GemvArgs a, hipStream_t stream) { return g512::launch_gemv_experts_impl(a, stream); }

}  // namespace mnemo
