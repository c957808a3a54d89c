// gemv_launch.hip -- picks the GEMV kernel and workgroup size per launch.  gemv.hip is compiled for
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
int launch_gemv_split_impl(GemvArgs a, hipStream_t stream);
int launch_gemv_q6stage_impl(GemvArgs a, hipStream_t stream);
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
    // The split-columns kernel (8 rows x 1024 columns per wave, an x image per wave of its own
    // columns) where the whole-row kernel leaves the chip short of work or a partial second
    // round.  Measured on MI355X, 94 layers of distinct weights: fused Q 8192 + K 512 + V 512
    // at 4096 columns 7.30 against 7.6-7.9 us (8.32 against 8.4-8.5 with the RMS norm); K + V
    // 512 + 512 3.77 against 5.02; 1536 rows 3.51 against 3.83; but 4096 or 8192 rows alone
    // 4.84 / 6.49 against 4.60 / 6.04, and O 4096 x 8192 6.61 against 6.25, stay whole-row.
    if (waves <= chip / 4 || (waves > chip && waves <= chip + chip / 4)) {
        const int rc = g512::launch_gemv_split_impl(a, stream);
        if (rc != kErrBadArg) return rc;
    }
    // Q6_K rows of 4096 values over several rounds of the chip (the lm_head): the staged
    // kernel's aligned lane-contiguous loads read the 2-byte-aligned blocks faster (151,936
    // rows: 97.5 against 106.8 us)
    if (waves > 2 * chip) {
        const int rc = g512::launch_gemv_q6stage_impl(a, stream);
        if (rc != kErrBadArg) return rc;
    }
    if (waves > chip && waves <= chip + chip / 4) return g256::launch_gemv_impl(a, stream);
    return g512::launch_gemv_impl(a, stream);
}

int launch_gemv_experts(GemvArgs a, hipStream_t stream) { return g512::launch_gemv_experts_impl(a, stream); }

}  // namespace mnemo
