/*
 * mnemo_host.c -- C host composition of the kernel ABI (see include/mnemo_host.h).
 * Compiled with the host C compiler; calls only the extern "C" entry points.
 */
#include "../../../include/mnemo_host.h"

#include <stdio.h>

int mnemo_matvec(const void *w, const float *x, float *y, int rows, int cols, int type_id,
                 hipStream_t stream) {
    switch (type_id) {
    case MNEMO_TYPE_F32: cuda_matvec_f32((const float *)w, x, y, rows, cols, stream); break;
    case MNEMO_TYPE_Q4_K: cuda_matvec_q4k(w, x, y, rows, cols, stream); break;
    case MNEMO_TYPE_Q6_K: cuda_matvec_q6k(w, x, y, rows, cols, stream); break;
    default:
        fprintf(stderr, "[mnemo] WARN unsupported type_id %d for matvec\n", type_id);
        return MNEMO_ERR_UNSUPPORTED_TYPE;
    }
    return mnemo_last_error();
}

int mnemo_down_type_id(size_t down_sz, int H, int EFF) {
    /* forward.c:871-872: expected Q4_K bytes = ceil(H*EFF/256) * 144 */
    size_t expected_q4k = (size_t)(((long long)H * EFF + 255) / 256) * 144;
    return ((double)down_sz > (double)expected_q4k * 1.2) ? MNEMO_TYPE_Q6_K : MNEMO_TYPE_Q4_K;
}

int mnemo_expert_fwd(const void *expert_data, size_t gate_sz, size_t up_sz, int H, int EFF,
                     int down_type_id, float weight, const float *x, float *gate_buf,
                     float *up_buf, float *moe_out, hipStream_t stream) {
    const char *base = (const char *)expert_data;
    if (!expert_data || !x || !gate_buf || !up_buf || !moe_out) return MNEMO_ERR_BAD_ARG;
    if (down_type_id != MNEMO_TYPE_Q4_K && down_type_id != MNEMO_TYPE_Q6_K) {
        fprintf(stderr, "[mnemo] WARN unsupported down type_id %d\n", down_type_id);
        return MNEMO_ERR_UNSUPPORTED_TYPE;
    }
    cuda_matvec_q4k_dual(base, base + gate_sz, x, gate_buf, up_buf, EFF, H, stream);
    int e = mnemo_last_error();
    if (e) return e;
    mnemo_matvec_swiglu_scaled_add(base + gate_sz + up_sz, down_type_id, gate_buf, up_buf, moe_out,
                                   H, EFF, weight, stream);
    return mnemo_last_error();
}
