/*
 * mnemo_host.h -- host-side (C) composition of the kernel entry points.
 *
 * These mirror the reference's own host helpers around the kernel library so that a
 * forward pass written against MnemoCUDA's forward.c keeps its call structure:
 *   mnemo_matvec        <- matvec() type dispatcher          (forward.c:160-173)
 *   mnemo_down_type_id  <- expert down-projection type guess (forward.c:866-872)
 *   mnemo_expert_fwd    <- expert_fwd()                      (forward.c:1122-1142)
 */
#ifndef MNEMO_HOST_H
#define MNEMO_HOST_H

#include "mnemo_kernels.h"

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF type ids accepted by the dispatcher. */
#define MNEMO_TYPE_F32 0
#define MNEMO_TYPE_Q8_0 8
#define MNEMO_TYPE_Q3_K 11
#define MNEMO_TYPE_Q4_K 12
#define MNEMO_TYPE_Q5_K 13
#define MNEMO_TYPE_Q6_K 14

/* y = W x for W of GGUF type type_id (0 F32, 12 Q4_K, 14 Q6_K).  Other ids print a
 * warning and do nothing, as the reference's default branch does; Q8_0/Q3_K/Q5_K are
 * outside this library's scope and take that branch.  Returns 0 when a kernel was
 * launched, else an MNEMO_ERR_* code. */
int mnemo_matvec(const void *w, const float *x, float *y, int rows, int cols, int type_id,
                 hipStream_t stream);

/* Down-projection type of a Q4_K_M expert blob [gate][up][down]: Q6_K (14) iff the down
 * tensor is more than 1.2x the size a Q4_K [H][EFF] tensor would have, else Q4_K (12). */
int mnemo_down_type_id(size_t down_sz, int H, int EFF);

/* One routed expert on a decode token:
 *   moe_out += weight * W_down (silu(W_gate x) * (W_up x))
 * expert_data points at the blob [gate (gate_sz B)][up (up_sz B)][down]; gate and up
 * are Q4_K [EFF][H], down is down_type_id (12 or 14) [H][EFF].  gate_buf and up_buf are
 * caller-owned device scratch of EFF floats.  Two launches (gate+up dual GEMV, then the
 * SwiGLU-fused scaled-add down GEMV) instead of the reference's four or five. */
int mnemo_expert_fwd(const void *expert_data, size_t gate_sz, size_t up_sz, int H, int EFF,
                     int down_type_id, float weight, const float *x, float *gate_buf,
                     float *up_buf, float *moe_out, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* MNEMO_HOST_H */
