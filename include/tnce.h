/* tnce.h -- C ABI of the fused linear + cross-entropy epilogues in libtnpa.so (MI355X, gfx950).
 *
 * The reference computes sum_i CE(x_i W^T, t_i) chunk by chunk so that only one chunk of logits exists at a time,
 * recomputing each chunk's logits in the backward (ref: tnlm/kernels/fused_ce.py:18-60). Per chunk it runs a matmul
 * and then a chain of elementwise and reduction ops over the (rows x V) logits: upcast, logsumexp, target gather, the
 * masked sum (forward); exp(logit - lse), the one-hot subtraction, the scale by valid * g and the downcast
 * (backward). The matmuls stay plain library GEMMs (hipBLASLt through torch); these entry points replace each op
 * chain by one pass over the chunk's logits in HBM, written for 64-wide wavefronts with 16-byte loads.
 *
 * Logits: n rows of V contiguous values with row stride ld elements, in dtype (the matmul's output type, so their
 * rounding is the reference's). Accumulation type acc = float for TNCE_BF16 / TNCE_F16 / TNCE_F32, double for
 * TNCE_F64 (the reference's torch.promote_types(cdtype, float32)). targets: n int64 class ids, ignore_index (-100)
 * marks rows without a target; other ids outside [0, V) give a NaN loss term (the reference raises instead).
 * Work is enqueued on the caller's stream; the library allocates nothing. Return 0 or a tnpa_status code with
 * tnpa_last_error() set (include/tnpa.h).
 */
#ifndef TNCE_H
#define TNCE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum { TNCE_BF16 = 0, TNCE_F32 = 1, TNCE_F16 = 2, TNCE_F64 = 3 } tnce_dtype;

/* Forward of one chunk: lse[i] = log sum_j exp(logits[i, j]) (acc type) for each of the n rows, and
 * *total += sum_i [targets[i] != ignore_index] (lse[i] - logits[i, targets[i]]) in acc type, the sum taken in a fixed
 * order (deterministic). row_loss is n acc-type values of caller scratch. Replaces the chunk body of
 * ref: tnlm/kernels/fused_ce.py:29-33 (logsumexp, gather and masked sum of one chunk). */
int tnce_forward_chunk(const void* logits, int32_t dtype, int64_t n, int64_t V, int64_t ld, const int64_t* targets,
                       int64_t ignore_index, void* lse, void* row_loss, void* total, void* stream);

/* Backward of one chunk, in place: logits[i, j] <- ((exp(logits[i, j] - lse[i]) - [j == targets[i]]) * valid_i * g)
 * rounded to dtype, with valid_i = targets[i] != ignore_index and g the upstream gradient (one acc-type value in
 * device memory). The result is the chunk's dL/dlogits for the dX and dW matmuls. Replaces
 * ref: tnlm/kernels/fused_ce.py:45-48. */
int tnce_backward_chunk(void* logits, int32_t dtype, int64_t n, int64_t V, int64_t ld, const int64_t* targets,
                        int64_t ignore_index, const void* lse, const void* g, void* stream);

/* dW accumulation of one chunk: acc[i] += (acc type) part[i] for n elements, part in dtype (the chunk's dW matmul
 * output, rounded as the reference's matmul output is), acc in the accumulation type; one pass instead of an
 * upcast copy and an add. Both pointers 16-byte aligned. Replaces ref: tnlm/kernels/fused_ce.py:50
 * (dw += (p.T @ x).to(acc)). */
int tnce_accumulate(void* acc, const void* part, int32_t dtype, int64_t n, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TNCE_H */
