/* tnpa.h -- C ABI of the MI355X (gfx950) causal polynomial attention library (libtnpa.so).
 *
 * The library replaces the Triton host orchestration and kernels of the reference operator
 * (ref: tnlm/kernels/poly_attn.py). Every entry point takes plain pointers, element strides and sizes; the caller
 * owns all device memory (the library never allocates), and work is enqueued asynchronously on the caller's HIP
 * stream (passed as void*, e.g. torch.cuda.current_stream().cuda_stream). Entry points return 0 on success and a
 * nonzero tnpa_status otherwise; tnpa_last_error() then describes the failure (thread-local). Argument errors are
 * detected before anything is enqueued.
 *
 * Semantics (ref: tnlm/attention.py:22-38,54-77; tnlm/kernels/poly_attn.py:1-16):
 *   y_i = row_scale_i * sum_{j visible from i} A(S1_ij, S2_ij) v_j,   S_ij = q_i . k_j / sqrt(dk)
 *   visible(i, j): j <= i, same (contiguous) document, both tokens real (doc id >= 0);
 *   A: signed_product S1*S2 | offset_square (S1 + b_h)^2 | lower_degree_mix c0 + c1 S1 + c2 S2 + c12 S1 S2
 *      | power S1^degree (this build's degree-p kind; degree 2 equals signed_product with q2 = q1, k2 = k1).
 *   The mask is applied after the polynomial; scores, products and accumulators are FP32; the masked product is
 *   rounded to the input dtype before each matrix-core product.
 */
#ifndef TNPA_H
#define TNPA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TNPA_ABI_VERSION 4

typedef enum {
  TNPA_OK = 0,
  TNPA_ERR_INVALID = 1,     /* bad shape / stride / dtype / pointer: maps to Python ValueError */
  TNPA_ERR_UNSUPPORTED = 2, /* valid per the reference contract but outside this build (e.g. head dim 512, fp32 with two q/k pairs above head dim 128) */
  TNPA_ERR_LAUNCH = 3       /* HIP launch failure: maps to Python RuntimeError */
} tnpa_status;

typedef enum { TNPA_BF16 = 0, TNPA_F32 = 1, TNPA_F16 = 2 } tnpa_dtype;

/* ref: tnlm/kernels/poly_attn.py:23 (KINDS) plus TNPA_POWER */
typedef enum { TNPA_SIGNED_PRODUCT = 0, TNPA_OFFSET_SQUARE = 1, TNPA_LOWER_DEGREE_MIX = 2, TNPA_POWER = 3 } tnpa_kind;

/* A (B, H, T, d) tensor view: element strides over batch, head and time; the head dim must have unit stride.
 * Row starts must be 16-byte aligned (data pointer and every stride times the element size). */
typedef struct {
  const void* data;
  int64_t stride_b, stride_h, stride_t;
} tnpa_tensor_t;

/* Inputs shared by forward and backward. q1/k1/q2/k2 are (B,H,T,dk); v is (B,H,T,dv). For kinds with one pair
 * (offset_square, power) q2/k2 are ignored. doc_start/query_end come from tnpa_doc_bounds (ref _block_bounds,
 * tnlm/kernels/poly_attn.py:205-218, restated per token). row_scale is (B,T) fp32 contiguous: n_visible^-p for real
 * tokens, 0 for padding (ref: tnlm/kernels/poly_attn.py:312-314). coef is (H,4) fp32 contiguous for
 * lower_degree_mix; offset is (H) fp32 contiguous for offset_square.
 * score_norms (optional, NULL to skip): an fp32 (pairs, 2, H) output of tnpa_forward, zero on entry, that receives
 * max over (b, t) of the Euclidean norm of q_pair[b,h,t,:] ([pair][0][h]) and of k_pair[b,h,t,:] ([pair][1][h]),
 * over every token (padding included), pairs = 2 for signed_product / lower_degree_mix and 1 otherwise: the two
 * factors of the reference's Cauchy-Schwarz score bound max|S| <= max|q| max|k| / sqrt(dk)
 * (ref: tnlm/model.py:33-38,83-85), taken from the rows the forward kernel reads anyway.
 * rope_cos / rope_sin (optional, both or neither): per-token rotary tables, (B, T, dk/2) fp32 contiguous and
 * 16-byte aligned, as the
 * reference's rope_tables builds them (ref: tnlm/attention.py:41-45; its (B, 1, T, dk/2) layout is the same memory).
 * With them, q1/k1 (q2/k2) are the inputs already rotated by these tables (tnpa_rope), tnpa_forward is unchanged,
 * and tnpa_backward returns dq/dk with respect to the unrotated inputs: the gradient of the rotation is applied to
 * them in the library (ref: tnlm/attention.py:48-51 and its autograd), so the caller runs no pass of its own. */
typedef struct {
  int32_t batch, heads, seq_len, head_dim_k, head_dim_v;
  int32_t kind;   /* tnpa_kind */
  int32_t degree; /* TNPA_POWER only, 1..8 */
  int32_t dtype;  /* tnpa_dtype of q1, k1, q2, k2, v and of every output / gradient */
  tnpa_tensor_t q1, k1, q2, k2, v;
  const int32_t* doc_start;
  const int32_t* query_end;
  const float* row_scale;
  const float* coef;
  const float* offset;
  float* score_norms;
  const float* rope_cos;
  const float* rope_sin;
} tnpa_problem_t;

/* Gradients for tnpa_backward. dout is dL/dy (B,H,T,dv). dq2/dk2 are ignored for one-pair kinds. dpar is an (H,4)
 * fp32 output (column 0 = db for offset_square, the 4 columns = dcoef for lower_degree_mix), required for those two
 * kinds and ignored otherwise. workspace is caller-allocated device memory of at least
 * tnpa_backward_workspace_bytes(problem) bytes, 256-byte aligned (NULL when that is 0); its contents on entry do not
 * matter and on return are unspecified. It stands for the reference's per-call scratch (the DPAR partials of
 * ref: tnlm/kernels/poly_attn.py:296), so the library itself never allocates. For 16-bit inputs at key head dim
 * 128 it also holds the bf16/fp16 gradient dS of every 32x32 (query, key) sub-block on or below the diagonal, one
 * set per q/k pair (about B*H*T^2 bytes per pair, 545 MB at B8 H16 T2048; only while all sets stay within 4 GiB),
 * from which each dQ is computed with one matrix product instead of recomputing S (both pairs) and dP. */
typedef struct {
  tnpa_tensor_t dout, dq1, dk1, dq2, dk2, dv;
  float* dpar;
  void* workspace;
  int64_t workspace_bytes;
} tnpa_grads_t;

/* Library ABI version (TNPA_ABI_VERSION). */
int tnpa_abi_version(void);

/* Message for the last nonzero return on this thread ("" if none). */
const char* tnpa_last_error(void);

/* Per-token visibility bounds from document ids (B,T), int32 (doc_is_int64 = 0) or int64 (1), row stride
 * doc_stride_b elements: doc_start[b,t] = first key visible from t (t + 1 for padding), query_end[b,t] = one past
 * the last query that sees key t. Replaces ref: tnlm/kernels/poly_attn.py:205-218 (_block_bounds) and
 * ref: tnlm/attention.py:12-19 (doc_positions); ids must be contiguous runs, negative = padding. */
int tnpa_doc_bounds(const void* doc_ids, int32_t doc_is_int64, int64_t doc_stride_b, int32_t batch,
                    int32_t seq_len, int32_t* doc_start, int32_t* query_end, void* stream);

/* Rotary position embedding of one (B,H,T,d) tensor x into out (same shape and dtype; out may be x itself) by
 * per-token tables cos / sin, (B, T, d/2) fp32 contiguous, 16-byte aligned (ref: tnlm/attention.py:41-45). One
 * pass, in fp32 with
 * x1 = x[..., :d/2], x2 = x[..., d/2:]: inverse = 0 gives out = (x1 cos - x2 sin, x1 sin + x2 cos), the reference's
 * apply_rope (ref: tnlm/attention.py:48-51, called at ref: tnlm/model.py:70-71,81-82); inverse = 1 gives the
 * gradient of that rotation with respect to its input, g -> (g1 cos + g2 sin, g2 cos - g1 sin). Every product and
 * sum is rounded to fp32 on its own and the result to the dtype, bit-identical to the reference's tensor
 * operations and their autograd. tnpa_backward applies the inverse itself when the problem carries the tables. */
int tnpa_rope(const tnpa_tensor_t* x, const tnpa_tensor_t* out, int32_t batch, int32_t heads, int32_t seq_len,
              int32_t head_dim, int32_t dtype, const float* cos, const float* sin, int32_t inverse, void* stream);

/* Forward: writes out (B,H,T,dv) in the problem dtype. Replaces ref: tnlm/kernels/poly_attn.py:271-280
 * (PolyAttention.forward launch of _fwd). */
int tnpa_forward(const tnpa_problem_t* problem, const tnpa_tensor_t* out, void* stream);

/* Bytes of device workspace tnpa_backward needs for this problem (0 if none; -1 and tnpa_last_error() for an invalid
 * problem). No counterpart in the reference, whose autograd function allocates its scratch itself
 * (ref: tnlm/kernels/poly_attn.py:294-296); here the caller allocates it and passes tnpa_grads_t.workspace. */
int64_t tnpa_backward_workspace_bytes(const tnpa_problem_t* problem);

/* Backward: writes dq1, dk1, (dq2, dk2), dv, and dpar. Replaces ref: tnlm/kernels/poly_attn.py:286-309
 * (PolyAttention.backward: _bwd_kv, _bwd_q and the fixed-order dcoef/db reduction). Deterministic: no atomics,
 * every reduction in a fixed order. How the work is split into kernel launches is internal to the library. */
int tnpa_backward(const tnpa_problem_t* problem, const tnpa_grads_t* grads, void* stream);

/* tnpa_backward without a caller workspace and without any device allocation, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. The same results as tnpa_backward (it runs the plan that streams no row-scaled dO, bit-identical to
 * tnpa_backward's, except that dQ is recomputed from S and dP where tnpa_backward reads the dS tiles it stored in its
 * workspace: 16-bit, key head dim 128; the two dQ then differ only by rounding inside the products);
 * grads->workspace and workspace_bytes are ignored. Its scratch is a fixed 1 MiB array in each
 * GPU's memory (the dcoef/db partials: B * H * ceil(T / 128 or 256) * 16 bytes), held until the process ends;
 * problems that need more fail with TNPA_ERR_UNSUPPORTED before anything is enqueued. Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (different streams or threads) race and must be serialised by the
 * caller. */
int tnpa_backward_noalloc(const tnpa_problem_t* problem, const tnpa_grads_t* grads, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TNPA_H */
