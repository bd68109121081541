// Fused cross-entropy epilogues of the chunked linear + cross-entropy (declared in include/tnce.h).
//
// One workgroup of 256 threads (four 64-wide wavefronts) per logits row. A row is read once with 16-byte loads
// (a scalar head up to 16-byte alignment and a scalar tail), so each pass over a chunk moves the chunk's logits once
// (forward) or twice (backward: read, write back in place) through HBM.
//   forward : per thread an online (max, sum of exp) over its elements in the accumulation type, combined across
//             the workgroup in a fixed butterfly/wave order; lse = max + log(sum); the row's loss term
//             lse - logit[target] (0 without a target); then one workgroup sums the row terms in a fixed order and
//             adds the sum to the caller's total.  ref: tnlm/kernels/fused_ce.py:29-33
//   backward: (exp(logit - lse) - onehot(target)) * valid * g, rounded to the logits' type, written in place.
//             ref: tnlm/kernels/fused_ce.py:45-48
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cmath>

#include "../../include/tnce.h"
#include "../../include/tnpa.h"
#include "tnpa_error.hpp"

namespace {

constexpr int NT = 256;

template <typename T> struct AccOf { typedef float type; };
template <> struct AccOf<double> { typedef double type; };

// exp(x) = 2^(x log2 e) on the hardware base-2 exponential (v_exp_f32, about 1 ulp) for float accumulation -- the
// relative error of the scaled argument stays below 1e-5 for |x| < 100, under fp32's use here (a sum of positive
// terms; a gradient rounded to the compute dtype); the full-precision exp for double.
__device__ inline float acc_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ inline double acc_exp(double x) { return exp(x); }
__device__ inline float acc_log(float x) { return logf(x); }
__device__ inline double acc_log(double x) { return log(x); }

template <typename A> __device__ inline A neg_inf() { return -__builtin_huge_valf(); }
template <> __device__ inline double neg_inf<double>() { return -__builtin_huge_val(); }

// (m, s) represents s * exp(m); merging keeps the larger exponent. -inf maxima carry no mass.
template <typename A> __device__ inline void lse_merge(A& m, A& s, A m2, A s2) {
  if (m2 == neg_inf<A>()) return;
  if (m == neg_inf<A>()) {
    m = m2;
    s = s2;
    return;
  }
  if (m2 > m) {
    s = s * acc_exp(m - m2) + s2;
    m = m2;
  } else {
    s = s + s2 * acc_exp(m2 - m);
  }
}

template <typename T>
__global__ void __launch_bounds__(NT) k_ce_fwd(const T* __restrict__ logits, int64_t V, int64_t ld,
                                               const int64_t* __restrict__ targets, int64_t ignore,
                                               typename AccOf<T>::type* __restrict__ lse,
                                               typename AccOf<T>::type* __restrict__ row_loss) {
  typedef typename AccOf<T>::type A;
  __shared__ A sm_[NT / 64], ss_[NT / 64];
  const int64_t i = blockIdx.x;
  const T* row = logits + i * ld;
  A m = neg_inf<A>(), s = 0;
  // an exact running max, rescaling the sum only when it grows: per element on the scalar head and tail, per
  // 16-byte chunk (its max first, then its terms) on the aligned body
  auto one = [&](A x) {
    if (x > m) {
      s = (m == neg_inf<A>() ? (A)0 : s * acc_exp(m - x)) + (A)1;
      m = x;
    } else {
      s += acc_exp(x - m);
    }
  };
  {
    constexpr int CE = 16 / (int)sizeof(T);
    const uintptr_t a = (uintptr_t)row;
    int64_t head = (a % 16 == 0) ? 0 : (a % sizeof(T) ? V : (int64_t)((16 - a % 16) / sizeof(T)));
    if (head > V) head = V;
    for (int64_t j = threadIdx.x; j < head; j += NT) one((A)row[j]);
    const int64_t nvec = (V - head) / CE;
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    for (int64_t v = threadIdx.x; v < nvec; v += NT) {
      const u4 raw = *(const u4*)(row + head + v * CE);
      const T* e = reinterpret_cast<const T*>(&raw);
      A x[CE];
      A cm = (A)e[0];
#pragma unroll
      for (int k = 0; k < CE; ++k) {
        x[k] = (A)e[k];
        cm = x[k] > cm ? x[k] : cm;
      }
      if (cm > m) {
        s = m == neg_inf<A>() ? (A)0 : s * acc_exp(m - cm);
        m = cm;
      }
      A cs = 0;
#pragma unroll
      for (int k = 0; k < CE; ++k) cs += acc_exp(x[k] - m);
      s += cs;
    }
    for (int64_t j = head + nvec * CE + threadIdx.x; j < V; j += NT) one((A)row[j]);
  }
  // fixed-order combine: butterfly inside each wavefront, then the wavefronts in index order
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const A m2 = __shfl_xor(m, o, 64), s2 = __shfl_xor(s, o, 64);
    // both lanes of a pair merge the same two values in the same order (smaller lane index first)
    const bool first = ((threadIdx.x & 63) & o) == 0;
    A ma = first ? m : m2, sa = first ? s : s2;
    lse_merge(ma, sa, first ? m2 : m, first ? s2 : s);
    m = ma;
    s = sa;
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sm_[w] = m;
    ss_[w] = s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    A M = sm_[0], S = ss_[0];
    for (int k = 1; k < NT / 64; ++k) lse_merge(M, S, sm_[k], ss_[k]);
    const A l = M + acc_log(S);
    lse[i] = l;
    const int64_t t = targets[i];
    A term = 0;
    if (t != ignore) term = (t >= 0 && t < V) ? l - (A)row[t] : (A)NAN;
    row_loss[i] = term;
  }
}

// total += sum of the n row terms, in a fixed order: thread k sums rows k, k + NT, ... in order, then a fixed tree.
template <typename A> __global__ void __launch_bounds__(NT) k_ce_sum(const A* __restrict__ row_loss, int64_t n, A* total) {
  __shared__ A part[NT];
  A acc = 0;
  for (int64_t r = threadIdx.x; r < n; r += NT) acc += row_loss[r];
  part[threadIdx.x] = acc;
  __syncthreads();
  for (int o = NT / 2; o >= 1; o >>= 1) {
    if ((int)threadIdx.x < o) part[threadIdx.x] += part[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) *total += part[0];
}

template <typename T>
__global__ void __launch_bounds__(NT) k_ce_bwd(T* __restrict__ logits, int64_t V, int64_t ld,
                                               const int64_t* __restrict__ targets, int64_t ignore,
                                               const typename AccOf<T>::type* __restrict__ lse,
                                               const typename AccOf<T>::type* __restrict__ g) {
  typedef typename AccOf<T>::type A;
  constexpr int CE = 16 / (int)sizeof(T);
  const int64_t i = blockIdx.x;
  T* row = logits + i * ld;
  const int64_t t = targets[i];
  const A scale = t != ignore ? *g : (A)0;
  const A l = lse[i];
  auto val = [&](int64_t j, A x) { return (T)((acc_exp(x - l) - (j == t ? (A)1 : (A)0)) * scale); };
  const uintptr_t a = (uintptr_t)row;
  int64_t head = (a % 16 == 0) ? 0 : (a % sizeof(T) ? V : (int64_t)((16 - a % 16) / sizeof(T)));
  if (head > V) head = V;
  for (int64_t j = threadIdx.x; j < head; j += NT) row[j] = val(j, (A)row[j]);
  const int64_t nvec = (V - head) / CE;
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
  for (int64_t v = threadIdx.x; v < nvec; v += NT) {
    u4 raw = *(const u4*)(row + head + v * CE);
    T* e = reinterpret_cast<T*>(&raw);
#pragma unroll
    for (int k = 0; k < CE; ++k) e[k] = val(head + v * CE + k, (A)e[k]);
    *(u4*)(row + head + v * CE) = raw;
  }
  for (int64_t j = head + nvec * CE + threadIdx.x; j < V; j += NT) row[j] = val(j, (A)row[j]);
}

// acc[i] += (A)part[i] over n elements: one chunk's dW product (rounded to the matmul's type, as the reference's
// `dw += (p.T @ x).to(acc)` rounds it) added to the accumulation-type dW in one pass, 16 bytes of part per thread
// step (grid-stride); the same single addition per element as the reference.
template <typename T>
__global__ void __launch_bounds__(NT) k_ce_acc(typename AccOf<T>::type* __restrict__ acc, const T* __restrict__ part,
                                               int64_t n) {
  typedef typename AccOf<T>::type A;
  constexpr int CE = 16 / (int)sizeof(T);
  const int64_t nvec = n / CE;
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
  const int64_t stride = (int64_t)gridDim.x * NT;
  for (int64_t v = (int64_t)blockIdx.x * NT + threadIdx.x; v < nvec; v += stride) {
    const u4 raw = *(const u4*)(part + v * CE);
    const T* e = reinterpret_cast<const T*>(&raw);
    A* d = acc + v * CE;
#pragma unroll
    for (int k = 0; k < CE; ++k) d[k] += (A)e[k];
  }
  for (int64_t j = nvec * CE + (int64_t)blockIdx.x * NT + threadIdx.x; j < n; j += stride) acc[j] += (A)part[j];
}

int check_args(const void* logits, int32_t dtype, int64_t n, int64_t V, int64_t ld, const int64_t* targets,
               const void* lse, const char* what) {
  if (dtype < TNCE_BF16 || dtype > TNCE_F64) return tnpa::set_error(TNPA_ERR_INVALID, "%s: unknown dtype %d", what, dtype);
  if (n < 0 || V <= 0 || ld < V)
    return tnpa::set_error(TNPA_ERR_INVALID, "%s: need n >= 0, V > 0 and ld >= V (got %lld, %lld, %lld)", what,
                           (long long)n, (long long)V, (long long)ld);
  if (n > 0x7fffffffLL) return tnpa::set_error(TNPA_ERR_UNSUPPORTED, "%s: more than 2^31 rows in one chunk", what);
  if (n > 0 && (logits == nullptr || targets == nullptr || lse == nullptr))
    return tnpa::set_error(TNPA_ERR_INVALID, "%s: null pointer", what);
  return TNPA_OK;
}

template <typename T>
hipError_t launch_fwd(const void* logits, int64_t n, int64_t V, int64_t ld, const int64_t* targets, int64_t ignore,
                      void* lse, void* row_loss, void* total, hipStream_t s) {
  typedef typename AccOf<T>::type A;
  if (n > 0)
    hipLaunchKernelGGL(k_ce_fwd<T>, dim3((unsigned)n), dim3(NT), 0, s, (const T*)logits, V, ld, targets, ignore,
                       (A*)lse, (A*)row_loss);
  hipLaunchKernelGGL(k_ce_sum<A>, dim3(1), dim3(NT), 0, s, (const A*)row_loss, n, (A*)total);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_bwd(void* logits, int64_t n, int64_t V, int64_t ld, const int64_t* targets, int64_t ignore,
                      const void* lse, const void* g, hipStream_t s) {
  typedef typename AccOf<T>::type A;
  if (n > 0)
    hipLaunchKernelGGL(k_ce_bwd<T>, dim3((unsigned)n), dim3(NT), 0, s, (T*)logits, V, ld, targets, ignore,
                       (const A*)lse, (const A*)g);
  return hipGetLastError();
}

template <typename T> hipError_t launch_acc(void* acc, const void* part, int64_t n, hipStream_t s) {
  typedef typename AccOf<T>::type A;
  constexpr int CE = 16 / (int)sizeof(T);
  const int64_t blocks = std::min<int64_t>((n / CE + NT - 1) / NT + 1, 8192);
  if (n > 0) hipLaunchKernelGGL(k_ce_acc<T>, dim3((unsigned)blocks), dim3(NT), 0, s, (A*)acc, (const T*)part, n);
  return hipGetLastError();
}

}  // namespace

extern "C" {

int tnce_accumulate(void* acc, const void* part, int32_t dtype, int64_t n, void* stream) {
  if (dtype < TNCE_BF16 || dtype > TNCE_F64) return tnpa::set_error(TNPA_ERR_INVALID, "tnce_accumulate: unknown dtype %d", dtype);
  if (n < 0) return tnpa::set_error(TNPA_ERR_INVALID, "tnce_accumulate: negative size");
  if (n > 0 && (acc == nullptr || part == nullptr)) return tnpa::set_error(TNPA_ERR_INVALID, "tnce_accumulate: null pointer");
  if (n > 0 && (((uintptr_t)acc) % 16 != 0 || ((uintptr_t)part) % 16 != 0))
    return tnpa::set_error(TNPA_ERR_INVALID, "tnce_accumulate: pointers must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  switch (dtype) {
    case TNCE_BF16: e = launch_acc<__bf16>(acc, part, n, s); break;
    case TNCE_F16: e = launch_acc<_Float16>(acc, part, n, s); break;
    case TNCE_F32: e = launch_acc<float>(acc, part, n, s); break;
    default: e = launch_acc<double>(acc, part, n, s); break;
  }
  if (e != hipSuccess) return tnpa::set_error(TNPA_ERR_LAUNCH, "tnce_accumulate: %s", hipGetErrorString(e));
  return tnpa::clear_error();
}

int tnce_forward_chunk(const void* logits, int32_t dtype, int64_t n, int64_t V, int64_t ld, const int64_t* targets,
                       int64_t ignore_index, void* lse, void* row_loss, void* total, void* stream) {
  int rc = check_args(logits, dtype, n, V, ld, targets, lse, "tnce_forward_chunk");
  if (rc) return rc;
  if (total == nullptr || (n > 0 && row_loss == nullptr))
    return tnpa::set_error(TNPA_ERR_INVALID, "tnce_forward_chunk: null row_loss / total");
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  switch (dtype) {
    case TNCE_BF16: e = launch_fwd<__bf16>(logits, n, V, ld, targets, ignore_index, lse, row_loss, total, s); break;
    case TNCE_F16: e = launch_fwd<_Float16>(logits, n, V, ld, targets, ignore_index, lse, row_loss, total, s); break;
    case TNCE_F32: e = launch_fwd<float>(logits, n, V, ld, targets, ignore_index, lse, row_loss, total, s); break;
    default: e = launch_fwd<double>(logits, n, V, ld, targets, ignore_index, lse, row_loss, total, s); break;
  }
  if (e != hipSuccess) return tnpa::set_error(TNPA_ERR_LAUNCH, "tnce_forward_chunk: %s", hipGetErrorString(e));
  return tnpa::clear_error();
}

int tnce_backward_chunk(void* logits, int32_t dtype, int64_t n, int64_t V, int64_t ld, const int64_t* targets,
                        int64_t ignore_index, const void* lse, const void* g, void* stream) {
  int rc = check_args(logits, dtype, n, V, ld, targets, lse, "tnce_backward_chunk");
  if (rc) return rc;
  if (g == nullptr) return tnpa::set_error(TNPA_ERR_INVALID, "tnce_backward_chunk: null g");
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  switch (dtype) {
    case TNCE_BF16: e = launch_bwd<__bf16>(logits, n, V, ld, targets, ignore_index, lse, g, s); break;
    case TNCE_F16: e = launch_bwd<_Float16>(logits, n, V, ld, targets, ignore_index, lse, g, s); break;
    case TNCE_F32: e = launch_bwd<float>(logits, n, V, ld, targets, ignore_index, lse, g, s); break;
    default: e = launch_bwd<double>(logits, n, V, ld, targets, ignore_index, lse, g, s); break;
  }
  if (e != hipSuccess) return tnpa::set_error(TNPA_ERR_LAUNCH, "tnce_backward_chunk: %s", hipGetErrorString(e));
  return tnpa::clear_error();
}

}  // extern "C"
