// C ABI of libtnpa.so: argument validation, dtype/kind/head-dim dispatch to the kernel instantiations, the
// document-bounds prepass, the backward plan (its launches and the carving of the caller's workspace) and the
// fixed-order dcoef/db reduction. Declared in include/tnpa.h and tnpa_internal.h.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "../../include/tnpa.h"
#include "tnpa_error.hpp"
#include "tnpa_internal.h"
#include "tnpa_params.hpp"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int ok() {
  g_err.clear();
  return TNPA_OK;
}

}  // namespace

namespace tnpa {
int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}
int clear_error() { return ok(); }
}  // namespace tnpa

namespace {

int esize(int dtype) { return dtype == TNPA_F32 ? 4 : 2; }

bool valid_dim(int d) { return d >= 16 && (d & (d - 1)) == 0; }

// Validates one (B,H,T,d) tensor view. `name` is used in messages.
int check_tensor(const tnpa_tensor_t& t, const char* name, const tnpa_problem_t& p, int es) {
  if (t.data == nullptr) return fail(TNPA_ERR_INVALID, "%s: null data pointer", name);
  if (((uintptr_t)t.data) % 16 != 0) return fail(TNPA_ERR_INVALID, "%s: data pointer not 16-byte aligned", name);
  if (t.stride_t <= 0 || (t.stride_t * es) % 16 != 0)
    return fail(TNPA_ERR_INVALID, "%s: time stride %lld elements must be positive with 16-byte aligned rows", name,
                (long long)t.stride_t);
  if (p.batch > 1 && (t.stride_b * es) % 16 != 0)
    return fail(TNPA_ERR_INVALID, "%s: batch stride %lld not 16-byte aligned", name, (long long)t.stride_b);
  if (p.heads > 1 && (t.stride_h * es) % 16 != 0)
    return fail(TNPA_ERR_INVALID, "%s: head stride %lld not 16-byte aligned", name, (long long)t.stride_h);
  return TNPA_OK;
}

bool two_pairs(int kind) { return kind == TNPA_SIGNED_PRODUCT || kind == TNPA_LOWER_DEGREE_MIX; }
int poly_of(const tnpa_problem_t& p);

int check_problem(const tnpa_problem_t* pp) {
  if (pp == nullptr) return fail(TNPA_ERR_INVALID, "null problem");
  const tnpa_problem_t& p = *pp;
  if (p.batch <= 0 || p.heads <= 0 || p.seq_len <= 0)
    return fail(TNPA_ERR_INVALID, "batch, heads and seq_len must be positive (got %d, %d, %d)", p.batch, p.heads,
                p.seq_len);
  if (!valid_dim(p.head_dim_k) || !valid_dim(p.head_dim_v))
    return fail(TNPA_ERR_INVALID, "head dims: powers of 2 >= 16 (got dk=%d, dv=%d)", p.head_dim_k, p.head_dim_v);
  if (p.head_dim_k > 256 || p.head_dim_v > 256)
    return fail(TNPA_ERR_UNSUPPORTED, "head dims above 256 are not built (got dk=%d, dv=%d)", p.head_dim_k,
                p.head_dim_v);
  if (p.kind < 0 || p.kind > 3) return fail(TNPA_ERR_INVALID, "unknown kind %d", p.kind);
  if (p.kind == TNPA_POWER && (p.degree < 1 || p.degree > 8))
    return fail(TNPA_ERR_INVALID, "power kind needs degree in 1..8 (got %d)", p.degree);
  if (p.dtype != TNPA_BF16 && p.dtype != TNPA_F32 && p.dtype != TNPA_F16)
    return fail(TNPA_ERR_INVALID, "unknown dtype %d", p.dtype);
  if (!tnpa::dims_built(p.dtype == TNPA_F32, poly_of(p), p.head_dim_k, p.head_dim_v))
    return fail(TNPA_ERR_UNSUPPORTED, "fp32 with two q/k pairs is built for head dims up to 128 (got dk=%d, dv=%d)",
                p.head_dim_k, p.head_dim_v);
  const long long blocks = (long long)p.batch * p.heads * ((p.seq_len + 31) / 32);
  if (blocks > 0x7fffffffLL) return fail(TNPA_ERR_UNSUPPORTED, "problem too large for one launch");
  const int es = esize(p.dtype);
  int rc;
  if ((rc = check_tensor(p.q1, "q1", p, es))) return rc;
  if ((rc = check_tensor(p.k1, "k1", p, es))) return rc;
  if (two_pairs(p.kind)) {
    if ((rc = check_tensor(p.q2, "q2", p, es))) return rc;
    if ((rc = check_tensor(p.k2, "k2", p, es))) return rc;
  }
  if ((rc = check_tensor(p.v, "v", p, es))) return rc;
  if (p.doc_start == nullptr || p.query_end == nullptr)
    return fail(TNPA_ERR_INVALID, "doc_start / query_end missing (run tnpa_doc_bounds first)");
  if (p.row_scale == nullptr) return fail(TNPA_ERR_INVALID, "row_scale missing");
  if (p.kind == TNPA_LOWER_DEGREE_MIX && p.coef == nullptr)
    return fail(TNPA_ERR_INVALID, "lower_degree_mix needs coef (H,4)");
  if (p.kind == TNPA_OFFSET_SQUARE && p.offset == nullptr)
    return fail(TNPA_ERR_INVALID, "offset_square needs offset (H)");
  if ((p.rope_cos == nullptr) != (p.rope_sin == nullptr))
    return fail(TNPA_ERR_INVALID, "rope_cos and rope_sin: both or neither");
  if (((uintptr_t)p.rope_cos) % 16 != 0 || ((uintptr_t)p.rope_sin) % 16 != 0)
    return fail(TNPA_ERR_INVALID, "rope_cos / rope_sin must be 16-byte aligned");
  return TNPA_OK;
}

tnpa::TDesc desc(const tnpa_tensor_t& t) { return tnpa::TDesc{t.data, t.stride_b, t.stride_h, t.stride_t}; }

tnpa::KParams make_params(const tnpa_problem_t& p) {
  tnpa::KParams k{};
  k.q1 = desc(p.q1);
  k.k1 = desc(p.k1);
  k.q2 = two_pairs(p.kind) ? desc(p.q2) : desc(p.q1);
  k.k2 = two_pairs(p.kind) ? desc(p.k2) : desc(p.k1);
  k.v = desc(p.v);
  k.dstart = p.doc_start;
  k.qend = p.query_end;
  k.rscale = p.row_scale;
  k.coef = p.coef;
  k.offs = p.offset;
  k.norms = p.score_norms;
  k.B = p.batch;
  k.H = p.heads;
  k.T = p.seq_len;
  k.kind = p.kind;
  k.deg = p.kind == TNPA_POWER ? p.degree : 2;
  const double sm = 1.0 / std::sqrt((double)p.head_dim_k);
  k.sm = (float)sm;
  // fp16: the kernels scale each score by sm before the polynomial (tnpa::prescaled), so only the chain-rule sm of
  // dS/dr remains for the gradients
  const bool pre = p.dtype == TNPA_F16;
  switch (p.kind) {
    case TNPA_SIGNED_PRODUCT:
      k.vf = pre ? 1.0f : (float)(sm * sm);
      k.gf = pre ? (float)sm : (float)(sm * sm);
      break;
    case TNPA_POWER:
      k.vf = pre ? 1.0f : (float)std::pow(sm, k.deg);
      k.gf = pre ? (float)(k.deg * sm) : (float)(k.deg * std::pow(sm, k.deg));
      break;
    default: k.vf = 1.0f; k.gf = (float)sm; break;
  }
  return k;
}

int poly_of(const tnpa_problem_t& p) {
  if (p.kind == TNPA_POWER) return p.degree == 2 ? tnpa::POLY_POW2 : p.degree == 4 ? tnpa::POLY_POW4 : tnpa::POLY_GEN1;
  if (p.kind == TNPA_OFFSET_SQUARE) return tnpa::POLY_OS;
  return p.kind == TNPA_SIGNED_PRODUCT ? tnpa::POLY_SP : tnpa::POLY_GEN2;
}

enum Phase { PH_FWD = 0, PH_BWD_KV = 1, PH_BWD_Q = 2 };

template <typename T, int POLY>
hipError_t run_dims(int ph, int dk, int dv, const tnpa::KParams& k, hipStream_t s) {
#define TNPA_CASE(DK_, DV_)                                                                   \
  if (dk == DK_ && dv == DV_)                                                                 \
    return ph == PH_FWD      ? tnpa::launch_fwd<T, POLY, DK_, DV_>(k, s)                      \
           : ph == PH_BWD_KV ? tnpa::launch_bwd_kv<T, POLY, DK_, DV_>(k, s)                   \
                             : tnpa::launch_bwd_q<T, POLY, DK_, DV_>(k, s);
#define TNPA_ROW(DK_) TNPA_CASE(DK_, 16) TNPA_CASE(DK_, 32) TNPA_CASE(DK_, 64) TNPA_CASE(DK_, 128) TNPA_CASE(DK_, 256)
  TNPA_ROW(16) TNPA_ROW(32) TNPA_ROW(64) TNPA_ROW(128) TNPA_ROW(256)
#undef TNPA_ROW
#undef TNPA_CASE
  return hipErrorInvalidValue;
}

template <typename T>
hipError_t run_poly(int ph, int poly, int dk, int dv, const tnpa::KParams& k, hipStream_t s) {
  switch (poly) {
    case tnpa::POLY_GEN1: return run_dims<T, tnpa::POLY_GEN1>(ph, dk, dv, k, s);
    case tnpa::POLY_GEN2: return run_dims<T, tnpa::POLY_GEN2>(ph, dk, dv, k, s);
    case tnpa::POLY_POW4: return run_dims<T, tnpa::POLY_POW4>(ph, dk, dv, k, s);
    case tnpa::POLY_OS: return run_dims<T, tnpa::POLY_OS>(ph, dk, dv, k, s);
    case tnpa::POLY_SP: return run_dims<T, tnpa::POLY_SP>(ph, dk, dv, k, s);
    default: return run_dims<T, tnpa::POLY_POW2>(ph, dk, dv, k, s);
  }
}

hipError_t run(int ph, const tnpa_problem_t& p, const tnpa::KParams& k, hipStream_t s) {
  const int poly = poly_of(p);
  switch (p.dtype) {
    case TNPA_BF16: return run_poly<__bf16>(ph, poly, p.head_dim_k, p.head_dim_v, k, s);
    case TNPA_F16: return run_poly<_Float16>(ph, poly, p.head_dim_k, p.head_dim_v, k, s);
    default: return run_poly<float>(ph, poly, p.head_dim_k, p.head_dim_v, k, s);
  }
}

// ---------------------------------------------------------------------------------------------- prepass kernels
// One workgroup of 1024 threads per batch row. A run start is a token whose id differs from its predecessor's;
// doc_start[t] = last run start <= t (t + 1 for padding), query_end[t] = first run start > t, or T (t for padding).
// The row goes through LDS in chunks of 4096 ids (coalesced loads; each thread then owns 4 consecutive tokens and
// writes them as one 16-byte store): a forward pass carries the last start across chunks with a max-scan, a
// backward pass the next start with a min-scan, starting on the chunk the forward pass left in LDS.
__global__ void __launch_bounds__(1024) k_doc_bounds(const void* doc, int is64, int64_t sb, int T, int* dstart,
                                                     int* qend) {
  constexpr int NT = 1024, L = 4, CH = NT * L, NW = NT / 64;
  __shared__ int64_t sid[CH + 1];  // sid[k] = id(c0 - 1 + k)
  __shared__ int wred[NW];
  const int b = blockIdx.x, t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t* d64 = (const int64_t*)doc + (int64_t)b * sb;
  const int* d32 = (const int*)doc + (int64_t)b * sb;
  int* ds = dstart + (int64_t)b * T;
  int* qe = qend + (int64_t)b * T;
  auto load_chunk = [&](int c0, int n) {
    for (int k = t; k <= n; k += NT) {
      const int i = c0 - 1 + k;
      sid[k] = i < 0 ? INT64_MIN : (is64 ? d64[i] : (int64_t)d32[i]);
    }
    __syncthreads();
  };
  // run start at chunk offset k (token c0 + k)
  auto start_at = [&](int c0, int k) { return c0 + k == 0 || sid[k + 1] != sid[k]; };

  int carry = -1;  // last run start before the chunk
  for (int c0 = 0; c0 < T; c0 += CH) {
    const int n = min(CH, T - c0);
    load_chunk(c0, n);
    int last = -1;
#pragma unroll
    for (int j = 0; j < L; ++j) {
      const int k = t * L + j;
      if (k < n && start_at(c0, k)) last = c0 + k;
    }
    int x = last;  // inclusive max-scan over the threads
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (lane >= o) x = max(x, y);
    }
    if (lane == 63) wred[w] = x;
    __syncthreads();
    int cur = carry, all = carry;
    for (int v = 0; v < NW; ++v) {
      if (v < w) cur = max(cur, wred[v]);
      all = max(all, wred[v]);
    }
    const int prev = __shfl_up(x, 1, 64);
    if (lane > 0) cur = max(cur, prev);
    if (t * L < n) {
      int o[L];
#pragma unroll
      for (int j = 0; j < L; ++j) {
        const int k = t * L + j;
        if (k < n && start_at(c0, k)) cur = c0 + k;
        o[j] = k < n && sid[k + 1] < 0 ? c0 + k + 1 : cur;
      }
      if (c0 + t * L + L <= T && ((uintptr_t)(ds + c0 + t * L) & 15) == 0) {
        *(int4*)(ds + c0 + t * L) = make_int4(o[0], o[1], o[2], o[3]);
      } else {
        for (int j = 0; j < L && t * L + j < n; ++j) ds[c0 + t * L + j] = o[j];
      }
    }
    carry = all;
    __syncthreads();  // before the next chunk overwrites sid and wred
  }

  int carry2 = T;  // first run start after the chunk
  const int clast = ((T - 1) / CH) * CH;  // still in LDS from the forward pass
  for (int c0 = clast; c0 >= 0; c0 -= CH) {
    const int n = min(CH, T - c0);
    if (c0 != clast) load_chunk(c0, n);
    int first = T;
#pragma unroll
    for (int j = L - 1; j >= 0; --j) {
      const int k = t * L + j;
      if (k < n && start_at(c0, k)) first = c0 + k;
    }
    int x = first;  // inclusive min-scan over the threads, from the end
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_down(x, o, 64);
      if (lane + o < 64) x = min(x, y);
    }
    if (lane == 0) wred[w] = x;
    __syncthreads();
    int nxt = carry2, all = carry2;
    for (int v = 0; v < NW; ++v) {
      if (v > w) nxt = min(nxt, wred[v]);
      all = min(all, wred[v]);
    }
    const int after = __shfl_down(x, 1, 64);
    if (lane < 63) nxt = min(nxt, after);
    if (t * L < n) {
      int o[L];
#pragma unroll
      for (int j = L - 1; j >= 0; --j) {
        const int k = t * L + j;
        o[j] = k < n && sid[k + 1] < 0 ? c0 + k : nxt;
        if (k < n && start_at(c0, k)) nxt = c0 + k;
      }
      if (c0 + t * L + L <= T && ((uintptr_t)(qe + c0 + t * L) & 15) == 0) {
        *(int4*)(qe + c0 + t * L) = make_int4(o[0], o[1], o[2], o[3]);
      } else {
        for (int j = 0; j < L && t * L + j < n; ++j) qe[c0 + t * L + j] = o[j];
      }
    }
    carry2 = all;
    __syncthreads();
  }
}

// out[b,h,t,:] = row_scale[b,t] * dout[b,h,t,:], one 16-byte chunk per thread (grid-stride), computed in fp32 and
// rounded to T exactly as the dK/dV pass rounds it when it scales dout while staging.
template <typename T>
__global__ void __launch_bounds__(256) k_scale_rows(const T* __restrict__ dout, int64_t sb, int64_t sh, int64_t st,
                                                    const float* __restrict__ rs, int B, int H, int T_, int D,
                                                    T* __restrict__ out, int64_t ob, int64_t oh, int64_t ot) {
  constexpr int CE = 16 / (int)sizeof(T);
  const int nch = D / CE;
  const int64_t total = (int64_t)B * H * T_ * nch;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(i % nch);
    const int64_t row = i / nch;
    const int t = (int)(row % T_);
    const int64_t bh = row / T_;
    const int h = (int)(bh % H), b = (int)(bh / H);
    const float f = rs[(int64_t)b * T_ + t];
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    u4 raw = *(const u4*)(dout + b * sb + h * sh + t * st + c * CE);
    if constexpr (sizeof(T) == 2) {
      T* e = reinterpret_cast<T*>(&raw);
#pragma unroll
      for (int j = 0; j < 8; ++j) e[j] = (T)((float)e[j] * f);
    } else {
      float* e = reinterpret_cast<float*>(&raw);
#pragma unroll
      for (int j = 0; j < 4; ++j) e[j] *= f;
    }
    *(u4*)(out + b * ob + h * oh + t * ot + c * CE) = raw;
  }
}

template <typename T>
hipError_t scale_rows(const tnpa_problem_t& p, const tnpa_tensor_t& d, const tnpa_tensor_t& o, hipStream_t s) {
  const int CE = 16 / (int)sizeof(T);
  const int64_t total = (int64_t)p.batch * p.heads * p.seq_len * (p.head_dim_v / CE);
  const int grid = (int)std::min<int64_t>((total + 255) / 256, 8192);
  hipLaunchKernelGGL(k_scale_rows<T>, dim3(grid), dim3(256), 0, s, (const T*)d.data, d.stride_b, d.stride_h,
                     d.stride_t, p.row_scale, p.batch, p.heads, p.seq_len, p.head_dim_v, (T*)o.data, o.stride_b,
                     o.stride_h, o.stride_t);
  return hipGetLastError();
}

// Rotary position embedding of a (B, H, T, d) tensor by per-token tables cos / sin, (B, T, d/2) fp32
// (ref: tnlm/attention.py:48-51): x1 = x[..., :d/2], x2 = x[..., d/2:] in fp32;
//   forward: out = (x1 cos - x2 sin, x1 sin + x2 cos);
//   INV, the gradient of the forward as autograd forms it from g = dL/dout: (g1 cos + g2 sin, g2 cos - g1 sin).
// Every product and sum is rounded to fp32 on its own (no fused multiply-add: the reference runs them as separate
// tensor operations), then rounded to T. One thread per 16-byte chunk of x1 with the matching chunk of x2
// (grid-stride); out may be x itself.
template <typename T, bool INV>
__global__ void __launch_bounds__(256) k_rope(const T* x, int64_t sb, int64_t sh, int64_t st, T* out, int64_t ob,
                                              int64_t oh, int64_t ot, const float* __restrict__ cs,
                                              const float* __restrict__ sn, int B, int H, int T_, int D) {
#pragma clang fp contract(off)
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
  typedef float f4 __attribute__((ext_vector_type(4)));
  constexpr int CE = 16 / (int)sizeof(T);
  const int half = D / 2, nch = half / CE;
  const int64_t total = (int64_t)B * H * T_ * nch;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(i % nch);
    const int64_t row = i / nch;
    const int t = (int)(row % T_);
    const int64_t bh = row / T_;
    const int h = (int)(bh % H), b = (int)(bh / H);
    const T* xr = x + b * sb + h * sh + t * st + c * CE;
    u4 r1 = *(const u4*)xr, r2 = *(const u4*)(xr + half);
    const int64_t tab = ((int64_t)b * T_ + t) * half + c * CE;
    float cv[CE], sv[CE];
#pragma unroll
    for (int j = 0; j < CE; j += 4) {
      const f4 a = *(const f4*)(cs + tab + j), z = *(const f4*)(sn + tab + j);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        cv[j + e] = a[e];
        sv[j + e] = z[e];
      }
    }
    T* e1 = reinterpret_cast<T*>(&r1);
    T* e2 = reinterpret_cast<T*>(&r2);
#pragma unroll
    for (int j = 0; j < CE; ++j) {
      const float a = (float)e1[j], z = (float)e2[j];
      const float p1 = a * cv[j], p2 = z * sv[j], p3 = a * sv[j], p4 = z * cv[j];
      if constexpr (INV) {
        e1[j] = (T)(p1 + p2);
        e2[j] = (T)(p4 - p3);
      } else {
        e1[j] = (T)(p1 - p2);
        e2[j] = (T)(p3 + p4);
      }
    }
    T* orow = out + b * ob + h * oh + t * ot + c * CE;
    *(u4*)orow = r1;
    *(u4*)(orow + half) = r2;
  }
}

template <typename T, bool INV>
hipError_t rope_rows(const tnpa_problem_t& p, const tnpa_tensor_t& x, const tnpa_tensor_t& o, hipStream_t s) {
  const int CE = 16 / (int)sizeof(T);
  const int64_t total = (int64_t)p.batch * p.heads * p.seq_len * (p.head_dim_k / 2 / CE);
  const int grid = (int)std::min<int64_t>((total + 255) / 256, 8192);
  hipLaunchKernelGGL((k_rope<T, INV>), dim3(grid), dim3(256), 0, s, (const T*)x.data, x.stride_b, x.stride_h,
                     x.stride_t, (T*)o.data, o.stride_b, o.stride_h, o.stride_t, p.rope_cos, p.rope_sin, p.batch,
                     p.heads, p.seq_len, p.head_dim_k);
  return hipGetLastError();
}

template <bool INV>
hipError_t rope_any(const tnpa_problem_t& p, const tnpa_tensor_t& x, const tnpa_tensor_t& o, hipStream_t s) {
  switch (p.dtype) {
    case TNPA_BF16: return rope_rows<__bf16, INV>(p, x, o, s);
    case TNPA_F16: return rope_rows<_Float16, INV>(p, x, o, s);
    default: return rope_rows<float, INV>(p, x, o, s);
  }
}

// dpar[h, c] = sum over (b, key block) of the per-block partials, in a fixed order.
// ref: tnlm/kernels/poly_attn.py:304 (dpar.view(B, H, NB, 4).sum((0, 2)))
__global__ void k_dpar_reduce(const float* part, int B, int H, int NNB, float* out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= H * 4) return;
  const int hd = i / 4, c = i % 4;
  float acc = 0.f;
  for (int b = 0; b < B; ++b)
    for (int nb = 0; nb < NNB; ++nb) acc += part[(((int64_t)b * H + hd) * NNB + nb) * 4 + c];
  out[i] = acc;
}

// ---------------------------------------------------------------------------------------------- backward plan
// The launches of one backward call and the carving of the caller's workspace:
//   scale  row_scale * dO into the workspace (where the key side cannot scale dO for free, or when forced)
//   kv     the combined dK/dV kernel (the wave-pair kernel for 16-bit, one q/k pair, head dims 128), or dv and
//          dk: the two passes of the split key side (16-bit, one q/k pair, other head dims above 64)
//   q      the dQ kernel (recomputes S and dP)
//   qds    dQ = dS K from the dS tiles the key side stored in the workspace (16-bit, key head dim 128, unless
//          TNPA_X_DS_OFF or the tiles would exceed kMaxDsTileBytes): one matrix product instead of three; two
//          q/k pairs run it once per pair (dQ1 = dS1 K1, dQ2 = dS2 K2)
//   dpar   the fixed-order dcoef/db reduction of the per-key-block partials (offset_square, lower_degree_mix)
//   rope   with rotary tables, the rotation's gradient on dK in place, where the key side writes dK from its
//          accumulators (two q/k pairs, head dim 16); the dQ and the other dK epilogues apply it themselves
enum LaunchKind { L_SCALE = 0, L_KV = 1, L_DV = 2, L_DK = 3, L_Q = 4, L_DPAR = 5, L_QDS = 6, L_ROPE = 7 };
const char* const kLaunchNames[] = {"scale", "kv", "dv", "dk", "q", "dpar", "qds", "rope"};

// Largest dS tile area the plan uses (B * H * T^2 bytes for 16-bit inputs, 545 MB at B8 H16 T2048); larger problems
// recompute S and dP in the dQ kernel instead.
constexpr int64_t kMaxDsTileBytes = 4LL << 30;

struct Plan {
  int n = 0;
  int what[7] = {0, 0, 0, 0, 0, 0, 0};
  bool prescale = false, par = false, ds = false;
  int nnb = 0;  // key blocks per row (dpar partials)
  int64_t dpar_off = 0, dos_off = 0, ds_off = 0, ds2_off = 0, bytes = 0;
};

int64_t align256(int64_t x) { return (x + 255) & ~(int64_t)255; }

int make_plan(const tnpa_problem_t& p, int opts, Plan& pl) {
  if ((opts & ~(TNPA_X_PRESCALE_ON | TNPA_X_PRESCALE_OFF | TNPA_X_DS_OFF)) != 0 ||
      (opts & (TNPA_X_PRESCALE_ON | TNPA_X_PRESCALE_OFF)) == (TNPA_X_PRESCALE_ON | TNPA_X_PRESCALE_OFF))
    return fail(TNPA_ERR_INVALID, "invalid backward options %d", opts);
  const bool f32 = p.dtype == TNPA_F32;
  const int poly = poly_of(p), dk = p.head_dim_k, dv = p.head_dim_v;
  const bool split = tnpa::kv_split(f32, poly, dk, dv);
  const bool helps = !tnpa::kv_scales_in_pass(f32, poly, dk, dv);
  pl = Plan{};
  pl.prescale = (opts & TNPA_X_PRESCALE_ON) ? true : (opts & TNPA_X_PRESCALE_OFF) ? false : helps;
  pl.par = p.kind == TNPA_OFFSET_SQUARE || p.kind == TNPA_LOWER_DEGREE_MIX;
  const int bk = tnpa::kv_block_keys(f32, poly, dk, dv);
  pl.nnb = (p.seq_len + bk - 1) / bk;
  const int64_t dpar_bytes = pl.par ? (int64_t)p.batch * p.heads * pl.nnb * 4 * (int64_t)sizeof(float) : 0;
  const int64_t dos_bytes = pl.prescale ? (int64_t)p.batch * p.heads * p.seq_len * dv * esize(p.dtype) : 0;
  const int64_t ds_bytes = tnpa::ds_tile_bytes(p.batch, p.heads, p.seq_len, esize(p.dtype));
  // dS tiles (one set per q/k pair) where the key side forms dS in a dK pass (one pair) or in the combined kernel
  // (two pairs; their split passes at head dims above 128 store none), for 16-bit inputs at key head dim 128
  const int npairs = tnpa::two_pair_poly(poly) ? 2 : 1;
  pl.ds = (npairs == 1 ? split : !split) && !f32 && dk == 128 && !(opts & TNPA_X_DS_OFF) &&
          npairs * ds_bytes <= kMaxDsTileBytes;
  pl.dpar_off = 0;
  pl.dos_off = align256(dpar_bytes);
  pl.ds_off = pl.dos_off + align256(dos_bytes);
  pl.ds2_off = pl.ds_off + align256(ds_bytes);
  pl.bytes = pl.ds_off + (pl.ds ? npairs * align256(ds_bytes) : 0);
  if (pl.prescale) pl.what[pl.n++] = L_SCALE;
  if (split && !tnpa::kv_pair(f32, poly, dk, dv)) {
    pl.what[pl.n++] = L_DV;
    pl.what[pl.n++] = L_DK;
  } else {
    pl.what[pl.n++] = L_KV;
  }
  pl.what[pl.n++] = pl.ds ? L_QDS : L_Q;
  if (pl.par) pl.what[pl.n++] = L_DPAR;
  // rotary tables: the dQ epilogues and (one pair, head dims >= 32) the dK epilogue apply the rotation's gradient;
  // otherwise dK gets it in one pass at the end
  if (p.rope_cos != nullptr && !tnpa::rope_dk_epilogue(f32, poly, dk, dv)) pl.what[pl.n++] = L_ROPE;
  return TNPA_OK;
}

int run_backward(const tnpa_problem_t* problem, const tnpa_grads_t* grads, int opts, int only, hipStream_t stream) {
  int rc = check_problem(problem);
  if (rc) return rc;
  if (grads == nullptr) return fail(TNPA_ERR_INVALID, "null grads");
  const tnpa_problem_t& p = *problem;
  Plan pl;
  if ((rc = make_plan(p, opts, pl))) return rc;
  if (only < -1 || only >= pl.n) return fail(TNPA_ERR_INVALID, "launch %d out of range (plan has %d)", only, pl.n);
  if (grads->workspace_bytes < pl.bytes)
    return fail(TNPA_ERR_INVALID, "workspace of %lld bytes, this problem needs %lld (tnpa_backward_workspace_bytes)",
                (long long)grads->workspace_bytes, (long long)pl.bytes);
  char* ws = (char*)grads->workspace;
  if (pl.bytes > 0 && (ws == nullptr || ((uintptr_t)ws) % 256 != 0))
    return fail(TNPA_ERR_INVALID, "workspace must be a non-null 256-byte aligned device pointer");
  const int es = esize(p.dtype);
  if ((rc = check_tensor(grads->dout, "dout", p, es))) return rc;
  if ((rc = check_tensor(grads->dq1, "dq1", p, es))) return rc;
  if ((rc = check_tensor(grads->dk1, "dk1", p, es))) return rc;
  if ((rc = check_tensor(grads->dv, "dv", p, es))) return rc;
  if (two_pairs(p.kind)) {
    if ((rc = check_tensor(grads->dq2, "dq2", p, es))) return rc;
    if ((rc = check_tensor(grads->dk2, "dk2", p, es))) return rc;
  }
  if (pl.par && grads->dpar == nullptr) return fail(TNPA_ERR_INVALID, "offset_square / lower_degree_mix need dpar (H,4)");
  tnpa::KParams k = make_params(p);
  k.dout = desc(grads->dout);
  k.dq1 = desc(grads->dq1);
  k.dk1 = desc(grads->dk1);
  k.dq2 = two_pairs(p.kind) ? desc(grads->dq2) : desc(grads->dq1);
  k.dk2 = two_pairs(p.kind) ? desc(grads->dk2) : desc(grads->dk1);
  k.dv = desc(grads->dv);
  k.dpar = pl.par ? (float*)(ws + pl.dpar_off) : nullptr;
  tnpa_tensor_t dos{};
  if (pl.prescale) {
    const int64_t st = p.head_dim_v;
    dos = tnpa_tensor_t{ws + pl.dos_off, (int64_t)p.heads * p.seq_len * st, (int64_t)p.seq_len * st, st};
    k.dsc = desc(dos);
    k.dpre = 1;
  }
  // rotary tables: the dQ / dK epilogues apply the rotation's gradient (dK only where rope_dk_epilogue holds;
  // the other key-side kernels never read the tables)
  k.rcos = p.rope_cos;
  k.rsin = p.rope_sin;
  if (pl.ds) {
    k.dstile = ws + pl.ds_off;
    if (two_pairs(p.kind)) k.dstile2 = ws + pl.ds2_off;
  }
  for (int i = 0; i < pl.n; ++i) {
    if (only != -1 && i != only) continue;
    hipError_t e = hipSuccess;
    switch (pl.what[i]) {
      case L_SCALE:
        switch (p.dtype) {
          case TNPA_BF16: e = scale_rows<__bf16>(p, grads->dout, dos, stream); break;
          case TNPA_F16: e = scale_rows<_Float16>(p, grads->dout, dos, stream); break;
          default: e = scale_rows<float>(p, grads->dout, dos, stream); break;
        }
        break;
      case L_KV: k.kvsel = 3; e = run(PH_BWD_KV, p, k, stream); break;
      case L_DV: k.kvsel = 1; e = run(PH_BWD_KV, p, k, stream); break;
      case L_DK: k.kvsel = 2; e = run(PH_BWD_KV, p, k, stream); break;
      case L_Q: e = run(PH_BWD_Q, p, k, stream); break;
      case L_QDS: {
        // dQ1 = dS1 K1, then (two pairs) dQ2 = dS2 K2 with the same kernel
        tnpa::KParams k2 = k;
        k2.k1 = k.k2;
        k2.dq1 = k.dq2;
        k2.dstile = k.dstile2;
        for (int pr = 0; pr < (two_pairs(p.kind) ? 2 : 1) && e == hipSuccess; ++pr)
          e = p.dtype == TNPA_BF16 ? tnpa::launch_bwd_q_ds<__bf16, 128>(pr ? k2 : k, stream)
                                   : tnpa::launch_bwd_q_ds<_Float16, 128>(pr ? k2 : k, stream);
        break;
      }
      case L_ROPE:
        e = rope_any<true>(p, grads->dk1, grads->dk1, stream);
        if (two_pairs(p.kind) && e == hipSuccess) e = rope_any<true>(p, grads->dk2, grads->dk2, stream);
        break;
      case L_DPAR: {
        const int n = p.heads * 4;
        hipLaunchKernelGGL(k_dpar_reduce, dim3((n + 255) / 256), dim3(256), 0, stream, (const float*)k.dpar, p.batch,
                           p.heads, pl.nnb, grads->dpar);
        e = hipGetLastError();
        break;
      }
    }
    if (e != hipSuccess)
      return fail(TNPA_ERR_LAUNCH, "tnpa_backward (%s): %s", kLaunchNames[pl.what[i]], hipGetErrorString(e));
  }
  return ok();
}

// ---------------------------------------------------------------------------------------------- static scratch
// The workspace of tnpa_backward_noalloc: a fixed array in device memory, one copy per GPU the library runs on,
// held until the process ends. The plan it runs (no row-scaled dO) needs scratch only for the dcoef/db partials,
// which every call overwrites in full, so nothing in it needs clearing between calls.
constexpr int64_t kScratchBytes = 1 << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current GPU's scratch copy, looked up once per device (the host-side name `scratch` is only a
// stand-in and must never reach a kernel). Null on failure, with the error set.
void* scratch_for_current_device(int* rc) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    *rc = fail(TNPA_ERR_LAUNCH, "tnpa_backward_noalloc: no current HIP device (%s)", hipGetErrorString(e));
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      *rc = fail(TNPA_ERR_LAUNCH, "tnpa_backward_noalloc: scratch address on device %d: %s", dev, hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" {

int tnpa_abi_version(void) { return TNPA_ABI_VERSION; }

const char* tnpa_last_error(void) { return g_err.c_str(); }

int tnpa_doc_bounds(const void* doc_ids, int32_t doc_is_int64, int64_t doc_stride_b, int32_t batch, int32_t seq_len,
                    int32_t* doc_start, int32_t* query_end, void* stream) {
  if (doc_ids == nullptr || doc_start == nullptr || query_end == nullptr)
    return fail(TNPA_ERR_INVALID, "tnpa_doc_bounds: null pointer");
  if (batch <= 0 || seq_len <= 0) return fail(TNPA_ERR_INVALID, "tnpa_doc_bounds: batch and seq_len must be positive");
  if (batch > 1 && doc_stride_b < seq_len)
    return fail(TNPA_ERR_INVALID, "tnpa_doc_bounds: batch stride %lld shorter than seq_len", (long long)doc_stride_b);
  hipLaunchKernelGGL(k_doc_bounds, dim3(batch), dim3(1024), 0, (hipStream_t)stream, doc_ids, doc_is_int64 ? 1 : 0,
                     doc_stride_b, seq_len, doc_start, query_end);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TNPA_ERR_LAUNCH, "tnpa_doc_bounds: %s", hipGetErrorString(e));
  return ok();
}

int tnpa_rope(const tnpa_tensor_t* x, const tnpa_tensor_t* out, int32_t batch, int32_t heads, int32_t seq_len,
              int32_t head_dim, int32_t dtype, const float* cos, const float* sin, int32_t inverse, void* stream) {
  if (x == nullptr || out == nullptr || cos == nullptr || sin == nullptr)
    return fail(TNPA_ERR_INVALID, "tnpa_rope: null pointer");
  if (((uintptr_t)cos) % 16 != 0 || ((uintptr_t)sin) % 16 != 0)
    return fail(TNPA_ERR_INVALID, "tnpa_rope: cos / sin must be 16-byte aligned");
  if (batch <= 0 || heads <= 0 || seq_len <= 0) return fail(TNPA_ERR_INVALID, "tnpa_rope: sizes must be positive");
  if (!valid_dim(head_dim)) return fail(TNPA_ERR_INVALID, "tnpa_rope: head dim must be a power of 2 >= 16");
  if (dtype != TNPA_BF16 && dtype != TNPA_F32 && dtype != TNPA_F16)
    return fail(TNPA_ERR_INVALID, "tnpa_rope: unknown dtype %d", dtype);
  tnpa_problem_t p{};
  p.batch = batch;
  p.heads = heads;
  p.seq_len = seq_len;
  p.head_dim_k = head_dim;
  p.dtype = dtype;
  p.rope_cos = cos;
  p.rope_sin = sin;
  const int es = esize(dtype);
  int rc;
  if ((rc = check_tensor(*x, "x", p, es)) || (rc = check_tensor(*out, "out", p, es))) return rc;
  const hipError_t e = inverse ? rope_any<true>(p, *x, *out, (hipStream_t)stream)
                               : rope_any<false>(p, *x, *out, (hipStream_t)stream);
  if (e != hipSuccess) return fail(TNPA_ERR_LAUNCH, "tnpa_rope: %s", hipGetErrorString(e));
  return ok();
}

int tnpa_forward(const tnpa_problem_t* problem, const tnpa_tensor_t* out, void* stream) {
  int rc = check_problem(problem);
  if (rc) return rc;
  if (out == nullptr) return fail(TNPA_ERR_INVALID, "null out");
  if ((rc = check_tensor(*out, "out", *problem, esize(problem->dtype)))) return rc;
  tnpa::KParams k = make_params(*problem);
  k.o = desc(*out);
  const hipError_t e = run(PH_FWD, *problem, k, (hipStream_t)stream);
  if (e != hipSuccess) return fail(TNPA_ERR_LAUNCH, "tnpa_forward: %s", hipGetErrorString(e));
  return ok();
}

int64_t tnpa_backward_workspace_bytes(const tnpa_problem_t* problem) { return tnpa_x_workspace_bytes(problem, 0); }

int tnpa_backward(const tnpa_problem_t* problem, const tnpa_grads_t* grads, void* stream) {
  return tnpa_x_backward(problem, grads, 0, -1, stream);
}

int tnpa_backward_noalloc(const tnpa_problem_t* problem, const tnpa_grads_t* grads, void* stream) {
  int rc = check_problem(problem);
  if (rc) return rc;
  if (grads == nullptr) return fail(TNPA_ERR_INVALID, "null grads");
  Plan pl;
  if ((rc = make_plan(*problem, TNPA_X_PRESCALE_OFF | TNPA_X_DS_OFF, pl))) return rc;
  if (pl.bytes > kScratchBytes)
    return fail(TNPA_ERR_UNSUPPORTED,
                "tnpa_backward_noalloc: this problem needs %lld bytes of scratch, more than the %lld it holds "
                "(use tnpa_backward with a workspace)", (long long)pl.bytes, (long long)kScratchBytes);
  void* ptr = scratch_for_current_device(&rc);
  if (ptr == nullptr) return rc;
  tnpa_grads_t g = *grads;
  g.workspace = ptr;
  g.workspace_bytes = kScratchBytes;
  return run_backward(problem, &g, TNPA_X_PRESCALE_OFF | TNPA_X_DS_OFF, -1, (hipStream_t)stream);
}

int64_t tnpa_x_workspace_bytes(const tnpa_problem_t* problem, int32_t opts) {
  Plan pl;
  if (check_problem(problem) || make_plan(*problem, opts, pl)) return -1;
  ok();
  return pl.bytes;
}

int32_t tnpa_x_launches(const tnpa_problem_t* problem, int32_t opts) {
  Plan pl;
  if (check_problem(problem) || make_plan(*problem, opts, pl)) return -1;
  ok();
  return pl.n;
}

const char* tnpa_x_launch_name(const tnpa_problem_t* problem, int32_t opts, int32_t i) {
  Plan pl;
  if (check_problem(problem) || make_plan(*problem, opts, pl) || i < 0 || i >= pl.n) return "";
  return kLaunchNames[pl.what[i]];
}

int tnpa_x_backward(const tnpa_problem_t* problem, const tnpa_grads_t* grads, int32_t opts, int32_t only,
                    void* stream) {
  return run_backward(problem, grads, opts, only, (hipStream_t)stream);
}

}  // extern "C"
