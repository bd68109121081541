// Causal polynomial attention kernels for gfx950: forward, dQ and dK/dV.
//
// Operator semantics follow ref: tnlm/kernels/poly_attn.py:1-16 and the dense reference
// ref: tnlm/attention.py:22-38,54-77:
//     y_i = scale_i * sum_{j visible from i} A(S1_ij, S2_ij) v_j,   S_ij = q_i . k_j / sqrt(dk),
// visible(i, j) <=> doc_start[i] <= j <= i (contiguous documents; padding rows see nothing), the mask applied
// after the polynomial, FP32 accumulation, the masked product cast to the input dtype before each MFMA.
//
// Work decomposition (one workgroup = NW wavefronts of 64 lanes):
//   forward, dQ:  a workgroup owns BM = NW*QW*32 queries; wave w owns QW 32-query subtiles whose Q (and dO)
//                 operands stay in registers; K/V tiles of BN keys are staged through double-buffered LDS.
//                 S^T = K Q^T and dP^T = V dO^T leave lane <-> query, so P^T/dS^T feed O^T += V^T P^T and
//                 dQ^T += K^T dS^T directly as B operands (V^T, K^T read with the LDS transpose read).
//   dK/dV:        a workgroup owns NW*KW*32 keys; K/V operands stay in registers; Q/dO tiles of BMQ queries are
//                 staged through LDS (dO pre-multiplied by the row scale while staging). S = Q K^T and
//                 dP = dO V^T leave lane <-> key, so P/dS feed dV^T += dO^T P and dK^T += Q^T dS.
// Causal skipping: the key/query loop bounds stop at the diagonal and at document starts (tile level), and each
// wave skips 32x32 sub-blocks that are fully invisible to it (wavefront level). Only sub-blocks that straddle the
// diagonal, a document edge or the sequence end evaluate the per-element mask.
// Work items are ordered heaviest first (longest causal range), and consecutive items cycle through (b, h) so
// that all blocks of one head land on the same XCD (blockIdx % 8) and share its L2.
#pragma once

#include <climits>
#include <type_traits>

#include "tnpa_device.hpp"
#include "tnpa_params.hpp"

namespace tnpa {

struct Coefs {
  float c0, c1, c2, c12;
};

__device__ inline Coefs load_coefs(const KParams& p, int hd) {
  Coefs c{0.f, 0.f, 0.f, 0.f};
  if (p.kind == KIND_LDM && p.coef) {
    c.c0 = p.coef[hd * 4 + 0]; c.c1 = p.coef[hd * 4 + 1]; c.c2 = p.coef[hd * 4 + 2]; c.c12 = p.coef[hd * 4 + 3];
  } else if (p.kind == KIND_OS && p.offs) {
    c.c0 = p.offs[hd];
  }
  return c;
}

// x^e for a wave-uniform exponent 0 <= e <= 15, by squaring: the exponent bits select factors (no loop, no branch).
__device__ inline float upow(float x, int e) {
  const float x2 = x * x, x4 = x2 * x2;
  float v = (e & 1) ? x : 1.0f;
  v = (e & 2) ? v * x2 : v;
  v = (e & 4) ? v * x4 : v;
  return (e & 8) ? v * (x4 * x4) : v;
}

// Whether the homogeneous families (power, signed_product) scale each raw score by sm before the polynomial, as
// the reference does (ref: tnlm/kernels/poly_attn.py:63,66): for fp16, whose range is 65504, the unscaled r^p would
// overflow where S^p does not (degree 4 at |q.k| > 16 with dk = 128). bf16 and fp32 keep fp32's range and fold sm^p
// into vf / gf instead (rounding is scale-invariant there, so both placements give the same products).
template <typename T, int POLY> __host__ __device__ constexpr bool prescaled() {
  return sizeof(T) == 2 && !std::is_same<T, __bf16>::value &&
         (POLY == POLY_POW2 || POLY == POLY_POW4 || POLY == POLY_GEN1 || POLY == POLY_SP);
}

// A(S1, S2) on raw dot products r = q.k (homogeneous kinds fold sm^p into vf unless PRE scales r by sm first).
// ref: tnlm/kernels/poly_attn.py:26-34
// KINDTEST (two-pair families only) keeps a never-taken test of the kind in the lower_degree_mix code: it changes
// nothing in the results, but without it the one-wave dK/dV kernel of that kind needs 4x more scratch spills.
template <int POLY, bool KINDTEST = false, bool PRE = false>
__device__ inline float poly_value(float r1, float r2, int kind, int deg, float sm, const Coefs& c) {
  if constexpr (PRE) {
    r1 *= sm;
    r2 *= sm;
  }
  if constexpr (POLY == POLY_POW2) {
    return r1 * r1;
  } else if constexpr (POLY == POLY_POW4) {
    const float a2 = r1 * r1;
    return a2 * a2;
  } else if constexpr (POLY == POLY_OS) {
    const float t = fmaf(r1, sm, c.c0);
    return t * t;
  } else if constexpr (POLY == POLY_GEN1) {
    return upow(r1, deg);
  } else if constexpr (POLY == POLY_SP) {
    return r1 * r2;
  } else {
    if (KINDTEST && kind == KIND_SP) return r1 * r2;
    const float s1 = r1 * sm, s2 = r2 * sm;
    return c.c0 + c.c1 * s1 + c.c2 * s2 + c.c12 * s1 * s2;
  }
}

// dS1, dS2 for a masked upstream H entry hg (gf carries the constant factors); optionally accumulates the
// head-scalar partial sums g[0..3].  ref: tnlm/kernels/poly_attn.py:123-135,189-196
template <int POLY, bool PAR, bool KINDTEST = false, bool PRE = false>
__device__ inline void poly_grad(float r1, float r2, float hg, int kind, int deg, float sm, const Coefs& c,
                                 float& d1, float& d2, float* g) {
  if constexpr (PRE) {
    r1 *= sm;
    r2 *= sm;
  }
  if constexpr (POLY == POLY_POW2) {
    d1 = hg * r1;
    d2 = 0.f;
  } else if constexpr (POLY == POLY_POW4) {
    d1 = hg * (r1 * (r1 * r1));
    d2 = 0.f;
  } else if constexpr (POLY == POLY_OS) {
    d1 = 2.0f * hg * fmaf(r1, sm, c.c0);
    d2 = 0.f;
    if constexpr (PAR) g[0] += d1;
  } else if constexpr (POLY == POLY_GEN1) {
    d1 = hg * upow(r1, deg - 1);
    d2 = 0.f;
  } else if constexpr (POLY == POLY_SP) {
    d1 = hg * r2;
    d2 = hg * r1;
  } else {
    if (KINDTEST && kind == KIND_SP) {
      d1 = hg * r2;
      d2 = hg * r1;
    } else {
      const float s1 = r1 * sm, s2 = r2 * sm;
      d1 = hg * (c.c1 + c.c12 * s2);
      d2 = hg * (c.c2 + c.c12 * s1);
      if constexpr (PAR) {
        g[0] += hg; g[1] += hg * s1; g[2] += hg * s2; g[3] += hg * s1 * s2;
      }
    }
  }
}

// Sum of squares of one operand fragment's elements in fp32.
template <typename T> __device__ inline float op_sumsq(const typename Mfma<T>::Op& a) {
  if constexpr (sizeof(T) == 2) {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < Mfma<T>::EPL; ++j) s += (float)a[j] * (float)a[j];
    return s;
  } else {
    return a * a;
  }
}

// Score-bound factor: sumsq holds, in lanes l and l ^ 32, the two halves of one row's sum of squares (the operand
// layout splits a row's contraction elements between the lane halves); the wave's largest row norm goes to *dst
// with an atomic max on the float's bits (norms are >= 0, so their bit patterns order like the values).
__device__ inline void norm_max_to(float sumsq, float* dst) {
  float x = sqrtf(sumsq + __shfl_xor(sumsq, 32, 64));
#pragma unroll
  for (int o = 16; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
  if ((threadIdx.x & 63) == 0) atomicMax((unsigned int*)dst, __float_as_uint(x));
}

// A condition every lane of the wave evaluates identically, moved to a scalar register so the compiler branches
// on it without exec masking.
__device__ inline bool uniform_bool(bool c) { return __builtin_amdgcn_readfirstlane((int)c) != 0; }

template <typename T> __device__ inline const T* head_ptr(const TDesc& d, int b, int hd) {
  return (const T*)d.p + (int64_t)b * d.sb + (int64_t)hd * d.sh;
}
template <typename T> __device__ inline T* head_ptr_w(const TDesc& d, int b, int hd) {
  return (T*)d.p + (int64_t)b * d.sb + (int64_t)hd * d.sh;
}

__host__ __device__ constexpr int cmax(int a, int b) { return a > b ? a : b; }

// ------------------------------------------------------------------------------------------------ tile configs
// NW waves per workgroup, QW / KW 32-row subtiles per wave, BN / BM rows per LDS tile, WPE = waves per SIMD the
// register allocation must allow (2 lets a second wave hide the first one's LDS latency).
template <typename T, int POLY, int DK, int DV> struct Cfg {
  static constexpr bool F32 = sizeof(T) == 4;
  static constexpr int NPAIR = two_pair_poly(POLY) ? 2 : 1;
  // Head dims above 128: four-wave workgroups at one wave per SIMD (a wave's 32 rows of operands and accumulators
  // take 128 registers per 256 columns), 32-row tiles, and the key side as separate dV and dK passes.
  static constexpr bool BIG = big_dims(DK, DV);
  // two waves per SIMD (16-bit, one pair): eight waves per workgroup, so each staged tile serves 256 rows
  static constexpr bool TWO = !F32 && NPAIR == 1 && !BIG;
  // Head dims up to 64: four-wave workgroups, two per CU (their LDS fits twice), so one workgroup's barrier waits,
  // prologue and epilogue overlap the other's MFMA work. Larger head dims: one eight-wave workgroup per CU.
  static constexpr bool SMALL = TWO && DK <= 64 && DV <= 64;
  static constexpr int NW2 = SMALL ? 4 : 8;
  // Two q/k pairs, 16-bit, head dims up to 64: the forward and dQ kernels fit 256 registers too (two waves per
  // SIMD, eight-wave workgroups). At head dim 128 the signed_product forward does so without its software pipeline
  // (two staging buffers; 16 registers spilled, still 19% faster than one wave per SIMD); lower_degree_mix's would
  // spill 315 registers and its dQ kernels would not fit either, so those stay at one wave per SIMD.
  static constexpr bool PAIR2_TWO = !F32 && NPAIR == 2 && DK <= 64 && DV <= 64;
  static constexpr bool FW2 = PAIR2_TWO || (!F32 && POLY == POLY_SP && !BIG);
  // (the two-pair forward up to head dim 64 in four-wave workgroups, two per CU with two staging buffers each: 10%
  // faster than one eight-wave workgroup; the two-pair dQ kernel measured no better that way)
  static constexpr int FW_NW = TWO ? NW2 : PAIR2_TWO ? 4 : FW2 ? 8 : 4, FW_QW = 1, FW_BN = F32 || BIG ? 32 : 64;
  static constexpr int FW_WPE = TWO || FW2 ? 2 : 1;
  static constexpr int BQ_NW = TWO ? NW2 : PAIR2_TWO ? 8 : 4, BQ_QW = 1, BQ_BN = F32 || BIG ? 32 : 64;
  static constexpr int BQ_WPE = TWO || PAIR2_TWO ? 2 : 1;
  // Key side: separate dV and dK passes at two waves per SIMD for head dim 128 (one kernel holding dK, dV, K and V
  // would need 376 registers there); up to 64 the combined kernel fits 256 registers and saves the S recompute.
  static constexpr bool KV_SPLIT = (TWO && !SMALL) || BIG;
  // (two pairs at head dim 128: 32-query tiles, whose operand reads the compiler keeps in flight fit the one-wave
  // kernel's 512 registers without spills; 64-query tiles spilled 13 registers and ran 20% slower. Two pairs up to
  // head dim 64: 32-query tiles at two waves per SIMD, two 28 KB workgroups per CU (41-76 registers spilled),
  // same-process A/B at the 100m shape: key side lower_degree_mix 0.257 -> 0.238 ms, signed_product 0.150 -> 0.149;
  // the 32-query tiles at one wave per SIMD alone were slower, 0.275 / 0.164)
  static constexpr int KV_NW = KV_SPLIT && !BIG ? NW2 : 4, KV_KW = 1;
  static constexpr int KV_BM = F32 || BIG || NPAIR == 2 ? 32 : 64;
  static constexpr int KV_WPE = SMALL || PAIR2_TWO ? 2 : 1, KV_SPLIT_WPE = BIG ? 1 : 2;
  // two pairs above head dim 128: the dK pass and the dQ kernel run once per pair (both pairs' accumulators spilled
  // ≈ 180 registers)
  static constexpr bool PAIRSPLIT = BIG && NPAIR == 2;
  static constexpr int KV_KEYS = KV_NW * KV_KW * 32;
};

// ------------------------------------------------------------------------------------------------ forward
// ref: tnlm/kernels/poly_attn.py:37-74 (_fwd)
template <typename T, int POLY, int DK, int DV, int NW, int QW, int BN, int WPE>
__global__ void __attribute__((amdgpu_flat_work_group_size(NW * 64, NW * 64), amdgpu_waves_per_eu(WPE)))
k_fwd(const KParams p) {
  // four-wave workgroups at two waves per SIMD share a CU in pairs: each gets half of the 160 KB of LDS
  constexpr int LDS_CAP = NW == 4 && WPE == 2 ? 80 * 1024 : 160 * 1024;
  typedef Mfma<T> M;
  typedef typename M::Op Op;
  constexpr int KC = M::KC, EPL = M::EPL, NT = NW * 64;
  constexpr int NPAIR = two_pair_poly(POLY) ? 2 : 1;
  constexpr bool PRE = prescaled<T, POLY>();
  constexpr int DKP = DK < 32 ? 32 : DK, DVP = DV < 32 ? 32 : DV;
  constexpr int NCK = DK / KC, NDV = DVP / 32, NKB = BN / 32, NC2 = 32 / KC;
  constexpr int BM = NW * QW * 32;
  typedef Tile<T, BN, DKP> KTile;
  typedef Tile<T, BN, DVP> VTile;
  constexpr int BUF = NPAIR * KTile::BYTES + VTile::BYTES;
  // three tile buffers for the pipelined unmasked run when they fit the 160 KB of LDS, else two (and two for the
  // two-wave signed_product forward above head dim 64, whose pipeline registers would not fit)
  constexpr bool CHUNKED = Stage<T, BN, DK, DKP, NT>::TOTAL % NT == 0 && Stage<T, BN, DV, DVP, NT>::TOTAL % NT == 0;
  constexpr int NBUF = CHUNKED && NKB >= 2 && 3 * BUF <= LDS_CAP && !(POLY == POLY_SP && (DK > 64 || DV > 64)) ? 3 : 2;
  // The block's Q rows come in, and its O rows go out, through LDS as whole coalesced rows (ROWLDS; not with
  // zero-padded head dims, whose pad columns in the tile buffers must stay zero).
  typedef Tile<T, BM, DKP> QTile;
  typedef Tile<T, BM, DVP> OTile;
  constexpr bool ROWLDS = DKP == DK && DVP == DV && NPAIR * QTile::BYTES <= LDS_CAP;
  constexpr int SMEM = cmax(NBUF * BUF, cmax(ROWLDS ? NPAIR * QTile::BYTES : 0, OTile::BYTES));
  static_assert(SMEM <= LDS_CAP, "LDS");
  __shared__ __attribute__((aligned(16))) char smem_[SMEM];
  char TNPA_LDS* smem = (char TNPA_LDS*)smem_;

  const int T_ = p.T, BH = p.B * p.H;
  const int NMB = (T_ + BM - 1) / BM;
  const int item = blockIdx.x;
  const int mb = NMB - 1 - item / BH, bh = item % BH, b = bh / p.H, hd = bh % p.H;
  const int m0 = mb * BM;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, l32 = lane & 31;

  const T* qp[2] = {head_ptr<T>(p.q1, b, hd), head_ptr<T>(p.q2, b, hd)};
  const T* kp[2] = {head_ptr<T>(p.k1, b, hd), head_ptr<T>(p.k2, b, hd)};
  const int64_t qst[2] = {p.q1.st, p.q2.st}, kst[2] = {p.k1.st, p.k2.st};
  const T* vp = head_ptr<T>(p.v, b, hd);
  const Coefs cf = load_coefs(p, hd);
  const int* dst = p.dstart + (int64_t)b * T_;
  const float* rsc = p.rscale + (int64_t)b * T_;

  if constexpr (DKP != DK || DVP != DV) {
    for (int i = threadIdx.x; i < SMEM / 16; i += NT) ((u32x4 TNPA_LDS*)smem)[i] = u32x4{0u, 0u, 0u, 0u};
    __syncthreads();
  }

  const int qw0 = m0 + wave * QW * 32;
  Op qf[NPAIR][QW][NCK];
  int dsq[QW], qa[QW], ql[QW], dsa[QW], dsl[QW];
  float scq[QW];
#pragma unroll
  for (int s = 0; s < QW; ++s) {
    qa[s] = qw0 + 32 * s;
    ql[s] = min(qa[s] + 31, T_ - 1);
    dsa[s] = qa[s] < T_ ? dst[qa[s]] : INT_MAX;
    dsl[s] = qa[s] < T_ ? dst[ql[s]] : INT_MAX;
    const int q = qa[s] + l32;
    const bool valid = q < T_;
    dsq[s] = valid ? dst[q] : INT_MAX;
    scq[s] = valid ? rsc[q] : 0.f;
    if constexpr (!ROWLDS) {
#pragma unroll
      for (int pr = 0; pr < NPAIR; ++pr)
#pragma unroll
        for (int c = 0; c < NCK; ++c) qf[pr][s][c] = valid ? load_op<T>(qp[pr] + (int64_t)q * qst[pr], c, h) : M::zero();
    }
  }
  // the first K/V tile is loaded together with the Q rows (independent latencies); it is written to LDS once the
  // Q fragments have been taken out of the same space
  const int lo = (dst[m0] / BN) * BN;
  const int hi = min(m0 + BM, T_);
  Stage<T, BN, DK, DKP, NT> sk[NPAIR];
  Stage<T, BN, DV, DVP, NT> sv;
#pragma unroll
  for (int pr = 0; pr < NPAIR; ++pr) sk[pr].load(kp[pr], kst[pr], lo, T_ - lo);
  sv.load(vp, p.v.st, lo, T_ - lo);
  if constexpr (ROWLDS) {
    Stage<T, BM, DK, DKP, NT> qs[NPAIR];
#pragma unroll
    for (int pr = 0; pr < NPAIR; ++pr) qs[pr].load(qp[pr], qst[pr], m0, T_ - m0);
#pragma unroll
    for (int pr = 0; pr < NPAIR; ++pr) qs[pr].store(smem + pr * QTile::BYTES);
    __syncthreads();
#pragma unroll
    for (int pr = 0; pr < NPAIR; ++pr)
#pragma unroll
      for (int s = 0; s < QW; ++s)
#pragma unroll
        for (int c = 0; c < NCK; ++c)
          qf[pr][s][c] = read_row<T, QTile>(smem + pr * QTile::BYTES, 32 * (wave * QW + s), l32, c, h);
    __syncthreads();
  }

  // score-bound factor max |q|: the wave's rows are in its Q fragments
  if (p.norms != nullptr) {
#pragma unroll
    for (int pr = 0; pr < NPAIR; ++pr) {
      float ss = 0.f;
#pragma unroll
      for (int s = 0; s < QW; ++s)
#pragma unroll
        for (int c = 0; c < NCK; ++c) ss += op_sumsq<T>(qf[pr][s][c]);
      norm_max_to(ss, p.norms + (pr * 2) * p.H + hd);
    }
  }

  f32x16 oacc[QW][NDV];
#pragma unroll
  for (int s = 0; s < QW; ++s)
#pragma unroll
    for (int d = 0; d < NDV; ++d) oacc[s][d] = zero16();

#pragma unroll
  for (int pr = 0; pr < NPAIR; ++pr) sk[pr].store(smem + pr * KTile::BYTES);
  sv.store(smem + NPAIR * KTile::BYTES);
  __syncthreads();

  int cur = 0;
  auto sub = [&](const char TNPA_LDS* base, const int n0, const int kb, const uint32_t am, const uint32_t fm, auto all_c, auto full_c) {
    constexpr bool ALL = decltype(all_c)::value, FULL = decltype(full_c)::value;
    const int key0 = n0 + 32 * kb;
    f32x16 sacc[NPAIR][QW];
#pragma unroll
    for (int pr = 0; pr < NPAIR; ++pr)
#pragma unroll
      for (int s = 0; s < QW; ++s) sacc[pr][s] = zero16();
    // score-bound factor max |k|: every key row is the A operand of exactly one diagonal sub-block (key0 == qa[0])
    const bool knorm = p.norms != nullptr && key0 == qa[0];
    float kss[NPAIR];
#pragma unroll
    for (int pr = 0; pr < NPAIR; ++pr) kss[pr] = 0.f;
#pragma unroll
    for (int c = 0; c < NCK; ++c)
#pragma unroll
      for (int pr = 0; pr < NPAIR; ++pr) {
        const Op a = read_row<T, KTile>(base + pr * KTile::BYTES, 32 * kb, kappa<T>(l32), c, h);
        if (knorm) kss[pr] += op_sumsq<T>(a);
#pragma unroll
        for (int s = 0; s < QW; ++s)
          if (ALL || ((am >> s) & 1u)) sacc[pr][s] = M::mma(a, qf[pr][s][c], sacc[pr][s]);
      }
    if (knorm) {
#pragma unroll
      for (int pr = 0; pr < NPAIR; ++pr) norm_max_to(kss[pr], p.norms + (pr * 2 + 1) * p.H + hd);
    }
    Op pop[QW][NC2];
#pragma unroll
    for (int s = 0; s < QW; ++s) {
      if (!(ALL || ((am >> s) & 1u))) continue;
      float pv[16];
      if (FULL || ((fm >> s) & 1u)) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          pv[r] = poly_value<POLY, false, PRE>(sacc[0][s][r], sacc[NPAIR - 1][s][r], p.kind, p.deg, p.sm, cf);
      } else {
        const int q = qa[s] + l32;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = key0 + key_off<T>(r, h);
          const float val = poly_value<POLY, false, PRE>(sacc[0][s][r], sacc[NPAIR - 1][s][r], p.kind, p.deg, p.sm, cf);
          pv[r] = (key > q || key < dsq[s]) ? 0.f : val;
        }
      }
#pragma unroll
      for (int c2 = 0; c2 < NC2; ++c2) pop[s][c2] = M::cvt(pv + c2 * EPL);
    }
#pragma unroll
    for (int d = 0; d < NDV; ++d)
#pragma unroll
      for (int c2 = 0; c2 < NC2; ++c2) {
        const Op a = read_col<T, VTile>(base + NPAIR * KTile::BYTES, 32 * kb + c2 * KC, 32 * d, lane);
#pragma unroll
        for (int s = 0; s < QW; ++s)
          if (ALL || ((am >> s) & 1u)) oacc[s][d] = M::mma(a, pop[s][c2], oacc[s][d]);
      }
  };

  typedef Stage<T, BN, DK, DKP, NT> KStage;
  typedef Stage<T, BN, DV, DVP, NT> VStage;
  auto next_buf = [](const int c) { return c + 1 == NBUF ? 0 : c + 1; };
  auto k_rows = [&](Op (&ka)[NPAIR][NCK], const char TNPA_LDS* base, const int kb) {
#pragma unroll
    for (int pr = 0; pr < NPAIR; ++pr)
#pragma unroll
      for (int c = 0; c < NCK; ++c) ka[pr][c] = read_row<T, KTile>(base + pr * KTile::BYTES, 32 * kb, kappa<T>(l32), c, h);
  };
  auto v_cols = [&](Op (&vt)[NDV][NC2], const char TNPA_LDS* base, const int kb) {
#pragma unroll
    for (int d = 0; d < NDV; ++d)
#pragma unroll
      for (int c2 = 0; c2 < NC2; ++c2)
        vt[d][c2] = read_col<T, VTile>(base + NPAIR * KTile::BYTES, 32 * kb + c2 * KC, 32 * d, lane);
  };
  auto s_mma = [&](f32x16 (&sacc)[NPAIR][QW], const Op (&ka)[NPAIR][NCK]) {
#pragma unroll
    for (int pr = 0; pr < NPAIR; ++pr)
#pragma unroll
      for (int s = 0; s < QW; ++s) sacc[pr][s] = zero16();
#pragma unroll
    for (int c = 0; c < NCK; ++c)
#pragma unroll
      for (int pr = 0; pr < NPAIR; ++pr)
#pragma unroll
        for (int s = 0; s < QW; ++s) sacc[pr][s] = M::mma(ka[pr][c], qf[pr][s][c], sacc[pr][s]);
  };
  auto power = [&](Op (&pop)[QW][NC2], const f32x16 (&sacc)[NPAIR][QW]) {
#pragma unroll
    for (int s = 0; s < QW; ++s) {
      float pv[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) pv[r] = poly_value<POLY, false, PRE>(sacc[0][s][r], sacc[NPAIR - 1][s][r], p.kind, p.deg, p.sm, cf);
#pragma unroll
      for (int c2 = 0; c2 < NC2; ++c2) pop[s][c2] = M::cvt(pv + c2 * EPL);
    }
  };
  // c2-major: consecutive MFMAs go to different accumulators
  auto pv_mma = [&](const Op (&vt)[NDV][NC2], const Op (&pop)[QW][NC2]) {
#pragma unroll
    for (int c2 = 0; c2 < NC2; ++c2)
#pragma unroll
      for (int d = 0; d < NDV; ++d)
#pragma unroll
        for (int s = 0; s < QW; ++s) oacc[s][d] = M::mma(vt[d][c2], pop[s][c2], oacc[s][d]);
  };
  // Buffer resource over rows n1.. of one head: rows at or past T_ read as zero.
  auto rows_rsrc = [&](const T* base, const int64_t st, const int n1, const int D) {
    const int64_t rem = n1 < T_ ? ((int64_t)(T_ - 1 - n1) * st + D) * (int64_t)sizeof(T) : 0;
    const int nrec = (int)(rem < 0x7fffffff ? rem : 0x7fffffff);
    return __builtin_amdgcn_make_buffer_rsrc((void*)(base + (int64_t)n1 * st), (short)0, nrec, 0x00020000);
  };
  uint32_t kvo[NPAIR][KStage::PER], vvo[VStage::PER];
#pragma unroll
  for (int pr = 0; pr < NPAIR; ++pr)
#pragma unroll
    for (int i = 0; i < KStage::PER; ++i) kvo[pr][i] = KStage::chunk_off(i, kst[pr]);
#pragma unroll
  for (int i = 0; i < VStage::PER; ++i) vvo[i] = VStage::chunk_off(i, p.v.st);
  // part 1: the K rows, part 2: the V rows (issued in different phases so the memory pipe drains in between)
  auto stage_load_buf = [&](const int n1, const int part) {
    if constexpr (!CHUNKED) return;
    if (part & 1) {
#pragma unroll
      for (int pr = 0; pr < NPAIR; ++pr) {
        const auto rs = rows_rsrc(kp[pr], kst[pr], n1, DK);
#pragma unroll
        for (int i = 0; i < KStage::PER; ++i) sk[pr].load_buf(i, rs, kvo[pr][i]);
      }
    }
    if (part & 2) {
      const auto rs = rows_rsrc(vp, p.v.st, n1, DV);
#pragma unroll
      for (int i = 0; i < VStage::PER; ++i) sv.load_buf(i, rs, vvo[i]);
    }
  };
  auto stage_store_raw = [&](char TNPA_LDS* dstb, const int part) {
    if (part & 1) {
#pragma unroll
      for (int pr = 0; pr < NPAIR; ++pr)
#pragma unroll
        for (int i = 0; i < KStage::PER; ++i) sk[pr].store_raw(i, dstb + pr * KTile::BYTES);
    }
    if (part & 2) {
#pragma unroll
      for (int i = 0; i < VStage::PER; ++i) sv.store_raw(i, dstb + NPAIR * KTile::BYTES);
    }
  };
  // Whole-tile staging of rows n1.. (buffer loads when the tile splits evenly over the threads, else the guarded
  // per-chunk copy)
  auto stage_load = [&](const int n1) {
    if constexpr (CHUNKED) {
      stage_load_buf(n1, 3);
    } else {
#pragma unroll
      for (int pr = 0; pr < NPAIR; ++pr) sk[pr].load(kp[pr], kst[pr], n1, T_ - n1);
      sv.load(vp, p.v.st, n1, T_ - n1);
    }
  };
  auto stage_store = [&](char TNPA_LDS* dstb) {
    if constexpr (CHUNKED) {
      stage_store_raw(dstb, 3);
    } else {
#pragma unroll
      for (int pr = 0; pr < NPAIR; ++pr) sk[pr].store(dstb + pr * KTile::BYTES);
      sv.store(dstb + NPAIR * KTile::BYTES);
    }
  };

  // Run of unmasked tiles jb..je-1 (no mask, no sub-block test).
  // Three buffers: software pipeline over the run's 32-key sub-blocks g. Phase A(g): the V^T(g) reads and the
  // S(g+1) MFMA chain, back to back; phase B(g): O += V^T(g) P(g) MFMAs, with the power of S(g+1) and the K-row
  // reads of g+2 between them. Every operand is read a phase ahead and the VALU work sits between independent
  // MFMAs, so one wave keeps the matrix pipe fed on its own. Tile j+1 is published by the barrier at the start of
  // B(NKB-2) of tile j, before the first read of its rows (tiles j, j+1 and j+2 in flight). Its staging is spread
  // so the memory pipe and LDS drain between parts: K rows loaded in B(NKB-2) of tile j-1 (after that barrier) and
  // written in B(NKB-1), V rows loaded in A(NKB-1) and written in A(NKB-2) of tile j. Two buffers: one tile per
  // step, loads before and stores after the compute.
  auto fast_run = [&](const int jb, const int je) {
    if constexpr (NBUF == 3) {
      Op ka[NPAIR][NCK], vt[NDV][NC2], pop[QW][NC2], pn[QW][NC2];
      f32x16 sn[NPAIR][QW];
      stage_load_buf(lo + (jb + 1) * BN, 3);  // the step before the run staged only tile jb
      k_rows(ka, smem + cur * BUF, 0);
      s_mma(sn, ka);
      k_rows(ka, smem + cur * BUF, 1);
      power(pop, sn);
      stage_store_raw(smem + next_buf(cur) * BUF, 1);  // its V rows follow in the first tile's A(NKB-2)
      // one tile; LAST (the run's final tile) drains the pipeline instead of starting the next tile
      auto tile = [&](const int j, auto last_c) {
        constexpr bool LAST = decltype(last_c)::value;
        const int nc = next_buf(cur);
        const char TNPA_LDS* base = smem + cur * BUF;
        char TNPA_LDS* b1 = smem + nc * BUF;
        char TNPA_LDS* b2 = smem + next_buf(nc) * BUF;
        const int n1 = lo + (j + 1) * BN;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
          const bool more_s = kb + 1 < NKB || !LAST;
          v_cols(vt, base, kb);
          if (kb == NKB - 2) stage_store_raw(b1, 2);
          if (kb == NKB - 1 && !LAST) stage_load_buf(n1 + BN, 2);
          if (more_s) s_mma(sn, ka);
          __builtin_amdgcn_sched_barrier(0);
          if (kb == NKB - 2) {
            __syncthreads();
            if (!LAST) stage_load_buf(n1 + BN, 1);
          }
          if (kb + 2 < NKB) k_rows(ka, base, kb + 2);
          else if (!LAST) k_rows(ka, b1, kb + 2 - NKB);
          pv_mma(vt, pop);
          if (more_s) power(pn, sn);
          if (kb == NKB - 1 && !LAST) stage_store_raw(b2, 1);
          // K-row reads first (a whole phase ahead of their use), then one MFMA per few VALU of the power
          if (kb + 2 < NKB || !LAST) __builtin_amdgcn_sched_group_barrier(0x100, NPAIR * NCK, 0);
#pragma unroll
          for (int i = 0; i < NDV * NC2 * QW; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int s = 0; s < QW; ++s)
#pragma unroll
            for (int c2 = 0; c2 < NC2; ++c2) pop[s][c2] = pn[s][c2];
        }
        cur = nc;
      };
      for (int j = jb; j + 1 < je; ++j) tile(j, std::false_type{});
      tile(je - 1, std::true_type{});
    } else {
      for (int j = jb; j < je; ++j) {
        const int n1 = lo + (j + 1) * BN;
        const bool more = n1 < hi;
        const char TNPA_LDS* base = smem + cur * BUF;
        if (more) stage_load(n1);
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
          Op ka[NPAIR][NCK], vt[NDV][NC2], pop[QW][NC2];
          f32x16 sacc[NPAIR][QW];
          k_rows(ka, base, kb);
          v_cols(vt, base, kb);
          s_mma(sacc, ka);
          power(pop, sacc);
          pv_mma(vt, pop);
        }
        if (more) stage_store(smem + next_buf(cur) * BUF);
        __syncthreads();
        cur = next_buf(cur);
      }
    }
  };

  // One masked tile step: prefetch the next K/V tile into registers, compute on the current LDS buffer, publish
  // the prefetched tile into the next buffer, one barrier.
  auto step = [&](const int n0) {
    const int n1 = n0 + BN;
    const bool more = n1 < hi;
    if (more) stage_load(n1);
    const char TNPA_LDS* base = smem + cur * BUF;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const int key0 = n0 + 32 * kb;
      uint32_t am = 0, fm = 0;
#pragma unroll
      for (int s = 0; s < QW; ++s) {
        if (qa[s] < T_ && key0 <= ql[s] && key0 + 31 >= dsa[s]) am |= 1u << s;
        if (key0 + 31 <= qa[s] && dsl[s] <= key0) fm |= 1u << s;
      }
      am = __builtin_amdgcn_readfirstlane(am);
      fm = __builtin_amdgcn_readfirstlane(fm);
      if (am == 0) continue;
      sub(base, n0, kb, am, fm, std::false_type{}, std::false_type{});
    }
    if (more) stage_store(smem + next_buf(cur) * BUF);
    __syncthreads();
    cur = next_buf(cur);
  };
  // Tiles lo, lo+BN, ... < hi, split per wave into three contiguous runs: before the document start of the
  // wave's last query (generic), fully visible from every query of the wave (fast: no mask, no per-subtile test),
  // and the diagonal (generic). Every wave steps through all tiles, so the barrier count matches across waves.
  const int ntile = (hi - lo + BN - 1) / BN;
  int j0 = 0, j1 = 0;
  if (qa[0] < T_) {
    const int dl = dst[min(qw0 + 32 * QW - 1, T_ - 1)];
    j0 = min(ntile, max(0, (dl - lo + BN - 1) / BN));
    j1 = max(j0, min(ntile, (qa[0] + 1 - lo) / BN));
  }
  j0 = __builtin_amdgcn_readfirstlane(j0);
  j1 = __builtin_amdgcn_readfirstlane(j1);
  int j = 0;
  for (; j < j0; ++j) step(lo + j * BN);
  if (j < j1) fast_run(j, j1);
  for (j = j1; j < ntile; ++j) step(lo + j * BN);

  // O rows: scaled in registers, gathered in LDS, written as whole rows
  T* op = head_ptr_w<T>(p.o, b, hd);
  __syncthreads();  // every wave is done with the tile buffers
#pragma unroll
  for (int s = 0; s < QW; ++s) acc_rows_to_lds<T, OTile, NDV>(smem, 32 * (wave * QW + s), l32, h, oacc[s], scq[s] * p.vf, DV);
  __syncthreads();
  Stage<T, BM, DV, DVP, NT> os;
  os.copy_out(smem, op, p.o.st, m0, T_ - m0);
}

// ------------------------------------------------------------------------------------------------ dQ
// ref: tnlm/kernels/poly_attn.py:151-202 (_bwd_q)
// QSEL: -1 accumulates dQ of every q/k pair; 0 or 1 only that pair's (two-pair kinds above head dim 128, one launch
// per pair: S1, S2 and dP are recomputed in each, and half the accumulators fit one wave's registers)
template <typename T, int POLY, int DK, int DV, int NW, int QW, int BN, int WPE, int QSEL = -1>
__global__ void __attribute__((amdgpu_flat_work_group_size(NW * 64, NW * 64), amdgpu_waves_per_eu(WPE)))
k_bwd_q(const KParams p) {
  // four-wave workgroups at two waves per SIMD share a CU in pairs: each gets half of the 160 KB of LDS
  constexpr int LDS_CAP = NW == 4 && WPE == 2 ? 80 * 1024 : 160 * 1024;
  typedef Mfma<T> M;
  typedef typename M::Op Op;
  constexpr int KC = M::KC, EPL = M::EPL, NT = NW * 64;
  constexpr int NPAIR = two_pair_poly(POLY) ? 2 : 1;
  constexpr bool PRE = prescaled<T, POLY>();
  constexpr int DKP = DK < 32 ? 32 : DK, DVP = DV < 32 ? 32 : DV;
  constexpr int NCK = DK / KC, NCV = DV / KC, NDK = DKP / 32, NKB = BN / 32, NC2 = 32 / KC;
  constexpr int BM = NW * QW * 32;
  typedef Tile<T, BN, DKP> KTile;
  typedef Tile<T, BN, DVP> VTile;
  constexpr int BUF = NPAIR * KTile::BYTES + VTile::BYTES;
  typedef PartStager<T, BN, DK, DKP, DV, DVP, NT, NPAIR> Stager;
  // three tile buffers (each tile staged over two steps, its parts in different sub-blocks) when they fit the
  // 160 KB of LDS and the tile splits evenly over the threads, else two
  constexpr int NBUF = Stager::OK && NKB >= 2 && 3 * BUF <= LDS_CAP ? 3 : 2;
  // The block's Q and dO rows come in, and its dQ rows go out, through LDS as whole coalesced rows (ROWLDS; not
  // with zero-padded head dims, whose pad columns in the tile buffers must stay zero).
  typedef Tile<T, BM, DKP> QTile;
  typedef Tile<T, BM, DVP> DOTile;
  constexpr bool ROWLDS = DKP == DK && DVP == DV && NPAIR * QTile::BYTES + DOTile::BYTES <= LDS_CAP;
  constexpr int SMEM = cmax(NBUF * BUF, cmax(ROWLDS ? NPAIR * QTile::BYTES + DOTile::BYTES : 0, QTile::BYTES));
  static_assert(SMEM <= LDS_CAP, "LDS");
  __shared__ __attribute__((aligned(16))) char smem_[SMEM];
  char TNPA_LDS* smem = (char TNPA_LDS*)smem_;

  const int T_ = p.T, BH = p.B * p.H;
  const int NMB = (T_ + BM - 1) / BM;
  const int item = blockIdx.x;
  const int mb = NMB - 1 - item / BH, bh = item % BH, b = bh / p.H, hd = bh % p.H;
  const int m0 = mb * BM;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, l32 = lane & 31;

  const T* qp[2] = {head_ptr<T>(p.q1, b, hd), head_ptr<T>(p.q2, b, hd)};
  const T* kp[2] = {head_ptr<T>(p.k1, b, hd), head_ptr<T>(p.k2, b, hd)};
  const int64_t qst[2] = {p.q1.st, p.q2.st}, kst[2] = {p.k1.st, p.k2.st};
  const T* vp = head_ptr<T>(p.v, b, hd);
  const T* dop = head_ptr<T>(p.dout, b, hd);
  const Coefs cf = load_coefs(p, hd);
  const int* dst = p.dstart + (int64_t)b * T_;
  const float* rsc = p.rscale + (int64_t)b * T_;

  if constexpr (DKP != DK || DVP != DV) {
    for (int i = threadIdx.x; i < SMEM / 16; i += NT) ((u32x4 TNPA_LDS*)smem)[i] = u32x4{0u, 0u, 0u, 0u};
    __syncthreads();
  }

  const int qw0 = m0 + wave * QW * 32;
  Op qf[NPAIR][QW][NCK];
  Op dof[QW][NCV];
  int dsq[QW], qa[QW], ql[QW], dsa[QW], dsl[QW];
  float scq[QW];
#pragma unroll
  for (int s = 0; s < QW; ++s) {
    qa[s] = qw0 + 32 * s;
    ql[s] = min(qa[s] + 31, T_ - 1);
    dsa[s] = qa[s] < T_ ? dst[qa[s]] : INT_MAX;
    dsl[s] = qa[s] < T_ ? dst[ql[s]] : INT_MAX;
    const int q = qa[s] + l32;
    const bool valid = q < T_;
    dsq[s] = valid ? dst[q] : INT_MAX;
    scq[s] = valid ? rsc[q] : 0.f;
    if constexpr (!ROWLDS) {
#pragma unroll
      for (int pr = 0; pr < NPAIR; ++pr)
#pragma unroll
        for (int c = 0; c < NCK; ++c) qf[pr][s][c] = valid ? load_op<T>(qp[pr] + (int64_t)q * qst[pr], c, h) : M::zero();
#pragma unroll
      for (int c = 0; c < NCV; ++c) dof[s][c] = valid ? load_op<T>(dop + (int64_t)q * p.dout.st, c, h) : M::zero();
    }
  }
  if constexpr (ROWLDS) {
    Stage<T, BM, DK, DKP, NT> qs[NPAIR];
    Stage<T, BM, DV, DVP, NT> ds;
#pragma unroll
    for (int pr = 0; pr < NPAIR; ++pr) qs[pr].load(qp[pr], qst[pr], m0, T_ - m0);
    ds.load(dop, p.dout.st, m0, T_ - m0);
#pragma unroll
    for (int pr = 0; pr < NPAIR; ++pr) qs[pr].store(smem + pr * QTile::BYTES);
    ds.store(smem + NPAIR * QTile::BYTES);
    __syncthreads();
#pragma unroll
    for (int s = 0; s < QW; ++s) {
#pragma unroll
      for (int pr = 0; pr < NPAIR; ++pr)
#pragma unroll
        for (int c = 0; c < NCK; ++c)
          qf[pr][s][c] = read_row<T, QTile>(smem + pr * QTile::BYTES, 32 * (wave * QW + s), l32, c, h);
#pragma unroll
      for (int c = 0; c < NCV; ++c)
        dof[s][c] = read_row<T, DOTile>(smem + NPAIR * QTile::BYTES, 32 * (wave * QW + s), l32, c, h);
    }
    __syncthreads();
  }

  // dQ accumulator sets: one per pair, or pair QSEL's alone (accumulator j holds pair qpair(j))
  constexpr int NQA = QSEL < 0 ? NPAIR : 1;
  auto qpair = [](int j) { return QSEL < 0 ? j : QSEL; };
  f32x16 dq[NQA][QW][NDK];
#pragma unroll
  for (int j = 0; j < NQA; ++j)
#pragma unroll
    for (int s = 0; s < QW; ++s)
#pragma unroll
      for (int d = 0; d < NDK; ++d) dq[j][s][d] = zero16();

  const int lo = (dst[m0] / BN) * BN;
  const int hi = min(m0 + BM, T_);
  Stage<T, BN, DK, DKP, NT> sk[NPAIR];
  Stage<T, BN, DV, DVP, NT> sv;
  Stager stg;
  if constexpr (NBUF == 3) {
    stg.init(kp, kst, vp, p.v.st, T_);
    stg.load(3, lo);
    stg.store(3, smem);
    stg.load(3, lo + BN);
  } else {
#pragma unroll
    for (int pr = 0; pr < NPAIR; ++pr) sk[pr].load(kp[pr], kst[pr], lo, T_ - lo);
    sv.load(vp, p.v.st, lo, T_ - lo);
#pragma unroll
    for (int pr = 0; pr < NPAIR; ++pr) sk[pr].store(smem + pr * KTile::BYTES);
    sv.store(smem + NPAIR * KTile::BYTES);
  }
  __syncthreads();
  auto next_buf = [](const int c) { return c + 1 == NBUF ? 0 : c + 1; };

  int cur = 0;
  // mid: work placed between the sub-block's S/dP MFMA chains and its VALU (the spread tile staging)
  auto sub = [&](const char TNPA_LDS* base, const int n0, const int kb, const uint32_t am, const uint32_t fm, auto all_c, auto full_c,
                 auto&& mid) {
    constexpr bool ALL = decltype(all_c)::value, FULL = decltype(full_c)::value;
    const int key0 = n0 + 32 * kb;
    f32x16 sacc[NPAIR][QW], pacc[QW];
#pragma unroll
    for (int s = 0; s < QW; ++s) {
      pacc[s] = zero16();
#pragma unroll
      for (int pr = 0; pr < NPAIR; ++pr) sacc[pr][s] = zero16();
    }
#pragma unroll
    for (int c = 0; c < NCK; ++c)
#pragma unroll
      for (int pr = 0; pr < NPAIR; ++pr) {
        const Op a = read_row<T, KTile>(base + pr * KTile::BYTES, 32 * kb, kappa<T>(l32), c, h);
#pragma unroll
        for (int s = 0; s < QW; ++s)
          if (ALL || ((am >> s) & 1u)) sacc[pr][s] = M::mma(a, qf[pr][s][c], sacc[pr][s]);
      }
#pragma unroll
    for (int c = 0; c < NCV; ++c) {
      const Op a = read_row<T, VTile>(base + NPAIR * KTile::BYTES, 32 * kb, kappa<T>(l32), c, h);
#pragma unroll
      for (int s = 0; s < QW; ++s)
        if (ALL || ((am >> s) & 1u)) pacc[s] = M::mma(a, dof[s][c], pacc[s]);
    }
    mid();
    // H = row_scale * dO V^T before dS is formed and rounded, as ref: tnlm/kernels/poly_attn.py:188 does (keeps fp16
    // dS in range where the unscaled H times S would not be)
    Op dso[NQA][QW][NC2];
#pragma unroll
    for (int s = 0; s < QW; ++s) {
      if (!(ALL || ((am >> s) & 1u))) continue;
      float d1[16], d2[16];
      if (FULL || ((fm >> s) & 1u)) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          poly_grad<POLY, false, false, PRE>(sacc[0][s][r], sacc[NPAIR - 1][s][r], pacc[s][r] * scq[s], p.kind, p.deg, p.sm, cf, d1[r],
                                 d2[r], nullptr);
      } else {
        const int q = qa[s] + l32;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = key0 + key_off<T>(r, h);
          const float hg = (key > q || key < dsq[s]) ? 0.f : pacc[s][r] * scq[s];
          poly_grad<POLY, false, false, PRE>(sacc[0][s][r], sacc[NPAIR - 1][s][r], hg, p.kind, p.deg, p.sm, cf, d1[r], d2[r],
                                 nullptr);
        }
      }
#pragma unroll
      for (int c2 = 0; c2 < NC2; ++c2) {
        if constexpr (QSEL < 0) {
          dso[0][s][c2] = M::cvt(d1 + c2 * EPL);
          if constexpr (NPAIR == 2) dso[NPAIR - 1][s][c2] = M::cvt(d2 + c2 * EPL);
        } else {
          dso[0][s][c2] = M::cvt((QSEL == 1 ? d2 : d1) + c2 * EPL);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < NQA; ++j)
#pragma unroll
      for (int d = 0; d < NDK; ++d)
#pragma unroll
        for (int c2 = 0; c2 < NC2; ++c2) {
          const Op a = read_col<T, KTile>(base + qpair(j) * KTile::BYTES, 32 * kb + c2 * KC, 32 * d, lane);
#pragma unroll
          for (int s = 0; s < QW; ++s)
            if (ALL || ((am >> s) & 1u)) dq[j][s][d] = M::mma(a, dso[j][s][c2], dq[j][s][d]);
        }
  };

  // One tile step: prefetch the next K/V tile into registers, compute on the current LDS buffer, publish the
  // prefetched tile into the other buffer, one barrier.
  auto step = [&](const int n0, auto fast_c) {
    constexpr bool FAST = decltype(fast_c)::value;
    const bool more = NBUF == 2 && n0 + BN < hi;
    // three buffers: tile j+1 (in registers since the previous step) is written to its buffer and tile j+2 loaded
    // in its place, one 16-byte chunk per thread at each of 2 * NKB points (the middle and the end of every
    // sub-block), so that the loads of all waves reach the memory pipe spread over the step
    char TNPA_LDS* b1 = smem + next_buf(cur) * BUF;
    auto stage_at = [&](const int point) {
      if constexpr (NBUF == 3) {
#pragma unroll
        for (int q = 0; q < Stager::NPARTS; ++q)
          if (q % (2 * NKB) == point) {
            stg.store_part(q, b1);
            stg.load_part(q, n0 + 2 * BN);
          }
      }
    };
    auto mid_for = [&](const int kb) { return [&, kb]() { stage_at(2 * kb); }; };
    if (more) {
#pragma unroll
      for (int pr = 0; pr < NPAIR; ++pr) sk[pr].load(kp[pr], kst[pr], n0 + BN, T_ - n0 - BN);
      sv.load(vp, p.v.st, n0 + BN, T_ - n0 - BN);
    }
    const char TNPA_LDS* base = smem + cur * BUF;
    if constexpr (FAST) {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        sub(base, n0, kb, 0u, 0u, std::true_type{}, std::true_type{}, mid_for(kb));
        stage_at(2 * kb + 1);
      }
    } else {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const int key0 = n0 + 32 * kb;
        uint32_t am = 0, fm = 0;
#pragma unroll
        for (int s = 0; s < QW; ++s) {
          if (qa[s] < T_ && key0 <= ql[s] && key0 + 31 >= dsa[s]) am |= 1u << s;
          if (key0 + 31 <= qa[s] && dsl[s] <= key0) fm |= 1u << s;
        }
        am = __builtin_amdgcn_readfirstlane(am);
        fm = __builtin_amdgcn_readfirstlane(fm);
        stage_at(2 * kb);  // outside the skip test: one code path, so no wait on the loads it issues
        stage_at(2 * kb + 1);
        if (am == 0) continue;
        sub(base, n0, kb, am, fm, std::false_type{}, std::false_type{}, [] {});
      }
    }
    if (more) {
#pragma unroll
      for (int pr = 0; pr < NPAIR; ++pr) sk[pr].store(b1 + pr * KTile::BYTES);
      sv.store(b1 + NPAIR * KTile::BYTES);
    }
    __syncthreads();
    cur = next_buf(cur);
  };
  // Tiles lo, lo+BN, ... < hi, split per wave into three contiguous runs: before the document start of the
  // wave's last query (generic), fully visible from every query of the wave (fast: no mask, no per-subtile test),
  // and the diagonal (generic). Every wave steps through all tiles, so the barrier count matches across waves.
  const int ntile = (hi - lo + BN - 1) / BN;
  int j0 = 0, j1 = 0;
  if (qa[0] < T_) {
    const int dl = dst[min(qw0 + 32 * QW - 1, T_ - 1)];
    j0 = min(ntile, max(0, (dl - lo + BN - 1) / BN));
    j1 = max(j0, min(ntile, (qa[0] + 1 - lo) / BN));
  }
  j0 = __builtin_amdgcn_readfirstlane(j0);
  j1 = __builtin_amdgcn_readfirstlane(j1);
  int j = 0;
  for (; j < j0; ++j) step(lo + j * BN, std::false_type{});
  for (; j < j1; ++j) step(lo + j * BN, std::true_type{});
  for (; j < ntile; ++j) step(lo + j * BN, std::false_type{});

  // dQ rows: scaled by the chain-rule factor in registers, gathered in LDS, written as whole rows
  const TDesc* outs[2] = {&p.dq1, &p.dq2};
#pragma unroll
  for (int j = 0; j < NQA; ++j) {
    const int pr = qpair(j);
    __syncthreads();  // every wave is done with the tile buffers (or with the previous pair's rows)
#pragma unroll
    for (int s = 0; s < QW; ++s)
      acc_rows_to_lds<T, QTile, NDK>(smem, 32 * (wave * QW + s), l32, h, dq[j][s], p.gf, DK);
    __syncthreads();
    Stage<T, BM, DK, DKP, NT> os;
    if (p.rcos != nullptr)
      os.copy_out_rope(smem, head_ptr_w<T>(*outs[pr], b, hd), outs[pr]->st, m0, T_ - m0, p.rcos, p.rsin,
                       (int64_t)b * T_ + m0);
    else
      os.copy_out(smem, head_ptr_w<T>(*outs[pr], b, hd), outs[pr]->st, m0, T_ - m0);
  }
}

// ------------------------------------------------------------------------------------------------ dK / dV
// ref: tnlm/kernels/poly_attn.py:77-148 (_bwd_kv)
// MODE: KV_BOTH computes dK and dV in one pass (one wave per SIMD: dK, dV, K and V all stay in registers);
// KV_DV and KV_DK split them into two passes that each fit two waves per SIMD (the S = Q K^T product is computed
// in both passes).
// KV_DK1 / KV_DK2: the dK pass of a two-pair kind accumulating dK1 or dK2 only (above head dim 128, one launch per
// pair: S1, S2 and dP are recomputed in each, and half the accumulators fit one wave's registers; the first writes
// the dcoef/db partials).
enum { KV_BOTH = 0, KV_DV = 1, KV_DK = 2, KV_DK1 = 3, KV_DK2 = 4 };
template <typename T, int POLY, int DK, int DV, int NW, int KW, int BMQ, int WPE, int MODE>
__global__ void __attribute__((amdgpu_flat_work_group_size(NW * 64, NW * 64), amdgpu_waves_per_eu(WPE)))
k_bwd_kv(const KParams p) {
  typedef Mfma<T> M;
  typedef typename M::Op Op;
  constexpr int KC = M::KC, EPL = M::EPL, NT = NW * 64;
  constexpr int NPAIR = two_pair_poly(POLY) ? 2 : 1;
  constexpr bool PRE = prescaled<T, POLY>();
  constexpr bool PAR = (POLY == POLY_OS || POLY == POLY_GEN2) && MODE != KV_DV && MODE != KV_DK2;  // head scalars
  constexpr bool WANT_DV = MODE == KV_BOTH || MODE == KV_DV, WANT_DK = MODE != KV_DV;
  // dK accumulator sets: one per pair, or one pair's alone (accumulator j holds pair kpair(j))
  constexpr int NDKA = MODE == KV_DK1 || MODE == KV_DK2 ? 1 : NPAIR;
  auto kpair = [](int j) { return MODE == KV_DK2 ? 1 : j; };
  constexpr int DKP = DK < 32 ? 32 : DK, DVP = DV < 32 ? 32 : DV;
  constexpr int NCK = DK / KC, NCV = DV / KC, NDK = DKP / 32, NDV = DVP / 32, NQB = BMQ / 32, NC2 = 32 / KC;
  constexpr int BNK = NW * KW * 32;
  typedef Tile<T, BMQ, DKP> QTile;
  typedef Tile<T, BMQ, DVP> OTile;
  // per buffer: the q tiles, the dO tile, the tile's document starts (int) and row scales (float)
  constexpr int BUF = NPAIR * QTile::BYTES + OTile::BYTES + BMQ * 8;
  typedef PartStager<T, BMQ, DK, DKP, DV, DVP, NT, NPAIR> Stager;
  // three tile buffers (each query tile staged over two steps, one chunk per thread at a time) when they fit the
  // 160 KB of LDS and the tile splits evenly over the threads, else two (and for the two-pair kinds, whose single
  // key-side kernel is already short of registers)
  constexpr int NBUF = Stager::OK && NPAIR == 1 && NQB >= 2 && 3 * BUF <= 160 * 1024 ? 3 : 2;
  static_assert((NBUF == 3) == kv_scales_in_pass(sizeof(T) == 4, POLY, DK, DV), "host mirror of the staging choice");
  // The block's K and V rows come in, and its dK / dV rows go out, through LDS as whole coalesced rows (ROWLDS;
  // not with zero-padded head dims, whose pad columns in the tile buffers must stay zero).
  typedef Tile<T, BNK, DKP> KRows;
  typedef Tile<T, BNK, DVP> VRows;
  constexpr bool ROWLDS = DKP == DK && DVP == DV && NPAIR == 1 && KRows::BYTES + VRows::BYTES <= 160 * 1024 - 16 * NW;
  static_assert(!rope_dk_epilogue(sizeof(T) == 4, POLY, DK, DV) || ROWLDS, "rotary gradient in the dK epilogue");
  constexpr int SMEM = cmax(NBUF * BUF, cmax(ROWLDS ? NPAIR * KRows::BYTES + VRows::BYTES : 0, cmax(KRows::BYTES, VRows::BYTES)));
  static_assert(SMEM <= 160 * 1024 - 16 * NW, "LDS");
  __shared__ __attribute__((aligned(16))) char smem_[SMEM];
  __shared__ float red_[NW][4];
  char TNPA_LDS* smem = (char TNPA_LDS*)smem_;

  const int T_ = p.T, BH = p.B * p.H;
  const int NNB = (T_ + BNK - 1) / BNK;
  const int item = blockIdx.x;
  const int nb = item / BH, bh = item % BH, b = bh / p.H, hd = bh % p.H;
  const int n0 = nb * BNK;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, l32 = lane & 31;

  const T* qp[2] = {head_ptr<T>(p.q1, b, hd), head_ptr<T>(p.q2, b, hd)};
  const T* kp[2] = {head_ptr<T>(p.k1, b, hd), head_ptr<T>(p.k2, b, hd)};
  const int64_t qst[2] = {p.q1.st, p.q2.st}, kst[2] = {p.k1.st, p.k2.st};
  const T* vp = head_ptr<T>(p.v, b, hd);
  const T* dop = head_ptr<T>(p.dout, b, hd);
  const Coefs cf = load_coefs(p, hd);
  const int* dst = p.dstart + (int64_t)b * T_;
  const float* rsc = p.rscale + (int64_t)b * T_;

  if constexpr (DKP != DK || DVP != DV) {
    for (int i = threadIdx.x; i < SMEM / 16; i += NT) ((u32x4 TNPA_LDS*)smem)[i] = u32x4{0u, 0u, 0u, 0u};
    __syncthreads();
  }

  const int nw0 = n0 + wave * KW * 32;
  Op kf[NPAIR][KW][NCK];
  Op vf[KW][NCV];
  int ka[KW];
#pragma unroll
  for (int s = 0; s < KW; ++s) {
    ka[s] = nw0 + 32 * s;
    const int key = ka[s] + l32;
    const bool valid = key < T_;
    if constexpr (!ROWLDS) {
#pragma unroll
      for (int pr = 0; pr < NPAIR; ++pr)
#pragma unroll
        for (int c = 0; c < NCK; ++c) kf[pr][s][c] = valid ? load_op<T>(kp[pr] + (int64_t)key * kst[pr], c, h) : M::zero();
#pragma unroll
      for (int c = 0; c < NCV; ++c) vf[s][c] = valid ? load_op<T>(vp + (int64_t)key * p.v.st, c, h) : M::zero();
    }
  }
  if constexpr (ROWLDS) {
    Stage<T, BNK, DK, DKP, NT> ks[NPAIR];
    Stage<T, BNK, DV, DVP, NT> vs;  // V only feeds dP (dK pass)
#pragma unroll
    for (int pr = 0; pr < NPAIR; ++pr) ks[pr].load(kp[pr], kst[pr], n0, T_ - n0);
    if constexpr (WANT_DK) vs.load(vp, p.v.st, n0, T_ - n0);
#pragma unroll
    for (int pr = 0; pr < NPAIR; ++pr) ks[pr].store(smem + pr * KRows::BYTES);
    if constexpr (WANT_DK) vs.store(smem + NPAIR * KRows::BYTES);
    __syncthreads();
#pragma unroll
    for (int s = 0; s < KW; ++s) {
#pragma unroll
      for (int pr = 0; pr < NPAIR; ++pr)
#pragma unroll
        for (int c = 0; c < NCK; ++c) kf[pr][s][c] = read_row<T, KRows>(smem + pr * KRows::BYTES, 32 * (wave * KW + s), l32, c, h);
#pragma unroll
      for (int c = 0; c < (WANT_DK ? NCV : 0); ++c)
        vf[s][c] = read_row<T, VRows>(smem + NPAIR * KRows::BYTES, 32 * (wave * KW + s), l32, c, h);
    }
    __syncthreads();
  }

  f32x16 dk[NDKA][KW][NDK], dv[KW][NDV];
#pragma unroll
  for (int s = 0; s < KW; ++s) {
#pragma unroll
    for (int d = 0; d < NDV; ++d) dv[s][d] = zero16();
#pragma unroll
    for (int j = 0; j < NDKA; ++j)
#pragma unroll
      for (int d = 0; d < NDK; ++d) dk[j][s][d] = zero16();
  }
  float gsum[4] = {0.f, 0.f, 0.f, 0.f};

  const int qlo = (n0 / BMQ) * BMQ;
  const int qhi = p.qend[(int64_t)b * T_ + min(n0 + BNK, T_) - 1];
  Stage<T, BMQ, DK, DKP, NT> sq[NPAIR];
  Stage<T, BMQ, DV, DVP, NT> so;
  constexpr int DSOFF = NPAIR * QTile::BYTES + OTile::BYTES;
  const T* dscp = head_ptr<T>(p.dsc, b, hd);
  auto ds_of = [&](const int m) { return m + (int)threadIdx.x < T_ ? dst[m + threadIdx.x] : INT_MAX; };
  // Three buffers: the row scale multiplies P and H in fp32 (as ref: tnlm/kernels/poly_attn.py:119-122 does), read
  // per query from LDS next to the document starts; 1 when the caller's dO is already scaled. Two buffers: dO is
  // scaled (by the caller, or here while staging) instead.
  auto sc_of = [&](const int m) {
    return p.dpre ? 1.0f : (m + (int)threadIdx.x < T_ ? rsc[m + threadIdx.x] : 0.f);
  };
  int dsv = 0;
  float scv = 0.f;
  Stager stg;
  if constexpr (NBUF == 3) {
    if (p.dpre) stg.init(qp, qst, dscp, p.dsc.st, T_);
    else stg.init(qp, qst, dop, p.dout.st, T_);
    stg.load(3, qlo);
    if (threadIdx.x < BMQ) {
      dsv = ds_of(qlo);
      scv = sc_of(qlo);
    }
#pragma unroll
    for (int q = 0; q < Stager::NPARTS; ++q) stg.store_part(q, smem);
    if (threadIdx.x < BMQ) {
      ((int TNPA_LDS*)(smem + DSOFF))[threadIdx.x] = dsv;
      ((float TNPA_LDS*)(smem + DSOFF + BMQ * 4))[threadIdx.x] = scv;
    }
    stg.load(3, qlo + BMQ);
    if (threadIdx.x < BMQ) {
      dsv = ds_of(qlo + BMQ);
      scv = sc_of(qlo + BMQ);
    }
  } else {
#pragma unroll
    for (int pr = 0; pr < NPAIR; ++pr) sq[pr].load(qp[pr], qst[pr], qlo, T_ - qlo);
    if (p.dpre) so.load(dscp, p.dsc.st, qlo, T_ - qlo);
    else so.load_scaled(dop, p.dout.st, qlo, T_ - qlo, rsc);
    if (threadIdx.x < BMQ) dsv = ds_of(qlo);
#pragma unroll
    for (int pr = 0; pr < NPAIR; ++pr) sq[pr].store(smem + pr * QTile::BYTES);
    so.store(smem + NPAIR * QTile::BYTES);
    if (threadIdx.x < BMQ) ((int TNPA_LDS*)(smem + DSOFF))[threadIdx.x] = dsv;
  }
  __syncthreads();
  auto next_buf = [](const int c) { return c + 1 == NBUF ? 0 : c + 1; };

  int cur = 0;
  // One 32-query sub-block for this wave. am / fm: wave-uniform bitmasks of the key subtiles seen by any query of
  // the sub-block / seen by all of them.
  // mid: work placed between the sub-block's S/dP MFMA chains and its VALU (the spread tile staging)
  auto sub = [&](const char TNPA_LDS* base, const int TNPA_LDS* dsl, const int m, const int qb, const uint32_t am, const uint32_t fm, auto all_c, auto full_c,
                 auto&& mid) {
    constexpr bool ALL = decltype(all_c)::value, FULL = decltype(full_c)::value;
    f32x16 sacc[NPAIR][KW], pacc[KW];
#pragma unroll
    for (int s = 0; s < KW; ++s) {
      pacc[s] = zero16();
#pragma unroll
      for (int pr = 0; pr < NPAIR; ++pr) sacc[pr][s] = zero16();
    }
#pragma unroll
    for (int c = 0; c < NCK; ++c)
#pragma unroll
      for (int pr = 0; pr < NPAIR; ++pr) {
        const Op a = read_row<T, QTile>(base + pr * QTile::BYTES, 32 * qb, kappa<T>(l32), c, h);
#pragma unroll
        for (int s = 0; s < KW; ++s)
          if (ALL || ((am >> s) & 1u)) sacc[pr][s] = M::mma(a, kf[pr][s][c], sacc[pr][s]);
      }
    if constexpr (WANT_DK) {
#pragma unroll
      for (int c = 0; c < NCV; ++c) {
        const Op a = read_row<T, OTile>(base + NPAIR * QTile::BYTES, 32 * qb, kappa<T>(l32), c, h);
#pragma unroll
        for (int s = 0; s < KW; ++s)
          if (ALL || ((am >> s) & 1u)) pacc[s] = M::mma(a, vf[s][c], pacc[s]);
      }
    }
    mid();
    Op po[KW][NC2];
    Op dso[NDKA][KW][NC2];
#pragma unroll
    for (int s = 0; s < KW; ++s) {
      if (!(ALL || ((am >> s) & 1u))) continue;
      float pv[16], d1[16], d2[16];
      // row scale of each accumulator row (query): from LDS with three-buffer staging, else 1 (dO came scaled)
      float rsr[16];
#pragma unroll
      for (int r = 0; r < 16; ++r)
        rsr[r] = NBUF == 3 ? ((const float TNPA_LDS*)(dsl + BMQ))[32 * qb + key_off<T>(r, h)] : 1.0f;
      if (FULL || ((fm >> s) & 1u)) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float r1 = sacc[0][s][r], r2 = sacc[NPAIR - 1][s][r];
          if constexpr (WANT_DV) pv[r] = poly_value<POLY, MODE == KV_BOTH, PRE>(r1, r2, p.kind, p.deg, p.sm, cf) * rsr[r];
          if constexpr (WANT_DK)
            poly_grad<POLY, PAR, MODE == KV_BOTH, PRE>(r1, r2, pacc[s][r] * rsr[r], p.kind, p.deg, p.sm, cf, d1[r], d2[r], gsum);
        }
      } else {
        const int key = ka[s] + l32;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qo = 32 * qb + key_off<T>(r, h);
          const bool vis = key <= m + qo && dsl[qo] <= key;
          const float r1 = sacc[0][s][r], r2 = sacc[NPAIR - 1][s][r];
          if constexpr (WANT_DV)
            pv[r] = vis ? poly_value<POLY, MODE == KV_BOTH, PRE>(r1, r2, p.kind, p.deg, p.sm, cf) * rsr[r] : 0.f;
          if constexpr (WANT_DK)
            poly_grad<POLY, PAR, MODE == KV_BOTH, PRE>(r1, r2, vis ? pacc[s][r] * rsr[r] : 0.f, p.kind, p.deg, p.sm, cf, d1[r], d2[r], gsum);
        }
      }
#pragma unroll
      for (int c2 = 0; c2 < NC2; ++c2) {
        if constexpr (WANT_DV) po[s][c2] = M::cvt(pv + c2 * EPL);
        if constexpr (WANT_DK && NDKA == NPAIR) {
          dso[0][s][c2] = M::cvt(d1 + c2 * EPL);
          if constexpr (NPAIR == 2) dso[NPAIR - 1][s][c2] = M::cvt(d2 + c2 * EPL);
        } else if constexpr (WANT_DK) {
          dso[0][s][c2] = M::cvt((MODE == KV_DK2 ? d2 : d1) + c2 * EPL);
        }
      }
    }
    // the dK pass of a one-pair 16-bit kind, and the combined kernel of a two-pair one, also store dS (dS1 and dS2)
    // for the dQ-from-dS kernel: tile (query sub-block, key sub-block), each of its two operands one contiguous KiB
    // (layout at ds_tile_rows). Issued between the dV and dK products for lower_degree_mix, after the dK products
    // otherwise (same-process timing of the three positions).
    auto store_ds = [&]() {
      if constexpr (((MODE == KV_DK && NPAIR == 1) || (MODE == KV_BOTH && NPAIR == 2)) && sizeof(T) == 2) {
        if (p.dstile != nullptr) {
          const int qi = (m >> 5) + qb;
          const int64_t toff = ((int64_t)bh * ds_tiles_per_head(T_) + (int64_t)qi * (qi + 1) / 2) * 1024 + l32 * 16 + h * 8;
#pragma unroll
          for (int pr = 0; pr < NPAIR; ++pr) {
            T* tb = (T*)(pr == 0 ? p.dstile : p.dstile2) + toff;
#pragma unroll
            for (int s = 0; s < KW; ++s) {
              if (!(ALL || ((am >> s) & 1u))) continue;
              T* tp = tb + (int64_t)(ka[s] >> 5) * 1024;
#pragma unroll
              for (int c2 = 0; c2 < NC2; ++c2) __builtin_nontemporal_store(dso[pr][s][c2], (Op*)(tp + 512 * c2));
            }
          }
        }
      }
    };
    constexpr bool DS_MID = POLY == POLY_GEN2;
    if constexpr (WANT_DV) {
#pragma unroll
      for (int d = 0; d < NDV; ++d)
#pragma unroll
        for (int c2 = 0; c2 < NC2; ++c2) {
          const Op a = read_col<T, OTile>(base + NPAIR * QTile::BYTES, 32 * qb + c2 * KC, 32 * d, lane);
#pragma unroll
          for (int s = 0; s < KW; ++s)
            if (ALL || ((am >> s) & 1u)) dv[s][d] = M::mma(a, po[s][c2], dv[s][d]);
        }
    }
    if constexpr (DS_MID) store_ds();
    if constexpr (WANT_DK) {
#pragma unroll
      for (int j = 0; j < NDKA; ++j)
#pragma unroll
        for (int d = 0; d < NDK; ++d)
#pragma unroll
          for (int c2 = 0; c2 < NC2; ++c2) {
            const Op a = read_col<T, QTile>(base + kpair(j) * QTile::BYTES, 32 * qb + c2 * KC, 32 * d, lane);
#pragma unroll
            for (int s = 0; s < KW; ++s)
              if (ALL || ((am >> s) & 1u)) dk[j][s][d] = M::mma(a, dso[j][s][c2], dk[j][s][d]);
          }
    }
    if constexpr (!DS_MID) store_ds();
  };

  auto step = [&](const int m, auto fast_c) {
    constexpr bool FAST = decltype(fast_c)::value;
    const bool more = NBUF == 2 && m + BMQ < qhi;
    // three buffers: tile j+1 (in registers since the previous step) is written to its buffer and tile j+2 loaded
    // in its place, one 16-byte chunk per thread at each of 2 * NQB points (the middle and the end of every
    // sub-block), so that the loads of all waves reach the memory pipe spread over the step
    char TNPA_LDS* b1 = smem + next_buf(cur) * BUF;
    auto stage_at = [&](const int point) {
      if constexpr (NBUF == 3) {
#pragma unroll
        for (int q = 0; q < Stager::NPARTS; ++q)
          if (q % (2 * NQB) == point) {
            stg.store_part(q, b1);
            stg.load_part(q, m + 2 * BMQ);
          }
        if (point == 0 && threadIdx.x < BMQ) {
          ((int TNPA_LDS*)(b1 + DSOFF))[threadIdx.x] = dsv;
          ((float TNPA_LDS*)(b1 + DSOFF + BMQ * 4))[threadIdx.x] = scv;
          dsv = ds_of(m + 2 * BMQ);
          scv = sc_of(m + 2 * BMQ);
        }
      }
    };
    auto mid_for = [&](const int qb) { return [&, qb]() { stage_at(2 * qb); }; };
    if (more) {
#pragma unroll
      for (int pr = 0; pr < NPAIR; ++pr) sq[pr].load(qp[pr], qst[pr], m + BMQ, T_ - m - BMQ);
      if (p.dpre) so.load(dscp, p.dsc.st, m + BMQ, T_ - m - BMQ);
      else so.load_scaled(dop, p.dout.st, m + BMQ, T_ - m - BMQ, rsc);
      if (threadIdx.x < BMQ) dsv = ds_of(m + BMQ);
    }
    const char TNPA_LDS* base = smem + cur * BUF;
    const int TNPA_LDS* dsl = (const int TNPA_LDS*)(base + DSOFF);
    if constexpr (FAST) {
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) {
        sub(base, dsl, m, qb, 0u, 0u, std::true_type{}, std::true_type{}, mid_for(qb));
        stage_at(2 * qb + 1);
      }
    } else {
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) {
        stage_at(2 * qb);  // outside the skip tests: one code path, so no wait on the loads it issues
        stage_at(2 * qb + 1);
        const int q0 = m + 32 * qb;
        if (q0 >= T_) continue;
        const int qlast = min(q0 + 31, T_ - 1);
        const int ds0 = dsl[32 * qb], dsL = dsl[qlast - m];
        uint32_t am = 0, fm = 0;
#pragma unroll
        for (int s = 0; s < KW; ++s) {
          if (ka[s] < T_ && ka[s] <= qlast && ka[s] + 31 >= ds0) am |= 1u << s;
          if (ka[s] + 31 <= q0 && dsL <= ka[s] && q0 + 31 < T_) fm |= 1u << s;
        }
        am = __builtin_amdgcn_readfirstlane(am);
        fm = __builtin_amdgcn_readfirstlane(fm);
        if (am == 0) continue;
        sub(base, dsl, m, qb, am, fm, std::false_type{}, std::false_type{}, [] {});
      }
    }
    if (more) {
#pragma unroll
      for (int pr = 0; pr < NPAIR; ++pr) sq[pr].store(b1 + pr * QTile::BYTES);
      so.store(b1 + NPAIR * QTile::BYTES);
      if (threadIdx.x < BMQ) ((int TNPA_LDS*)(b1 + DSOFF))[threadIdx.x] = dsv;
    }
    __syncthreads();
    cur = next_buf(cur);
  };
  // Query tiles qlo, qlo+BMQ, ... < qhi, split per wave into: the diagonal (generic), tiles whose every query sees
  // every key of the wave (fast), and tiles past the wave's document end or the sequence end (generic).
  const int ntile = (qhi - qlo + BMQ - 1) / BMQ;
  int j0 = ntile, j1 = ntile;
  if (nw0 < T_) {
    const int klast = nw0 + 32 * KW - 1;
    const int qe = min(T_, p.qend[(int64_t)b * T_ + nw0]);
    j0 = min(ntile, max(0, (klast - qlo + BMQ - 1) / BMQ));
    j1 = max(j0, min(ntile, (qe - qlo) / BMQ));
  }
  j0 = __builtin_amdgcn_readfirstlane(j0);
  j1 = __builtin_amdgcn_readfirstlane(j1);
  int j = 0;
  for (; j < j0; ++j) step(qlo + j * BMQ, std::false_type{});
  for (; j < j1; ++j) step(qlo + j * BMQ, std::true_type{});
  for (; j < ntile; ++j) step(qlo + j * BMQ, std::false_type{});

  // dV and dK rows: scaled in registers, then (ROWLDS) gathered in LDS and written as whole rows, else stored from
  // the accumulators (the two-pair and padded-head-dim kernels: gathering in LDS there costs spills in the loop; with
  // rotary tables their dK is rotated by a pass after the kernel)
  const TDesc* kouts[2] = {&p.dk1, &p.dk2};
  if constexpr (ROWLDS) {
    if constexpr (WANT_DV) {
      __syncthreads();  // every wave is done with the tile buffers
#pragma unroll
      for (int s = 0; s < KW; ++s) acc_rows_to_lds<T, VRows, NDV>(smem, 32 * (wave * KW + s), l32, h, dv[s], p.vf, DV);
      __syncthreads();
      Stage<T, BNK, DV, DVP, NT> os;
      os.copy_out(smem, head_ptr_w<T>(p.dv, b, hd), p.dv.st, n0, T_ - n0);
    }
    if constexpr (WANT_DK) {
#pragma unroll
      for (int j = 0; j < NDKA; ++j) {
        const int pr = kpair(j);
        __syncthreads();  // every wave is done with the tile buffers (or with the previous rows)
#pragma unroll
        for (int s = 0; s < KW; ++s) acc_rows_to_lds<T, KRows, NDK>(smem, 32 * (wave * KW + s), l32, h, dk[j][s], p.gf, DK);
        __syncthreads();
        Stage<T, BNK, DK, DKP, NT> os;
        if (p.rcos != nullptr)
          os.copy_out_rope(smem, head_ptr_w<T>(*kouts[pr], b, hd), kouts[pr]->st, n0, T_ - n0, p.rcos, p.rsin,
                           (int64_t)b * T_ + n0);
        else
          os.copy_out(smem, head_ptr_w<T>(*kouts[pr], b, hd), kouts[pr]->st, n0, T_ - n0);
      }
    }
  } else {
#pragma unroll
    for (int s = 0; s < KW; ++s) {
      const int key = ka[s] + l32;
      if (key >= T_) continue;
      T* vrow = head_ptr_w<T>(p.dv, b, hd) + (int64_t)key * p.dv.st;
#pragma unroll
      for (int d = 0; d < (WANT_DV ? NDV : 0); ++d)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int col = 32 * d + 8 * g + 4 * h;
          if (col < DV)
            store4<T>(vrow + col, dv[s][d][4 * g] * p.vf, dv[s][d][4 * g + 1] * p.vf, dv[s][d][4 * g + 2] * p.vf,
                      dv[s][d][4 * g + 3] * p.vf);
        }
#pragma unroll
      for (int j = 0; j < (WANT_DK ? NDKA : 0); ++j) {
        const int pr = kpair(j);
        T* krow = head_ptr_w<T>(*kouts[pr], b, hd) + (int64_t)key * kouts[pr]->st;
#pragma unroll
        for (int d = 0; d < NDK; ++d)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int col = 32 * d + 8 * g + 4 * h;
            if (col < DK)
              store4<T>(krow + col, dk[j][s][d][4 * g] * p.gf, dk[j][s][d][4 * g + 1] * p.gf,
                        dk[j][s][d][4 * g + 2] * p.gf, dk[j][s][d][4 * g + 3] * p.gf);
          }
      }
    }
  }

  if constexpr (PAR) {
    if (p.dpar != nullptr && (p.kind == KIND_OS || p.kind == KIND_LDM)) {
      // fixed-order reduction: lanes (butterfly), then waves in index order
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float x = gsum[i];
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
        gsum[i] = x;
      }
      if (lane == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) red_[wave][i] = gsum[i];
      }
      __syncthreads();
      if (threadIdx.x < 4) {
        float acc = 0.f;
        for (int w = 0; w < NW; ++w) acc += red_[w][threadIdx.x];
        p.dpar[((int64_t)bh * NNB + nb) * 4 + threadIdx.x] = acc;
      }
    }
  }
}

// ------------------------------------------------------------------------------------------------ dK / dV, wave pairs
// ref: tnlm/kernels/poly_attn.py:77-148 (_bwd_kv), for 16-bit inputs, one q/k pair, head dim 128. S and dP are computed
// once per (query, key) sub-block, by splitting the work of 32 keys between two waves on one SIMD by product rather
// than by rows (each role then holds half the state, so both fit two waves per SIMD):
//   producer (waves 0-3): the K and V rows of its 32 keys in registers; per 32-query sub-block S = Q K^T and
//            dP = dO V^T from LDS row reads of the staged Q / dO tile; P = mask(A(S)) * row_scale and
//            dS = mask(A'(S) * dP * row_scale) in fp32 (ref: tnlm/kernels/poly_attn.py:113-136), each rounded to the
//            input dtype into the pair's exchange slot in LDS (and dS into the dS tiles when dQ is read from them);
//   consumer (waves 4-7): one sub-block behind, dV^T += dO^T P and dK^T += Q^T dS from transposed reads of the same
//            staged tiles, the dV and dK accumulators in registers. The consumers also stage the Q / dO tiles, so
//            the producers' global stores never sit ahead of a load somebody waits for (loads and stores retire in
//            issue order).
// A workgroup owns 128 keys (pair p: keys n0 + 32 p .. + 31; waves p and p + 4 share SIMD p). One barrier per 32-query
// step publishes the exchange slot and the staged tiles: step k runs producer sub-block k and consumer sub-block k-1.
// Per sub-block and pair 16 + 16 matrix instructions, against 16 + 24 for the separate dV and dK passes. The rounding
// points are those of the passes, so dK and dV are bit-identical to theirs.
template <typename T, int POLY, int DK, int DV>
__global__ void __attribute__((amdgpu_flat_work_group_size(512, 512), amdgpu_waves_per_eu(2)))
k_bwd_kv_pair(const KParams p) {
  typedef Mfma<T> M;
  typedef typename M::Op Op;
  static_assert(sizeof(T) == 2 && !two_pair_poly(POLY) && DK == 128 && DV == 128, "16-bit, one pair, head dim 128");
  constexpr int KC = M::KC, EPL = M::EPL;
  constexpr bool PRE = prescaled<T, POLY>();
  constexpr bool PAR = POLY == POLY_OS;
  constexpr int NCK = DK / KC, NCV = DV / KC, NDK = DK / 32, NDV = DV / 32, NC2 = 32 / KC;
  constexpr int NPR = 4, BNK = 32 * NPR, BMQ = 64;
  typedef Tile<T, BMQ, DK> QTile;
  typedef Tile<T, BMQ, DV> OTile;
  typedef Tile<T, BNK, DK> KRows;
  typedef Tile<T, BNK, DV> VRows;
  constexpr int DSOFF = QTile::BYTES + OTile::BYTES;  // per query of the tile: doc start (int), row scale (float)
  constexpr int BUF = DSOFF + BMQ * 8;
  constexpr int NBUF = 3;
  constexpr int XSLOT = 2 * NC2 * 64 * 16;  // P and dS operands of one sub-block, 16 bytes per lane each
  constexpr int XOFF = NBUF * BUF;
  constexpr int SMEM = cmax(XOFF + NPR * 2 * XSLOT, KRows::BYTES + VRows::BYTES);
  static_assert(SMEM <= 160 * 1024 - 64, "LDS");
  __shared__ __attribute__((aligned(16))) char smem_[SMEM];
  __shared__ float red_[NPR][4];
  char TNPA_LDS* smem = (char TNPA_LDS*)smem_;

  const int T_ = p.T, BH = p.B * p.H;
  const int NNB = (T_ + BNK - 1) / BNK;
  const int item = blockIdx.x;
  const int nb = item / BH, bh = item % BH, b = bh / p.H, hd = bh % p.H;
  const int n0 = nb * BNK;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, l32 = lane & 31;
  const bool prod = wave < NPR;
  const int pr = wave & (NPR - 1);
  const int ka = n0 + 32 * pr;
  const T* qp = head_ptr<T>(p.q1, b, hd);
  const T* kp = head_ptr<T>(p.k1, b, hd);
  const T* vp = head_ptr<T>(p.v, b, hd);
  const T* dop = p.dpre ? head_ptr<T>(p.dsc, b, hd) : head_ptr<T>(p.dout, b, hd);
  const int64_t dost = p.dpre ? p.dsc.st : p.dout.st;
  const Coefs cf = load_coefs(p, hd);
  const int* dst = p.dstart + (int64_t)b * T_;
  const float* rsc = p.rscale + (int64_t)b * T_;

  // K and V rows of the block through LDS as whole rows (every thread); the producers take their operands from there
  {
    Stage<T, BNK, DK, DK, 512> ks;
    Stage<T, BNK, DV, DV, 512> vs;
    ks.load(kp, p.k1.st, n0, T_ - n0);
    vs.load(vp, p.v.st, n0, T_ - n0);
    ks.store(smem);
    vs.store(smem + KRows::BYTES);
  }
  __syncthreads();

  const int qlo = (n0 / BMQ) * BMQ;
  const int qhi = min(T_, p.qend[(int64_t)b * T_ + min(n0 + BNK, T_) - 1]);
  const int ntile = max(0, (qhi - qlo + BMQ - 1) / BMQ);
  const int nsb = 2 * ntile;

  // whether (this pair's keys, query sub-block k) has a visible pair, and whether all its pairs are visible: the
  // producer and the consumer evaluate it identically from the staged doc starts
  auto sub_state = [&](const int k, const char TNPA_LDS*& base, int& m, int& qb, bool& any, bool& full) {
    const int t = k >> 1;
    qb = k & 1;
    base = smem + (t % NBUF) * BUF;
    m = qlo + t * BMQ;
    const int q0 = m + 32 * qb;
    const int TNPA_LDS* dsl = (const int TNPA_LDS*)(base + DSOFF);
    const int qlast = min(q0 + 31, T_ - 1);
    const int ds0 = dsl[32 * qb], dsL = dsl[max(0, qlast - m)];
    any = uniform_bool(q0 < T_ && ka < T_ && ka <= qlast && ka + 31 >= ds0);
    full = uniform_bool(ka + 31 <= q0 && dsL <= ka && q0 + 31 < T_);
  };
  float gsum[4] = {0.f, 0.f, 0.f, 0.f};

  // Both roles run the same barrier sequence: K/V operands (1), staging prologue (2), one per step, epilogue (4).
  if (prod) {
    Op kf[NCK], vf[NCV];
#pragma unroll
    for (int c = 0; c < NCK; ++c) kf[c] = read_row<T, KRows>(smem, 32 * pr, l32, c, h);
#pragma unroll
    for (int c = 0; c < NCV; ++c) vf[c] = read_row<T, VRows>(smem + KRows::BYTES, 32 * pr, l32, c, h);
    __syncthreads();
    __syncthreads();
    T* dsrow = p.dstile == nullptr ? nullptr
                                   : (T*)p.dstile + (int64_t)bh * ds_tiles_per_head(T_) * 1024 + l32 * 16 + h * 8;
    auto produce = [&](const int k, const char TNPA_LDS* base, const int m, const int qb, auto full_c) {
      constexpr bool FULL = decltype(full_c)::value;
      f32x16 sacc = zero16(), pacc = zero16();
#pragma unroll
      for (int c = 0; c < NCK; ++c) sacc = M::mma(read_row<T, QTile>(base, 32 * qb, kappa<T>(l32), c, h), kf[c], sacc);
#pragma unroll
      for (int c = 0; c < NCV; ++c)
        pacc = M::mma(read_row<T, OTile>(base + QTile::BYTES, 32 * qb, kappa<T>(l32), c, h), vf[c], pacc);
      // row scale of accumulator row r: query 32 qb + key_off(r, h), two runs of 8 consecutive queries
      const float TNPA_LDS* rsl = (const float TNPA_LDS*)(base + DSOFF + BMQ * 4) + 32 * qb + 8 * h;
      float rsr[16];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 x = *(const f32x4 TNPA_LDS*)(rsl + 16 * (g >> 1) + 4 * (g & 1));
#pragma unroll
        for (int i = 0; i < 4; ++i) rsr[4 * g + i] = x[i];
      }
      float pv[16], d1[16], d2[16];
      if constexpr (FULL) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          pv[r] = poly_value<POLY, false, PRE>(sacc[r], sacc[r], p.kind, p.deg, p.sm, cf) * rsr[r];
          poly_grad<POLY, PAR, false, PRE>(sacc[r], sacc[r], pacc[r] * rsr[r], p.kind, p.deg, p.sm, cf, d1[r], d2[r],
                                           gsum);
        }
      } else {
        const int TNPA_LDS* dsl = (const int TNPA_LDS*)(base + DSOFF);
        const int key = ka + l32;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qo = 32 * qb + key_off<T>(r, h);
          const bool vis = key <= m + qo && dsl[qo] <= key;
          pv[r] = vis ? poly_value<POLY, false, PRE>(sacc[r], sacc[r], p.kind, p.deg, p.sm, cf) * rsr[r] : 0.f;
          poly_grad<POLY, PAR, false, PRE>(sacc[r], sacc[r], vis ? pacc[r] * rsr[r] : 0.f, p.kind, p.deg, p.sm, cf,
                                           d1[r], d2[r], gsum);
        }
      }
      char TNPA_LDS* xs = smem + XOFF + (pr * 2 + (k & 1)) * XSLOT;
#pragma unroll
      for (int c2 = 0; c2 < NC2; ++c2) {
        const Op po = M::cvt(pv + c2 * EPL), so = M::cvt(d1 + c2 * EPL);
        *(Op TNPA_LDS*)(xs + (c2 * 64 + lane) * 16) = po;
        *(Op TNPA_LDS*)(xs + ((NC2 + c2) * 64 + lane) * 16) = so;
        if (dsrow != nullptr) {
          const int qi = (m >> 5) + qb;
          __builtin_nontemporal_store(so, (Op*)(dsrow + ((int64_t)qi * (qi + 1) / 2 + (ka >> 5)) * 1024 + 512 * c2));
        }
      }
    };
    for (int k = 0; k <= nsb; ++k) {
      if (k < nsb) {
        const char TNPA_LDS* base;
        int m, qb;
        bool any, full;
        sub_state(k, base, m, qb, any, full);
        if (full) produce(k, base, m, qb, std::true_type{});
        else if (any) produce(k, base, m, qb, std::false_type{});
      }
      __syncthreads();
    }
    // epilogue: the consumers gather dV, then dK, every thread copies the rows out
    __syncthreads();
    {
      Stage<T, BNK, DV, DV, 512> os;
      os.copy_out(smem, head_ptr_w<T>(p.dv, b, hd), p.dv.st, n0, T_ - n0);
    }
    __syncthreads();
    __syncthreads();
    {
      Stage<T, BNK, DK, DK, 512> os;
      if (p.rcos != nullptr)
        os.copy_out_rope(smem, head_ptr_w<T>(p.dk1, b, hd), p.dk1.st, n0, T_ - n0, p.rcos, p.rsin, (int64_t)b * T_ + n0);
      else
        os.copy_out(smem, head_ptr_w<T>(p.dk1, b, hd), p.dk1.st, n0, T_ - n0);
    }
  } else {
    __syncthreads();  // the producers have their K / V operands: the row area is free
    // staging of the Q (part 0, with the doc starts and row scales) and dO (part 1) rows of a 64-query tile: 4 chunks
    // of 16 bytes per consumer thread and part, consecutive threads along a row
    const int ct = (int)threadIdx.x - NPR * 64;
    u32x4 sr[4];
    uint32_t qoff[4], ooff[4], loff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int idx = ct + 256 * i, row = idx >> 4, c = idx & 15;
      qoff[i] = (uint32_t)(((int64_t)row * p.q1.st + c * 8) * 2);
      ooff[i] = (uint32_t)(((int64_t)row * dost + c * 8) * 2);
      loff[i] = QTile::off(row, c * 8);
    }
    int dsv = 0;
    float scv = 0.f;
    auto load_part = [&](const int part, const int m) {
      if (part == 0) {
        const auto rs = rows_rsrc<T>(qp, p.q1.st, m, T_, DK);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          sr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)qoff[i], 0, 0));
        if (ct < BMQ) {
          const int q = m + ct;
          dsv = q < T_ ? dst[q] : INT_MAX;
          scv = p.dpre ? 1.0f : (q < T_ ? rsc[q] : 0.f);
        }
      } else {
        const auto rs = rows_rsrc<T>(dop, dost, m, T_, DV);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          sr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)ooff[i], 0, 0));
      }
    };
    auto store_part = [&](const int part, char TNPA_LDS* buf) {
      char TNPA_LDS* tb = buf + (part ? QTile::BYTES : 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) *(u32x4 TNPA_LDS*)(tb + loff[i]) = sr[i];
      if (part == 0 && ct < BMQ) {
        ((int TNPA_LDS*)(buf + DSOFF))[ct] = dsv;
        ((float TNPA_LDS*)(buf + DSOFF + BMQ * 4))[ct] = scv;
      }
    };
    // tiles 0 and 1 in LDS before the loop (the dO part of tile 1 is written in step 0); tile u >= 2 is loaded in
    // steps 2u-4 (Q) and 2u-3 (dO) and written one step later, into the buffer of tile u-3 (last read in step 2u-4)
    load_part(0, qlo);
    store_part(0, smem);
    load_part(1, qlo);
    store_part(1, smem);
    load_part(0, qlo + BMQ);
    store_part(0, smem + BUF);
    load_part(1, qlo + BMQ);
    __syncthreads();

    f32x16 dv[NDV], dk[NDK];
#pragma unroll
    for (int d = 0; d < NDV; ++d) dv[d] = zero16();
#pragma unroll
    for (int d = 0; d < NDK; ++d) dk[d] = zero16();
    auto consume = [&](const int k) {
      const char TNPA_LDS* base;
      int m, qb;
      bool any, full;
      sub_state(k, base, m, qb, any, full);
      if (!any) return;
      const char TNPA_LDS* xs = smem + XOFF + (pr * 2 + (k & 1)) * XSLOT;
      Op po[NC2], so[NC2];
#pragma unroll
      for (int c2 = 0; c2 < NC2; ++c2) {
        po[c2] = *(const Op TNPA_LDS*)(xs + (c2 * 64 + lane) * 16);
        so[c2] = *(const Op TNPA_LDS*)(xs + ((NC2 + c2) * 64 + lane) * 16);
      }
#pragma unroll
      for (int d = 0; d < NDV; ++d)
#pragma unroll
        for (int c2 = 0; c2 < NC2; ++c2)
          dv[d] = M::mma(read_col<T, OTile>(base + QTile::BYTES, 32 * qb + c2 * KC, 32 * d, lane), po[c2], dv[d]);
#pragma unroll
      for (int d = 0; d < NDK; ++d)
#pragma unroll
        for (int c2 = 0; c2 < NC2; ++c2)
          dk[d] = M::mma(read_col<T, QTile>(base, 32 * qb + c2 * KC, 32 * d, lane), so[c2], dk[d]);
    };
    for (int k = 0; k <= nsb; ++k) {
      const int kp = k - 1;
      store_part(kp & 1, smem + (((kp >> 1) + 2) % NBUF) * BUF);
      load_part(k & 1, qlo + ((k >> 1) + 2) * BMQ);
      if (k >= 1) consume(k - 1);
      __syncthreads();
    }
    // epilogue: dV rows, then dK rows, through LDS; every thread copies them out
    acc_rows_to_lds<T, VRows, NDV>(smem, 32 * pr, l32, h, dv, p.vf, DV);
    __syncthreads();
    {
      Stage<T, BNK, DV, DV, 512> os;
      os.copy_out(smem, head_ptr_w<T>(p.dv, b, hd), p.dv.st, n0, T_ - n0);
    }
    __syncthreads();
    acc_rows_to_lds<T, KRows, NDK>(smem, 32 * pr, l32, h, dk, p.gf, DK);
    __syncthreads();
    {
      Stage<T, BNK, DK, DK, 512> os;
      if (p.rcos != nullptr)
        os.copy_out_rope(smem, head_ptr_w<T>(p.dk1, b, hd), p.dk1.st, n0, T_ - n0, p.rcos, p.rsin, (int64_t)b * T_ + n0);
      else
        os.copy_out(smem, head_ptr_w<T>(p.dk1, b, hd), p.dk1.st, n0, T_ - n0);
    }
  }

  if constexpr (PAR) {
    if (p.dpar != nullptr) {
      // fixed-order reduction: lanes (butterfly), then the producer waves in index order
      if (prod) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float x = gsum[i];
#pragma unroll
          for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
          if (lane == 0) red_[pr][i] = x;
        }
      }
      __syncthreads();
      if (threadIdx.x < 4) {
        float acc = 0.f;
        for (int w = 0; w < NPR; ++w) acc += red_[w][threadIdx.x];
        p.dpar[((int64_t)bh * NNB + nb) * 4 + threadIdx.x] = acc;
      }
    }
  }
}

// ------------------------------------------------------------------------------------------------ dQ from dS
// dQ = gf * dS K from the dS tiles the key side stored (for two q/k pairs the host launches it once per pair, with
// K2 / dS2 / dQ2 in place of K1 / dS1 / dQ1): one matrix product per (query, key) sub-block instead of the
// S and dP recompute of k_bwd_q. A workgroup owns BM = NW*32 queries; wave w accumulates dQ^T = K^T dS^T for its
// 32-query subtile (lane <-> query). K tiles of BN keys go through three LDS buffers shared by the workgroup (one
// barrier per tile); each wave's dS tiles come from global memory straight into registers two tiles ahead, then
// through a private LDS area of the wave, whose transposed read yields the lane <-> query operand (no barrier: a
// wave reads back only what it wrote). A sub-block without a visible (query, key) pair is skipped and its tile never
// read (its load is pointed past the buffer resource, which returns zeros without a memory access); the dK pass
// stores every sub-block that has one. Same operand rounding as ref: tnlm/kernels/poly_attn.py:196-200 (dS cast to
// the input dtype before the K product, FP32 accumulation).
#ifndef TNPA_DS_LOAD_AUX
#define TNPA_DS_LOAD_AUX 2
#endif
template <typename T, int DK, int NW, int BN>
__global__ void __attribute__((amdgpu_flat_work_group_size(NW * 64, NW * 64), amdgpu_waves_per_eu(2)))
k_bwd_q_ds(const KParams p) {
  typedef Mfma<T> M;
  typedef typename M::Op Op;
  constexpr int KC = M::KC, NT = NW * 64, NDK = DK / 32, NKB = BN / 32, NC2 = 32 / KC;
  constexpr int BM = NW * 32;
  typedef Tile<T, BN, DK> KTile;
  typedef Tile<T, 32, 32> STile;  // one dS sub-block: rows = keys, columns = queries
  typedef Tile<T, BM, DK> QTile;
  typedef Stage<T, BN, DK, DK, NT> KStage;
  static_assert(sizeof(T) == 2 && KStage::TOTAL % NT == 0, "16-bit types, K tiles split evenly over the threads");
  constexpr int NBUF = 3;
  constexpr int PRIV = 2 * NKB * STile::BYTES;  // per wave: the dS tiles of two steps
  constexpr int KOFF = NW * PRIV;
  constexpr int SMEM = cmax(KOFF + NBUF * KTile::BYTES, QTile::BYTES);
  static_assert(SMEM <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(16))) char smem_[SMEM];
  char TNPA_LDS* smem = (char TNPA_LDS*)smem_;

  const int T_ = p.T, BH = p.B * p.H;
  const int NMB = (T_ + BM - 1) / BM;
  const int item = blockIdx.x;
  const int mb = NMB - 1 - item / BH, bh = item % BH, b = bh / p.H, hd = bh % p.H;
  const int m0 = mb * BM;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, l32 = lane & 31;
  const T* kp = head_ptr<T>(p.k1, b, hd);
  const int* dst = p.dstart + (int64_t)b * T_;
  const int qa = m0 + wave * 32, q = qa + l32;
  const int dsq = q < T_ ? dst[q] : INT_MAX;  // first key visible from query q (q + 1 for padding)
  const int qi = qa >> 5;
  // buffer resource over the wave's row of dS tiles (tiles j = 0 .. qi of query sub-block qi)
  const T* trow = (const T*)p.dstile + ((int64_t)bh * ds_tiles_per_head(T_) + (int64_t)qi * (qi + 1) / 2) * 1024;
  const int tbytes = qa < T_ ? (qi + 1) * 2048 : 0;
  const auto srs = __builtin_amdgcn_make_buffer_rsrc((void*)trow, (short)0, tbytes, 0x00020000);
  const uint32_t soff = (uint32_t)(l32 * 32 + h * 16);  // + 1024 * c2 + 2048 * j
  char TNPA_LDS* priv = smem + wave * PRIV;
  char TNPA_LDS* kbuf = smem + KOFF;

  // sub-block (wave's queries, keys key0 .. key0 + 31) has a visible pair: wave-uniform
  auto visible = [&](const int key0) {
    const bool v = q < T_ && max(dsq, key0) <= min(q, key0 + 31);
    return __builtin_amdgcn_readfirstlane((int)(__ballot(v) != 0)) != 0;
  };
  u32x4 sreg[2][NKB][NC2];
  auto load_ds = [&](u32x4 (&r)[NKB][NC2], const int n0) {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const int key0 = n0 + 32 * kb;
      const uint32_t base = visible(key0) ? (uint32_t)((key0 >> 5) * 2048) : (uint32_t)tbytes;
#pragma unroll
      for (int c2 = 0; c2 < NC2; ++c2)
        r[kb][c2] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(srs, (int)(base + soff + 1024 * c2), 0, TNPA_DS_LOAD_AUX));
    }
  };
  auto store_ds = [&](char TNPA_LDS* pt, const u32x4 (&r)[NKB][NC2]) {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int c2 = 0; c2 < NC2; ++c2)
        *(u32x4 TNPA_LDS*)(pt + kb * STile::BYTES + STile::off(l32, 16 * c2 + 8 * h)) = r[kb][c2];
  };

  const int lo = (dst[m0] / BN) * BN;
  const int hi = min(m0 + BM, T_);
  const int ntile = (hi - lo + BN - 1) / BN;
  KStage ks;
  uint32_t kvo[KStage::PER];
#pragma unroll
  for (int i = 0; i < KStage::PER; ++i) kvo[i] = KStage::chunk_off(i, p.k1.st);
  auto load_k = [&](const int n1) {
    const auto rs = rows_rsrc<T>(kp, p.k1.st, n1, T_, DK);
#pragma unroll
    for (int i = 0; i < KStage::PER; ++i) ks.load_buf(i, rs, kvo[i]);
  };
  auto store_k = [&](char TNPA_LDS* dstb) {
#pragma unroll
    for (int i = 0; i < KStage::PER; ++i) ks.store_raw(i, dstb);
  };

  f32x16 dq[NDK];
#pragma unroll
  for (int d = 0; d < NDK; ++d) dq[d] = zero16();

  // prologue: K tile 0 into buffer 0, K tile 1 into registers; dS of tiles 0 and 1 into the two register sets
  load_k(lo);
  load_ds(sreg[0], lo);
  store_k(kbuf);
  load_k(lo + BN);
  load_ds(sreg[1], lo + BN);
  __syncthreads();

  int cur = 0;
  auto next_buf = [](const int c) { return c + 1 == NBUF ? 0 : c + 1; };
  auto step = [&](const int j, auto par_c) {
    constexpr int P = decltype(par_c)::value;
    const int n0 = lo + j * BN;
    char TNPA_LDS* pt = priv + P * NKB * STile::BYTES;
    store_ds(pt, sreg[P]);
    load_ds(sreg[P], n0 + 2 * BN);
    const int nb = next_buf(cur);
    store_k(kbuf + nb * KTile::BYTES);
    load_k(n0 + 2 * BN);
    const char TNPA_LDS* kt = kbuf + cur * KTile::BYTES;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      if (!visible(n0 + 32 * kb)) continue;
      Op bs[NC2];
#pragma unroll
      for (int c2 = 0; c2 < NC2; ++c2) bs[c2] = read_col<T, STile>(pt + kb * STile::BYTES, c2 * KC, 0, lane);
#pragma unroll
      for (int c2 = 0; c2 < NC2; ++c2)
#pragma unroll
        for (int d = 0; d < NDK; ++d) {
          const Op a = read_col<T, KTile>(kt, 32 * kb + c2 * KC, 32 * d, lane);
          dq[d] = M::mma(a, bs[c2], dq[d]);
        }
    }
    __syncthreads();
    cur = nb;
  };
  for (int j = 0; j < ntile; j += 2) {
    step(j, std::integral_constant<int, 0>{});
    if (j + 1 < ntile) step(j + 1, std::integral_constant<int, 1>{});
  }

  // dQ rows: scaled by the chain-rule factor, gathered in LDS, written as whole rows
  __syncthreads();
  acc_rows_to_lds<T, QTile, NDK>(smem, 32 * wave, l32, h, dq, p.gf, DK);
  __syncthreads();
  Stage<T, BM, DK, DK, NT> os;
  if (p.rcos != nullptr)
    os.copy_out_rope(smem, head_ptr_w<T>(p.dq1, b, hd), p.dq1.st, m0, T_ - m0, p.rcos, p.rsin, (int64_t)b * T_ + m0);
  else
    os.copy_out(smem, head_ptr_w<T>(p.dq1, b, hd), p.dq1.st, m0, T_ - m0);
}

// ------------------------------------------------------------------------------------------------ launchers
template <typename T, int POLY, int DK, int DV> hipError_t launch_fwd(const KParams& p, hipStream_t st) {
  if constexpr (!dims_built(sizeof(T) == 4, POLY, DK, DV)) return hipErrorInvalidValue;
  else {
  typedef Cfg<T, POLY, DK, DV> C;
  constexpr int BM = C::FW_NW * C::FW_QW * 32;
  const int grid = p.B * p.H * ((p.T + BM - 1) / BM);
  hipLaunchKernelGGL((k_fwd<T, POLY, DK, DV, C::FW_NW, C::FW_QW, C::FW_BN, C::FW_WPE>), dim3(grid), dim3(C::FW_NW * 64), 0, st, p);
  return hipGetLastError();
  }
}

template <typename T, int POLY, int DK, int DV> hipError_t launch_bwd_kv(const KParams& p, hipStream_t st) {
  if constexpr (!dims_built(sizeof(T) == 4, POLY, DK, DV)) return hipErrorInvalidValue;
  else {
  typedef Cfg<T, POLY, DK, DV> C;
  static_assert(C::KV_KEYS == (C::KV_SPLIT && !C::BIG ? 256 : 128), "dK/dV block size mirrors kv_block_keys()");
  if constexpr (kv_pair_cfg<T, POLY, DK, DV>()) {
    const int grid = p.B * p.H * ((p.T + 127) / 128);
    hipLaunchKernelGGL((k_bwd_kv_pair<T, POLY, DK, DV>), dim3(grid), dim3(512), 0, st, p);
    return hipGetLastError();
  }
  const int grid = p.B * p.H * ((p.T + C::KV_KEYS - 1) / C::KV_KEYS);
  if constexpr (C::KV_SPLIT) {
    if (p.kvsel & 1)
      hipLaunchKernelGGL((k_bwd_kv<T, POLY, DK, DV, C::KV_NW, C::KV_KW, C::KV_BM, C::KV_SPLIT_WPE, KV_DV>), dim3(grid),
                         dim3(C::KV_NW * 64), 0, st, p);
    if (p.kvsel & 2) {
      if constexpr (C::PAIRSPLIT) {
        hipLaunchKernelGGL((k_bwd_kv<T, POLY, DK, DV, C::KV_NW, C::KV_KW, C::KV_BM, C::KV_SPLIT_WPE, KV_DK1>),
                           dim3(grid), dim3(C::KV_NW * 64), 0, st, p);
        hipLaunchKernelGGL((k_bwd_kv<T, POLY, DK, DV, C::KV_NW, C::KV_KW, C::KV_BM, C::KV_SPLIT_WPE, KV_DK2>),
                           dim3(grid), dim3(C::KV_NW * 64), 0, st, p);
      } else {
        hipLaunchKernelGGL((k_bwd_kv<T, POLY, DK, DV, C::KV_NW, C::KV_KW, C::KV_BM, C::KV_SPLIT_WPE, KV_DK>),
                           dim3(grid), dim3(C::KV_NW * 64), 0, st, p);
      }
    }
  } else {
    hipLaunchKernelGGL((k_bwd_kv<T, POLY, DK, DV, C::KV_NW, C::KV_KW, C::KV_BM, C::KV_WPE, KV_BOTH>), dim3(grid),
                       dim3(C::KV_NW * 64), 0, st, p);
  }
  return hipGetLastError();
  }
}

template <typename T, int POLY, int DK, int DV> hipError_t launch_bwd_q(const KParams& p, hipStream_t st) {
  if constexpr (!dims_built(sizeof(T) == 4, POLY, DK, DV)) return hipErrorInvalidValue;
  else {
  typedef Cfg<T, POLY, DK, DV> C;
  constexpr int BM = C::BQ_NW * C::BQ_QW * 32;
  const int grid = p.B * p.H * ((p.T + BM - 1) / BM);
  if constexpr (C::PAIRSPLIT) {
    hipLaunchKernelGGL((k_bwd_q<T, POLY, DK, DV, C::BQ_NW, C::BQ_QW, C::BQ_BN, C::BQ_WPE, 0>), dim3(grid),
                       dim3(C::BQ_NW * 64), 0, st, p);
    hipLaunchKernelGGL((k_bwd_q<T, POLY, DK, DV, C::BQ_NW, C::BQ_QW, C::BQ_BN, C::BQ_WPE, 1>), dim3(grid),
                       dim3(C::BQ_NW * 64), 0, st, p);
  } else {
    hipLaunchKernelGGL((k_bwd_q<T, POLY, DK, DV, C::BQ_NW, C::BQ_QW, C::BQ_BN, C::BQ_WPE>), dim3(grid),
                       dim3(C::BQ_NW * 64), 0, st, p);
  }
  return hipGetLastError();
  }
}

template <typename T, int DK> hipError_t launch_bwd_q_ds(const KParams& p, hipStream_t st) {
  if constexpr (sizeof(T) == 2 && DK == 128) {
    constexpr int NW = 8, BN = 64, BM = NW * 32;
    const int grid = p.B * p.H * ((p.T + BM - 1) / BM);
    hipLaunchKernelGGL((k_bwd_q_ds<T, DK, NW, BN>), dim3(grid), dim3(NW * 64), 0, st, p);
    return hipGetLastError();
  } else {
    return hipErrorInvalidValue;
  }
}

}  // namespace tnpa
