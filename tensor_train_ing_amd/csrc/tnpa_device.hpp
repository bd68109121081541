// Device primitives for the CDNA4 (gfx950) causal polynomial attention kernels.
//
// Everything here is written for 64-wide wavefronts and the gfx950 MFMA units:
//   * bf16/fp16 inputs use v_mfma_f32_32x32x16_{bf16,f16}: per lane an 8-element A and B operand, 16 fp32
//     accumulators; fp32 inputs use v_mfma_f32_32x32x2_f32 (one element per lane).
//   * 32x32 accumulator layout (probed on the MI355X): register r of lane l holds row
//     8*(r/4) + 4*(l/32) + r%4, column l%32. Operand layout: lane l supplies row/column l%32 and the K elements
//     EPL*(l/32) .. EPL*(l/32)+EPL-1 of each KC-wide chunk.
//   * An accumulator is reused as the next MFMA's operand without any shuffle: the rows of the tile that is read
//     as the A operand are permuted by `kappa` so that accumulator register r of lane-half h holds K index
//     key_off(r, h) = (r/EPL)*KC + h*EPL + r%EPL, which is exactly the natural operand order.
//   * Operands whose contraction runs along the tile rows are read with ds_read_b64_tr_b16 (gfx950 LDS transpose
//     read): inside each 16-lane group, lanes 4r..4r+3 each supply 4 consecutive elements of row r and lane i
//     receives element i of rows 0..3.
//   * LDS tiles are row-major with a 16-byte-chunk XOR swizzle so that both the row-wise 128-bit reads and the
//     transposed 64-bit reads avoid bank conflicts.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define TNPA_LDS __attribute__((address_space(3)))

namespace tnpa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------------------------------------ MFMA traits
template <typename T> struct Mfma;

template <> struct Mfma<__bf16> {
  static constexpr int KC = 16;  // contraction length of one MFMA
  static constexpr int EPL = 8;  // operand elements per lane
  typedef bf16x8 Op;
  __device__ static inline f32x16 mma(Op a, Op b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static inline Op cvt(const float* f) {
    Op o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = (__bf16)f[j];
    return o;
  }
  __device__ static inline Op zero() {
    Op o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = (__bf16)0.0f;
    return o;
  }
};

template <> struct Mfma<_Float16> {
  static constexpr int KC = 16;
  static constexpr int EPL = 8;
  typedef f16x8 Op;
  __device__ static inline f32x16 mma(Op a, Op b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ static inline Op cvt(const float* f) {
    Op o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = (_Float16)f[j];
    return o;
  }
  __device__ static inline Op zero() {
    Op o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = (_Float16)0.0f;
    return o;
  }
};

template <> struct Mfma<float> {
  static constexpr int KC = 2;
  static constexpr int EPL = 1;
  typedef float Op;
  __device__ static inline f32x16 mma(Op a, Op b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
  __device__ static inline Op cvt(const float* f) { return f[0]; }
  __device__ static inline Op zero() { return 0.0f; }
};

__device__ inline f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

// K index held by accumulator register r of lane-half h once the A-operand rows were read through kappa().
template <typename T> __device__ constexpr inline int key_off(int r, int h) {
  return (r / Mfma<T>::EPL) * Mfma<T>::KC + h * Mfma<T>::EPL + r % Mfma<T>::EPL;
}
// Tile row that lane (l % 32) = i must supply as the A operand so that register r / half h holds key_off(r, h).
template <typename T> __device__ constexpr inline int kappa(int i) {
  return key_off<T>(4 * (i / 8) + i % 4, (i / 4) % 2);
}

// ------------------------------------------------------------------------------------------------ LDS tiles
// Row-major ROWS x WID tile of T (WID a multiple of 32; head dims below 32 are zero padded). Rows are padded by
// 16 bytes and, for 16-bit types, permuted inside each 16-row group by prow(): logical row l is stored at
// 4*(l%4) + 2*((l/8)%2) + (l/4)%2. With that pitch and permutation both access patterns are bank-conflict free:
// the row reads (16 lanes reading 16 different rows of one 16-byte column chunk) and the transposed reads (each
// half-wave reading 4 rows k0+4s+0..3 of 64 bytes, which land 16 banks apart). Every offset is a per-lane base
// plus a compile-time immediate, so the kernels keep one address register per access pattern.
template <typename T, int ROWS, int WID> struct Tile {
  static constexpr int PITCH = WID * (int)sizeof(T) + 16;  // bytes per row
  static constexpr int BYTES = ROWS * PITCH;
  static_assert(WID % 32 == 0, "tile width");
  __device__ static constexpr int prow(int r) {
    if constexpr (sizeof(T) == 2) {
      const int l = r & 15;
      return (r & ~15) | (4 * (l & 3) + 2 * ((l >> 3) & 1) + ((l >> 2) & 1));
    } else {
      return r;
    }
  }
  // byte offset of element (r, col)
  __device__ static inline uint32_t off(int r, int col) { return (uint32_t)(prow(r) * PITCH + col * (int)sizeof(T)); }
};

// A/B operand whose contraction runs along the row (head dim): elements [c*KC + h*EPL, +EPL) of tile row
// rbase + lrow, where rbase is a multiple of 16 shared by the wave and lrow in [0, 32) is per lane.
template <typename T, typename TL>
__device__ inline typename Mfma<T>::Op read_row(const char TNPA_LDS* tile, int rbase, int lrow, int c, int h) {
  typedef typename Mfma<T>::Op Op;
  const int col = c * Mfma<T>::KC + h * Mfma<T>::EPL;
  return *(const Op TNPA_LDS*)(tile + rbase * TL::PITCH + TL::prow(lrow) * TL::PITCH + col * (int)sizeof(T));
}

// A/B operand whose contraction runs down the rows: lane (n = l%32, h) gets tile[k0 + h*EPL + j][col0 + n]
// (k0 a multiple of 16 for 16-bit types).
template <typename T, typename TL>
__device__ inline typename Mfma<T>::Op read_col(const char TNPA_LDS* tile, int k0, int col0, int lane) {
  typedef typename Mfma<T>::Op Op;
  if constexpr (sizeof(T) == 2) {
    // logical rows k0 + 8*hh + 4*s + (i>>2) sit at physical rows k0 + 4*(i>>2) + 2*hh + s
    const int i = lane & 15, g = lane >> 4, hh = lane >> 5;
    const char TNPA_LDS* p = tile + (k0 + 4 * (i >> 2) + 2 * hh) * TL::PITCH + (col0 + 16 * (g & 1) + 4 * (i & 3)) * 2;
    s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((s16x4 TNPA_LDS*)p);
    s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((s16x4 TNPA_LDS*)(p + TL::PITCH));
    s16x8 both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(Op, both);
  } else {
    return *(const float TNPA_LDS*)(tile + (k0 + (lane >> 5)) * TL::PITCH + (col0 + (lane & 31)) * 4);
  }
}

// Operand loaded straight from global memory (kept in registers for the whole kernel): row-major global row
// pointer, elements [c*KC + h*EPL, +EPL).
template <typename T>
__device__ inline typename Mfma<T>::Op load_op(const T* __restrict__ rowp, int c, int h) {
  typedef typename Mfma<T>::Op Op;
  return *(const Op*)(rowp + c * Mfma<T>::KC + h * Mfma<T>::EPL);
}

// ------------------------------------------------------------------------------------------------ staging
// Global -> registers -> LDS copy of a ROWS x D tile (D real columns of a WID-wide LDS tile), 16 bytes per
// access; consecutive threads take consecutive chunks of a row (coalesced). Rows at or past `nvalid` read as
// zero. Optionally scales each row by a per-row factor (used to fold the row scale into dO).
template <typename T, int ROWS, int D, int WID, int NT> struct Stage {
  static constexpr int CE = 16 / (int)sizeof(T);
  static constexpr int NCHG = D / CE;
  static constexpr int TOTAL = ROWS * NCHG;
  static constexpr int PER = (TOTAL + NT - 1) / NT;
  typedef Tile<T, ROWS, WID> TL;
  u32x4 r[PER];

  __device__ inline void load(const T* __restrict__ g, int64_t st, int row0, int nvalid) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int idx = (int)threadIdx.x + i * NT;
      r[i] = u32x4{0u, 0u, 0u, 0u};
      if (TOTAL % NT == 0 || idx < TOTAL) {
        const int rr = idx / NCHG, c = idx % NCHG;
        if (rr < nvalid) r[i] = *(const u32x4*)(g + (int64_t)(row0 + rr) * st + c * CE);
      }
    }
  }
  // same, scaling row rr by scale[row0 + rr]
  __device__ inline void load_scaled(const T* __restrict__ g, int64_t st, int row0, int nvalid,
                                     const float* __restrict__ scale) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int idx = (int)threadIdx.x + i * NT;
      r[i] = u32x4{0u, 0u, 0u, 0u};
      if (TOTAL % NT == 0 || idx < TOTAL) {
        const int rr = idx / NCHG, c = idx % NCHG;
        if (rr < nvalid) {
          u32x4 raw = *(const u32x4*)(g + (int64_t)(row0 + rr) * st + c * CE);
          const float f = scale[row0 + rr];
          if constexpr (sizeof(T) == 2) {
            T* e = reinterpret_cast<T*>(&raw);
#pragma unroll
            for (int j = 0; j < 8; ++j) e[j] = (T)((float)e[j] * f);
          } else {
            float* e = reinterpret_cast<float*>(&raw);
#pragma unroll
            for (int j = 0; j < 4; ++j) e[j] *= f;
          }
          r[i] = raw;
        }
      }
    }
  }
  __device__ inline void store(char TNPA_LDS* tile) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int idx = (int)threadIdx.x + i * NT;
      if (TOTAL % NT == 0 || idx < TOTAL) {
        const int rr = idx / NCHG, c = idx % NCHG;
        *(u32x4 TNPA_LDS*)(tile + TL::off(rr, c * CE)) = r[i];
      }
    }
  }
  // LDS tile -> global rows row0 + rr for rr < nvalid: the reverse of load() + store(), same coalesced chunks.
  __device__ inline void copy_out(const char TNPA_LDS* tile, T* __restrict__ g, int64_t st, int row0, int nvalid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int idx = (int)threadIdx.x + i * NT;
      if (TOTAL % NT == 0 || idx < TOTAL) {
        const int rr = idx / NCHG, c = idx % NCHG;
        if (rr < nvalid) *(u32x4*)(g + (int64_t)(row0 + rr) * st + c * CE) = *(const u32x4 TNPA_LDS*)(tile + TL::off(rr, c * CE));
      }
    }
  }
  // copy_out with the gradient of a rotary embedding applied to every row (ref: tnlm/attention.py:48-51 and its
  // autograd): row rr is token row0 + rr, whose tables start at cs / sn + (trow0 + rr) * D/2. Chunk c of a row pairs
  // with chunk c ^ NCHG/2 (columns j and j + D/2), held by thread idx ^ NCHG/2 = lane ^ NCHG/2 of the same wave;
  // out = (g1 cos + g2 sin, g2 cos - g1 sin) in fp32, each product and sum rounded on its own, then rounded to T.
  // The table loads of RG chunks are issued together before any of them is used (one memory latency per group).
  __device__ inline void copy_out_rope(const char TNPA_LDS* tile, T* __restrict__ g, int64_t st, int row0, int nvalid,
                                       const float* __restrict__ cs, const float* __restrict__ sn, int64_t trow0) const {
#pragma clang fp contract(off)
    static_assert(NT % NCHG == 0 && NCHG >= 2 && NCHG / 2 <= 32, "row chunks within one wave");
    typedef float f32x4_ __attribute__((ext_vector_type(4)));
    constexpr int HC = NCHG / 2, HALF = D / 2, NV = CE / 4, RG = PER < 4 ? PER : 4;
#pragma unroll
    for (int i0 = 0; i0 < PER; i0 += RG) {
      f32x4_ cv[RG][NV], sv[RG][NV];
      u32x4 own[RG], oth[RG];
#pragma unroll
      for (int u = 0; u < RG; ++u) {
        const int idx = (int)threadIdx.x + (i0 + u) * NT;
        const int rr = idx / NCHG, c = idx % NCHG;
        const bool ok = (TOTAL % NT == 0 || idx < TOTAL) && rr < nvalid;
        const int64_t to = (trow0 + (ok ? rr : 0)) * HALF + (c % HC) * CE;
#pragma unroll
        for (int v = 0; v < NV; ++v) {
          cv[u][v] = *(const f32x4_*)(cs + to + 4 * v);
          sv[u][v] = *(const f32x4_*)(sn + to + 4 * v);
        }
        own[u] = u32x4{0u, 0u, 0u, 0u};
        if (TOTAL % NT == 0 || idx < TOTAL) own[u] = *(const u32x4 TNPA_LDS*)(tile + TL::off(rr, c * CE));
#pragma unroll
        for (int e = 0; e < 4; ++e) oth[u][e] = (uint32_t)__shfl_xor((int)own[u][e], HC, 64);
      }
#pragma unroll
      for (int u = 0; u < RG; ++u) {
        const int idx = (int)threadIdx.x + (i0 + u) * NT;
        const int rr = idx / NCHG, c = idx % NCHG;
        if ((TOTAL % NT == 0 || idx < TOTAL) && rr < nvalid) {
          const bool lo = c < HC;
          u32x4 a = lo ? own[u] : oth[u], b = lo ? oth[u] : own[u], res;
          const T* e1 = reinterpret_cast<const T*>(&a);
          const T* e2 = reinterpret_cast<const T*>(&b);
          T* eo = reinterpret_cast<T*>(&res);
#pragma unroll
          for (int j = 0; j < CE; ++j) {
            const float g1 = (float)e1[j], g2 = (float)e2[j], c1 = cv[u][j / 4][j % 4], s1 = sv[u][j / 4][j % 4];
            const float p1 = g1 * c1, p2 = g2 * s1, p3 = g1 * s1, p4 = g2 * c1;
            eo[j] = (T)(lo ? p1 + p2 : p4 - p3);
          }
          *(u32x4*)(g + (int64_t)(row0 + rr) * st + c * CE) = res;
        }
      }
    }
  }
  // Chunk i through a buffer resource over the tile's rows (rows past the resource's end read as zero): one
  // instruction, no address arithmetic or branch, so it can sit between matrix instructions. voff = byte offset of
  // the thread's chunk i inside the tile. Needs TOTAL % NT == 0.
  __device__ inline void load_buf(int i, __amdgpu_buffer_rsrc_t rs, uint32_t voff) {
    r[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)voff, 0, 0));
  }
  // byte offset of the thread's chunk i inside a tile of row stride st (elements)
  __device__ static inline uint32_t chunk_off(int i, int64_t st) {
    const int idx = (int)threadIdx.x + i * NT;
    return (uint32_t)(((int64_t)(idx / NCHG) * st + (idx % NCHG) * CE) * (int64_t)sizeof(T));
  }
  __device__ inline void store_raw(int i, char TNPA_LDS* tile) const {
    const int idx = (int)threadIdx.x + i * NT;
    *(u32x4 TNPA_LDS*)(tile + TL::off(idx / NCHG, (idx % NCHG) * CE)) = r[i];
  }
};

// Buffer resource over rows n1.. of one (b, h) head of row stride st (elements) and D real columns: rows at or
// past T read as zero (the hardware range check), so staged tiles need no clamp or select.
template <typename T>
__device__ inline __amdgpu_buffer_rsrc_t rows_rsrc(const T* base, int64_t st, int n1, int T_, int D) {
  const int64_t rem = n1 < T_ ? ((int64_t)(T_ - 1 - n1) * st + D) * (int64_t)sizeof(T) : 0;
  const int nrec = (int)(rem < 0x7fffffff ? rem : 0x7fffffff);
  return __builtin_amdgcn_make_buffer_rsrc((void*)(base + (int64_t)n1 * st), (short)0, nrec, 0x00020000);
}

// Staging of one streamed tile made of NA tiles of DA columns (part 1) and one tile of DB columns (part 2),
// through buffer loads into registers and 16-byte LDS stores, in two independently placed parts. In LDS the
// A tiles sit at buf + i * TA::BYTES and the B tile after them.
template <typename T, int ROWS, int DA, int DAP, int DB, int DBP, int NT, int NA> struct PartStager {
  typedef Stage<T, ROWS, DA, DAP, NT> SA;
  typedef Stage<T, ROWS, DB, DBP, NT> SB;
  typedef Tile<T, ROWS, DAP> TA;
  static constexpr bool OK = SA::TOTAL % NT == 0 && SB::TOTAL % NT == 0;
  SA sa[NA];
  SB sb;
  uint32_t oa[NA][SA::PER], ob[SB::PER];
  const T* pa[NA];
  const T* pb;
  int64_t sta[NA], stb;
  int T_;

  __device__ inline void init(const T* const* a, const int64_t* ast, const T* b, int64_t bst, int nrows) {
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      pa[i] = a[i];
      sta[i] = ast[i];
#pragma unroll
      for (int k = 0; k < SA::PER; ++k) oa[i][k] = SA::chunk_off(k, ast[i]);
    }
    pb = b;
    stb = bst;
#pragma unroll
    for (int k = 0; k < SB::PER; ++k) ob[k] = SB::chunk_off(k, bst);
    T_ = nrows;
  }
  // The same, one 16-byte chunk per thread at a time: parts 0 .. NPARTS-1, A chunks first.
  static constexpr int NPARTS = NA * SA::PER + SB::PER;
  __device__ inline void load_part(int q, int n1) {
    if (q < NA * SA::PER) {
      const int i = q / SA::PER, k = q % SA::PER;
      sa[i].load_buf(k, rows_rsrc<T>(pa[i], sta[i], n1, T_, DA), oa[i][k]);
    } else {
      const int k = q - NA * SA::PER;
      sb.load_buf(k, rows_rsrc<T>(pb, stb, n1, T_, DB), ob[k]);
    }
  }
  __device__ inline void store_part(int q, char TNPA_LDS* buf) const {
    if (q < NA * SA::PER) {
      const int i = q / SA::PER, k = q % SA::PER;
      sa[i].store_raw(k, buf + i * TA::BYTES);
    } else {
      const int k = q - NA * SA::PER;
      sb.store_raw(k, buf + NA * TA::BYTES);
    }
  }
  // rows n1 .. n1 + ROWS - 1 into registers / registers into an LDS buffer: part 1 = the A tiles, 2 = the B tile
  __device__ inline void load(int part, int n1) {
#pragma unroll
    for (int q = 0; q < NPARTS; ++q)
      if (part & (q < NA * SA::PER ? 1 : 2)) load_part(q, n1);
  }
  __device__ inline void store(int part, char TNPA_LDS* buf) const {
#pragma unroll
    for (int q = 0; q < NPARTS; ++q)
      if (part & (q < NA * SA::PER ? 1 : 2)) store_part(q, buf);
  }
};

// One wave's 32-row accumulator block -> rows rbase .. rbase + 31 of an LDS tile of T: lane (l32, h) holds, for
// row rbase + l32, columns 32 d + 8 g + 4 h + (0..3) in acc[d][4 g + (0..3)]; each is scaled by f and rounded to T.
// Columns at or past ncol are not written. Used to turn the per-lane output layout into coalesced row stores.
template <typename T, typename TL, int ND>
__device__ inline void acc_rows_to_lds(char TNPA_LDS* tile, int rbase, int l32, int h, const f32x16 (&acc)[ND], float f,
                                       int ncol) {
#pragma unroll
  for (int d = 0; d < ND; ++d)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int col = 32 * d + 8 * g + 4 * h;
      if (col >= ncol) continue;
      char TNPA_LDS* q = tile + TL::off(rbase + l32, col);
      if constexpr (sizeof(T) == 2) {
        typedef T T4 __attribute__((ext_vector_type(4)));
        T4 v;
        v[0] = (T)(acc[d][4 * g] * f); v[1] = (T)(acc[d][4 * g + 1] * f);
        v[2] = (T)(acc[d][4 * g + 2] * f); v[3] = (T)(acc[d][4 * g + 3] * f);
        *(T4 TNPA_LDS*)q = v;
      } else {
        *(f32x4 TNPA_LDS*)q = f32x4{acc[d][4 * g] * f, acc[d][4 * g + 1] * f, acc[d][4 * g + 2] * f, acc[d][4 * g + 3] * f};
      }
    }
}

// Stores 4 consecutive output elements (one accumulator register group) converted to T.
template <typename T> __device__ inline void store4(T* __restrict__ p, float a, float b, float c, float d) {
  if constexpr (sizeof(T) == 2) {
    typedef T T4 __attribute__((ext_vector_type(4)));
    T4 v;
    v[0] = (T)a; v[1] = (T)b; v[2] = (T)c; v[3] = (T)d;
    *(T4*)p = v;
  } else {
    *(f32x4*)p = f32x4{a, b, c, d};
  }
}

}  // namespace tnpa
