// Kernel parameter block and launcher declarations shared by the C-ABI translation unit and the kernel
// instantiation units (the API unit sees only these declarations, so it compiles no kernel).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tnpa {

enum Kind { KIND_SP = 0, KIND_OS = 1, KIND_LDM = 2, KIND_POW = 3 };
// Compile-time polynomial families, so that no kind or degree test sits in the inner loops: GEN1 = power of another
// degree (1, 3, 5..8; exponent bits applied with selects), GEN2 = lower_degree_mix, SP = signed_product with two
// distinct pairs, POW2 / POW4 = power of degree 2 (also signed_product with shared pairs) / 4, OS = offset_square.
enum Poly { POLY_GEN1 = 0, POLY_GEN2 = 1, POLY_POW2 = 2, POLY_POW4 = 3, POLY_OS = 4, POLY_SP = 5 };
// The families with two q/k pairs (two score products per key).
constexpr bool two_pair_poly(int poly) { return poly == POLY_GEN2 || poly == POLY_SP; }

struct TDesc {
  const void* p;
  int64_t sb, sh, st;  // element strides over batch, head, time; unit stride over the head dim
};

struct KParams {
  TDesc q1, k1, q2, k2, v, o;
  TDesc dout, dq1, dk1, dq2, dk2, dv;
  TDesc dsc;           // row_scale * dout (same shape), read by the dK/dV pass when dpre != 0
  const int* dstart;   // (B, T) first visible key of each query (q + 1 for padding)
  const int* qend;     // (B, T) one past the last query that sees each key
  const float* rscale; // (B, T) row scale n_visible^-p (0 for padding)
  const float* coef;   // (H, 4) lower_degree_mix coefficients or null
  const float* offs;   // (H) offset_square offsets or null
  float* norms;        // (NPAIR, 2, H) max row norms of q and k (forward), or null
  float* dpar;         // (B*H, NNB, 4) per-key-block partial sums for dcoef / db, or null
  void* dstile;        // dS tiles written by the key side and read by the dQ-from-dS kernel, or null (see ds_tile_*)
  void* dstile2;       // the same for the second q/k pair (dS2), or null
  const float* rcos;   // (B, T, dk/2) rotary tables: the dQ / dK epilogues apply the rotation's gradient, or null
                       // (dQ always; dK where rope_dk_epilogue, else a pass after the key side)
  const float* rsin;
  int dpre;            // 1: dsc holds the row-scaled dout; 0: the dK/dV pass scales dout while staging it
  int kvsel;           // key-side kernels to launch: 1 = dV pass, 2 = dK pass, 3 = both (or the combined kernel)
  int B, H, T;
  int kind, deg;
  float sm;  // 1/sqrt(dk)
  float vf;  // factor on forward outputs and dV (sm^p for homogeneous kinds, else 1)
  float gf;  // factor on dQ and dK (p*sm^p, sm^2 or sm)
};

// Head dims above 128 (256): one wave per SIMD, 32-row tiles, split key side (Cfg::BIG).
__host__ __device__ constexpr bool big_dims(int dk, int dv) { return dk > 128 || dv > 128; }

// Whether kernels are built for these head dims (powers of two from 16 to 256 otherwise): not fp32 with two q/k
// pairs above head dim 128, whose two K tiles and V tile of 32 rows at 1 KB each exceed LDS at two buffers.
constexpr bool dims_built(bool f32, int poly, int dk, int dv) { return !(f32 && two_pair_poly(poly) && big_dims(dk, dv)); }

// Whether the key side runs as separate dV and dK passes (16-bit inputs, one q/k pair, a head dim above 64; any
// input with a head dim above 128); mirrors Cfg::KV_SPLIT.
inline bool kv_split(bool f32, int poly, int dk, int dv) {
  return big_dims(dk, dv) || (!f32 && !two_pair_poly(poly) && (dk > 64 || dv > 64));
}

// Whether the key side is the wave-pair kernel k_bwd_kv_pair (16-bit inputs, one q/k pair, head dims 128): one launch
// computing S and dP once per sub-block, in place of the separate dV and dK passes.
constexpr bool kv_pair(bool f32, int poly, int dk, int dv) {
  return !f32 && !two_pair_poly(poly) && dk == 128 && dv == 128;
}
template <typename T, int POLY, int DK, int DV> constexpr bool kv_pair_cfg() {
  return kv_pair(sizeof(T) == 4, POLY, DK, DV);
}

// Whether the key side writes dK as whole rows from LDS, where its epilogue applies the gradient of a rotary
// embedding (copy_out_rope): one q/k pair and no padded head dim (fp32 at head dim 256: its K and V rows do not fit
// LDS together). The other key sides store dK from the accumulators, and the backward rotates it in a pass after
// them. (Every dQ kernel writes whole rows.)
constexpr bool rope_dk_epilogue(bool f32, int poly, int dk, int dv) {
  return !two_pair_poly(poly) && dk >= 32 && dv >= 32 && !(f32 && big_dims(dk, dv));
}

// Keys per dK/dV workgroup (sizes the dcoef/db partials); mirrors Cfg::KV_KEYS: eight waves of 32 keys for the split
// passes up to head dim 128, four waves (or four wave pairs) otherwise.
inline int kv_block_keys(bool f32, int poly, int dk, int dv) {
  return kv_split(f32, poly, dk, dv) && !kv_pair(f32, poly, dk, dv) && !big_dims(dk, dv) ? 256 : 128;
}

// Whether the dK/dV passes scale dO by the row scale themselves at no cost: they stage the dO rows a step ahead and
// apply the factor when writing them to LDS (three-buffer staging; 16-bit inputs, one q/k pair, and 64-row tiles
// of q and dO that split into whole 16-byte chunks per thread: 8*d chunks over 256 threads for head dims up to 64,
// 512 threads up to 128). Then a separate pre-scaling pass costs more than it saves. Mirrors k_bwd_kv's NBUF == 3.
constexpr bool kv_scales_in_pass(bool f32, int poly, int dk, int dv) {
  const int nt = dk <= 64 && dv <= 64 ? 256 : 512;
  return !f32 && !two_pair_poly(poly) && !big_dims(dk, dv) && (8 * dk) % nt == 0 && (8 * dv) % nt == 0;
}

// dS tiles: the masked, row-scaled gradient dS of every 32x32 (query, key) sub-block i >= j of one (b, h) head,
// rounded to the input dtype, 1024 elements each, lower-triangular order (tile i*(i+1)/2 + j), heads one after
// another. Inside a tile, element (key kk, query qq) sits at 512*(qq/16) + 16*kk + qq%16: the dK pass's register
// layout (lane kk + 32*((qq/8)%2) holds queries 8*((qq/8)%2) + 16*c .. +7 of chunk c = qq/16), so each of its two
// 16-byte stores per lane writes one contiguous KiB.
__host__ __device__ inline int ds_tile_rows(int T) { return (T + 31) / 32; }
__host__ __device__ inline int64_t ds_tiles_per_head(int T) {
  const int64_t n = ds_tile_rows(T);
  return n * (n + 1) / 2;
}
inline int64_t ds_tile_bytes(int B, int H, int T, int esize) {
  return (int64_t)B * H * ds_tiles_per_head(T) * 1024 * esize;
}

template <typename T, int POLY, int DK, int DV> hipError_t launch_fwd(const KParams& p, hipStream_t st);
template <typename T, int POLY, int DK, int DV> hipError_t launch_bwd_kv(const KParams& p, hipStream_t st);
template <typename T, int POLY, int DK, int DV> hipError_t launch_bwd_q(const KParams& p, hipStream_t st);
template <typename T, int DK> hipError_t launch_bwd_q_ds(const KParams& p, hipStream_t st);

}  // namespace tnpa
