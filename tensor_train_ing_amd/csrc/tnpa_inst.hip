// Explicit instantiation unit: compiled once per (element type, key head dim) with
//   -DTNPA_INST_T=<__bf16|_Float16|float> -DTNPA_INST_DK=<16|32|64|128|256>
// so that the kernel variants build in parallel translation units.
#include "tnpa_kernels.hpp"

#ifndef TNPA_INST_T
#error "define TNPA_INST_T"
#endif
#ifndef TNPA_INST_DK
#error "define TNPA_INST_DK"
#endif

namespace tnpa {
#define TNPA_INST(POLY, DV)                                                                                  \
  template hipError_t launch_fwd<TNPA_INST_T, POLY, TNPA_INST_DK, DV>(const KParams&, hipStream_t);        \
  template hipError_t launch_bwd_kv<TNPA_INST_T, POLY, TNPA_INST_DK, DV>(const KParams&, hipStream_t);        \
  template hipError_t launch_bwd_q<TNPA_INST_T, POLY, TNPA_INST_DK, DV>(const KParams&, hipStream_t);
#define TNPA_INST_DVS(POLY) \
  TNPA_INST(POLY, 16) TNPA_INST(POLY, 32) TNPA_INST(POLY, 64) TNPA_INST(POLY, 128) TNPA_INST(POLY, 256)
TNPA_INST_DVS(POLY_GEN1)
TNPA_INST_DVS(POLY_GEN2)
TNPA_INST_DVS(POLY_POW2)
TNPA_INST_DVS(POLY_POW4)
TNPA_INST_DVS(POLY_OS)
TNPA_INST_DVS(POLY_SP)
template hipError_t launch_bwd_q_ds<TNPA_INST_T, TNPA_INST_DK>(const KParams&, hipStream_t);
}  // namespace tnpa
