// Launch-side view of the grouped MFMA GEMM kernels (gemm_mfma_kernel, 128- and 32-row tiles;
// gemm_wide_kernel, 256-row tiles). The launcher is instantiated in gemm_inst.hip, compiled once
// per (E4B_INST_DT, E4B_INST_FMT) pair so the GEMM instantiations build in parallel.
#pragma once

#include <hip/hip_runtime.h>

#include "e4b_amd.h"

namespace e4b {

struct GemmArgs;

// One launch over the tile list a.rt (a.rt.tile_m = 256, 128 or 32 rows per tile): the kernel
// for that tile height, in the fp16 matrix-core mode when a.a_exp is set.
template <int DT, int FMT>
void launch_mfma_gemm(const GemmArgs& a, hipStream_t s);

// Whether a grouped GEMM with a LoRA epilogue (GemmArgs::lt) or fp16 down rows
// (GemmArgs::out_f16_shift) can run: fp16 mode over 256-row tiles (the eight-wave wide kernel), or
// over 32-row tiles with K a whole number of the narrow kernel's step pairs.
inline bool lora_gemm_fits(int tile_m, int64_t k) {
  return tile_m == 256 || (tile_m == 32 && k > 0 && k % 256 == 0 && k <= 256 * 64);
}

#define E4B_GEMM_EXTERN(DT, FMT) extern template void launch_mfma_gemm<DT, FMT>(const GemmArgs&, hipStream_t);
E4B_GEMM_EXTERN(E4B_BF16, E4B_FMT_NF4)
E4B_GEMM_EXTERN(E4B_BF16, E4B_FMT_NF4_DQ)
E4B_GEMM_EXTERN(E4B_BF16, E4B_FMT_MXFP4)
E4B_GEMM_EXTERN(E4B_FP16, E4B_FMT_NF4)
E4B_GEMM_EXTERN(E4B_FP16, E4B_FMT_NF4_DQ)
E4B_GEMM_EXTERN(E4B_FP16, E4B_FMT_MXFP4)
#undef E4B_GEMM_EXTERN

}  // namespace e4b
