// Grouped MFMA GEMM instantiations for one (activation dtype, weight format) pair, selected by
// -DE4B_INST_DT=<e4b_dtype> -DE4B_INST_FMT=<e4b_format> (the build compiles this file once per
// pair, in parallel).
#include "gemm.h"
#include "gemm_launch.h"
#include "gemm_narrow.h"
#include "gemm_wide.h"
#include "gemm_wide8.h"

#ifndef E4B_INST_DT
#error "E4B_INST_DT must be defined"
#endif
#ifndef E4B_INST_FMT
#error "E4B_INST_FMT must be defined"
#endif

namespace e4b {

namespace {

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// 256-row tiles run a wide kernel (fp16 mode, or MXFP4 with bf16 activations: eight waves of
// 128 x 64; otherwise four of 128 x 128), the others gemm_mfma_kernel.
template <int DT, int FMT, int BM, bool F16C>
void launch_mfma_kernel(const GemmArgs& a, dim3 grid, hipStream_t s) {
  if constexpr (BM == kTileMBig && F16C) {
    if (a.out_f16_shift)  // fp16 down rows (the host asks only for them here and in the narrow kernel)
      hipLaunchKernelGGL((gemm_wide8_kernel<DT, FMT, true, false, true>), grid, dim3(kWide8Threads), 0, s, a);
    else
      hipLaunchKernelGGL((gemm_wide8_kernel<DT, FMT, true>), grid, dim3(kWide8Threads), 0, s, a);
  } else if constexpr (BM == kTileMBig && DT == E4B_BF16 && FMT == E4B_FMT_MXFP4) {
    hipLaunchKernelGGL((gemm_wide8_kernel<DT, FMT, F16C>), grid, dim3(kWide8Threads), 0, s, a);
  } else if constexpr (BM == kTileMBig) {
    hipLaunchKernelGGL((gemm_wide_kernel<DT, FMT, F16C>), grid, dim3(kWideThreads), 0, s, a);
  } else {
    hipLaunchKernelGGL((gemm_mfma_kernel<DT, FMT, BM, F16C>), grid, dim3(gemm_threads(BM)), 0, s, a);
  }
}

// One tile height; the fp16 mode (a.a_exp set: A rows stored as scaled fp16) exists for bf16
// activations with NF4 weights.
template <int DT, int FMT, int BM>
void launch_mfma_bm(const GemmArgs& a, dim3 grid, hipStream_t s) {
  if constexpr (DT == E4B_BF16 && FMT != E4B_FMT_MXFP4) {
    if (a.a_exp) {
      launch_mfma_kernel<DT, FMT, BM, true>(a, grid, s);
      return;
    }
  }
  launch_mfma_kernel<DT, FMT, BM, false>(a, grid, s);
}

// 8 XCDs x ceil(max_tiles / 8) M tiles x n_tiles blocks (tiles of nw weight rows), mapped to
// tiles in the kernel
dim3 gemm_grid(const GemmArgs& a, int64_t nw) {
  const int64_t cols = is_gated(a.epi) ? nw / 2 : nw;
  return dim3(static_cast<unsigned>(kXcds * cdiv(a.rt.max_tiles, kXcds) * cdiv(a.n_out, cols)));
}

}  // namespace

template <int DT, int FMT>
void launch_mfma_gemm(const GemmArgs& a, hipStream_t s) {
  if constexpr (DT == E4B_BF16 && FMT != E4B_FMT_MXFP4) {
    // the LoRA epilogue: fp16 mode, 256-row tiles (wide) or 32-row tiles the narrow kernel takes
    // (the host checks lora_gemm_fits before asking)
    if (a.lt) {
      if (a.rt.tile_m == kTileMBig)
        hipLaunchKernelGGL((gemm_wide8_kernel<DT, FMT, true, true>), gemm_grid(a, kWideTileN), dim3(kWide8Threads), 0,
                           s, a);
      else
        hipLaunchKernelGGL((gemm_narrow_kernel<FMT, true>), gemm_grid(a, kNarrowN), dim3(kNarrowThreads), 0, s, a);
      return;
    }
    // 32-row tiles in the fp16 mode: the narrow kernel, when K is a whole number of its steps
    if (a.rt.tile_m == kTileMSmall && a.a_exp && narrow_fits(a.w.k)) {
      if (a.out_f16_shift)
        hipLaunchKernelGGL((gemm_narrow_kernel<FMT, false, true>), gemm_grid(a, kNarrowN), dim3(kNarrowThreads), 0, s,
                           a);
      else
        hipLaunchKernelGGL((gemm_narrow_kernel<FMT>), gemm_grid(a, kNarrowN), dim3(kNarrowThreads), 0, s, a);
      return;
    }
  }
  const dim3 grid = gemm_grid(a, gemm_tile_nw(a.rt.tile_m));
  if (a.rt.tile_m == kTileMSmall) launch_mfma_bm<DT, FMT, kTileMSmall>(a, grid, s);
  else if (a.rt.tile_m == kTileMBig) launch_mfma_bm<DT, FMT, kTileMBig>(a, grid, s);
  else launch_mfma_bm<DT, FMT, kTileM>(a, grid, s);
}

template void launch_mfma_gemm<E4B_INST_DT, E4B_INST_FMT>(const GemmArgs&, hipStream_t);

}  // namespace e4b
