// Decode-kernel instantiations for one (activation dtype, weight format) pair, selected by
// -DE4B_INST_DT=<e4b_dtype> -DE4B_INST_FMT=<e4b_format> (the build compiles this file once per
// pair, in parallel).
#include "decode.h"
#include "decode_launch.h"

#include <algorithm>
#include <atomic>

#ifndef E4B_INST_DT
#error "E4B_INST_DT must be defined"
#endif
#ifndef E4B_INST_FMT
#error "E4B_INST_FMT must be defined"
#endif

namespace e4b {

namespace {

// compute units of the current device, read once per device (threads racing on the first
// read store the same value)
int device_cus() {
  static std::atomic<int> cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int c = cus[dev].load(std::memory_order_relaxed);
  if (c == 0) {
    int v = 0;
    c = (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) ? v : 256;
    cus[dev].store(c, std::memory_order_relaxed);
  }
  return c;
}

template <int DT, int FMT, int G, int CPL, bool FULL, int LR>
void up_gc(const DecodeArgs& a, int64_t max_active, hipStream_t s) {
  constexpr int cols_per_block = kDecWaves * (kWave / G);
  dim3 grid(static_cast<unsigned>((a.n_out + cols_per_block - 1) / cols_per_block), static_cast<unsigned>(max_active));
  if (is_gated(a.epi))
    hipLaunchKernelGGL((decode_up_kernel<DT, FMT, G, CPL, FULL, true, LR>), grid, dim3(kDecThreads), 0, s, a);
  else
    hipLaunchKernelGGL((decode_up_kernel<DT, FMT, G, CPL, FULL, false, LR>), grid, dim3(kDecThreads), 0, s, a);
}

// item kernel: one block per CU (its LDS holds one block), no more blocks than items / waves
template <int DT, int FMT, int G, int CPL, bool FULL, int LR>
void up_items_gc(const DecodeArgs& a, int64_t max_active, hipStream_t s) {
  constexpr int cols_per_item = kWave / G;
  const int64_t items = max_active * ((a.n_out + cols_per_item - 1) / cols_per_item);
  const int64_t blocks = std::min<int64_t>(device_cus(), (items + kItemWaves - 1) / kItemWaves);
  dim3 grid(static_cast<unsigned>(std::max<int64_t>(blocks, 1)));
  if (is_gated(a.epi))
    hipLaunchKernelGGL((decode_up_items_kernel<DT, FMT, G, CPL, FULL, true, LR>), grid, dim3(kItemThreads), 0, s, a);
  else
    hipLaunchKernelGGL((decode_up_items_kernel<DT, FMT, G, CPL, FULL, false, LR>), grid, dim3(kItemThreads), 0, s, a);
}

template <int DT, int FMT, int G, int CPL, int JOBS, bool FULL, int LR>
void down_gc(const DecodeArgs& a, hipStream_t s) {
  dim3 grid(static_cast<unsigned>((a.w.n + kDownCols - 1) / kDownCols));
  hipLaunchKernelGGL((decode_down_kernel<DT, FMT, G, CPL, JOBS, FULL, LR>), grid, dim3(kDecThreads), 0, s, a);
}

}  // namespace

template <int DT, int FMT, int LR>
void launch_decode_up_l(const DecodeArgs& a, DecShape d, int64_t max_active, hipStream_t s) {
  const bool items = decode_up_items(a.tokens, a.w.k);
#define E4B_UP(g, c)                                                                \
  if (d.G == g && d.CPL == c) {                                                     \
    if (items && d.full) up_items_gc<DT, FMT, g, c, true, LR>(a, max_active, s);  \
    else if (items) up_items_gc<DT, FMT, g, c, false, LR>(a, max_active, s);      \
    else if (d.full) up_gc<DT, FMT, g, c, true, LR>(a, max_active, s);            \
    else up_gc<DT, FMT, g, c, false, LR>(a, max_active, s);                       \
    return;                                                                         \
  }
  E4B_UP(4, 2) E4B_UP(4, 4) E4B_UP(8, 4) E4B_UP(16, 4) E4B_UP(16, 6) E4B_UP(32, 4)
#undef E4B_UP
}

template <int DT, int FMT>
void launch_decode_up(const DecodeArgs& a, DecShape d, int64_t max_active, hipStream_t s) {
  if constexpr (FMT != E4B_FMT_MXFP4) {  // LoRA wraps the NF4 bases only
    if (a.lt && a.lr <= 16) return launch_decode_up_l<DT, FMT, 16>(a, d, max_active, s);
    if (a.lt) return launch_decode_up_l<DT, FMT, kDecLoraMaxRank>(a, d, max_active, s);
  }
  launch_decode_up_l<DT, FMT, 0>(a, d, max_active, s);
}

template <int DT, int FMT, int LR>
void launch_decode_down_l(const DecodeArgs& a, DecShape d, hipStream_t s) {
#define E4B_DOWN(g, c, j)                                               \
  if (d.G == g && d.CPL == c && d.JOBS == j) {                          \
    if (d.full) down_gc<DT, FMT, g, c, j, true, LR>(a, s);            \
    else down_gc<DT, FMT, g, c, j, false, LR>(a, s);                  \
    return;                                                             \
  }
  E4B_DOWN(16, 1, 2) E4B_DOWN(32, 1, 1) E4B_DOWN(32, 2, 1) E4B_DOWN(32, 3, 1)
  E4B_DOWN(32, 4, 1)
#undef E4B_DOWN
}

template <int DT, int FMT>
void launch_decode_down(const DecodeArgs& a, DecShape d, hipStream_t s) {
  if constexpr (FMT != E4B_FMT_MXFP4) {  // LoRA wraps the NF4 bases only
    if (a.lt && a.lr <= 16) return launch_decode_down_l<DT, FMT, 16>(a, d, s);
    if (a.lt) return launch_decode_down_l<DT, FMT, kDecLoraMaxRank>(a, d, s);
  }
  launch_decode_down_l<DT, FMT, 0>(a, d, s);
}

template void launch_decode_up<E4B_INST_DT, E4B_INST_FMT>(const DecodeArgs&, DecShape, int64_t, hipStream_t);
template void launch_decode_down<E4B_INST_DT, E4B_INST_FMT>(const DecodeArgs&, DecShape, hipStream_t);

}  // namespace e4b
