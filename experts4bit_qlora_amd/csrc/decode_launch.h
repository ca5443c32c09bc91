// Launch-side view of the decode kernels: shape selection (host) and the per-(dtype, format)
// launchers. The launchers are instantiated in decode_inst.hip, compiled once per
// (E4B_INST_DT, E4B_INST_FMT) pair so the decode instantiations build in parallel.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "e4b_amd.h"

namespace e4b {

struct DecodeArgs;

// G lanes per weight row, CPL 16-byte chunks per lane, JOBS routed experts per group in flight
// (down kernel), and whether the row's chunk count is exactly G * CPL. G == 0: unsupported.
struct DecShape {
  int G, CPL, JOBS;
  bool full;
};

inline DecShape dec_finish(int64_t chunks, int G, int CPL, int JOBS) {
  return DecShape{G, CPL, JOBS, chunks == int64_t(G) * CPL};
}

// gate_up: about four chunks per lane (two weight rows per lane).
inline DecShape decode_up_shape(int64_t k) {
  const int64_t c = k / 32;
  if (c <= 8) return dec_finish(c, 4, 2, 1);
  if (c <= 16) return dec_finish(c, 4, 4, 1);
  if (c <= 32) return dec_finish(c, 8, 4, 1);
  if (c <= 64) return dec_finish(c, 16, 4, 1);
  if (c <= 96) return dec_finish(c, 16, 6, 1);
  if (c <= 128) return dec_finish(c, 32, 4, 1);
  return DecShape{0, 0, 0, false};
}

// gate_up over work items (decode_up_items_kernel): 2..8 tokens whose activations fit the
// kernel's 16384-element LDS stage. One token keeps decode_up_kernel, whose blocks each take
// one routed expert for a column tile with the activations staged once.
inline bool decode_up_items(int64_t tokens, int64_t k) { return tokens >= 2 && tokens <= 8 && tokens * k <= 16384; }

// down: a group takes one routed expert for all of the block's columns. 32-lane groups (8 per
// block) whatever the batch, except rows of at most 16 chunks with more than 8 routed rows:
// 16-lane groups, two jobs in flight. (16-lane groups with two chunks per lane were measured at
// bs=8 on OLMoE: 39.6 us against 26 us for 32 lanes x 1 chunk, their 312 VGPRs leaving one wave
// per SIMD.)
inline DecShape decode_down_shape(int64_t k, int64_t M) {
  const int64_t c = k / 32;
  if (c > 128) return DecShape{0, 0, 0, false};
  if (M > 8 && c <= 16) return dec_finish(c, 16, 1, 2);
  const int cpl = c <= 32 ? 1 : c <= 64 ? 2 : c <= 96 ? 3 : 4;
  return dec_finish(c, 32, cpl, 1);
}

template <int DT, int FMT>
void launch_decode_up(const DecodeArgs& a, DecShape d, int64_t max_active, hipStream_t s);

template <int DT, int FMT>
void launch_decode_down(const DecodeArgs& a, DecShape d, hipStream_t s);

#define E4B_DECODE_EXTERN(DT, FMT)                                                                   \
  extern template void launch_decode_up<DT, FMT>(const DecodeArgs&, DecShape, int64_t, hipStream_t); \
  extern template void launch_decode_down<DT, FMT>(const DecodeArgs&, DecShape, hipStream_t);
E4B_DECODE_EXTERN(E4B_BF16, E4B_FMT_NF4)
E4B_DECODE_EXTERN(E4B_BF16, E4B_FMT_NF4_DQ)
E4B_DECODE_EXTERN(E4B_BF16, E4B_FMT_MXFP4)
E4B_DECODE_EXTERN(E4B_FP16, E4B_FMT_NF4)
E4B_DECODE_EXTERN(E4B_FP16, E4B_FMT_NF4_DQ)
E4B_DECODE_EXTERN(E4B_FP16, E4B_FMT_MXFP4)
#undef E4B_DECODE_EXTERN

}  // namespace e4b
