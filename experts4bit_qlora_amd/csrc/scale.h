// Power-of-two scales of the fp16 matrix-core mode of the fused forward.
//
// With bf16 activations the MFMA GEMMs can run on fp16 operands instead: three more significant
// bits for the dequantized weights (the largest error term of the bf16 GEMM against an fp32
// reference) at the same matrix-core rate. fp16's range is narrower than bf16's, so operands
// are scaled by powers of two, which is exact and removed from the fp32 sums afterwards:
//   row_exp_kernel       the largest biased exponent of every activation row (one wave per
//                        row) and the row as scaled fp16: the tokens before the gate_up GEMM,
//                        h (in place) before the down GEMM;
//   weight_shift_kernel  per expert, the shift that brings its largest block scale (decoded, for
//                        double quantization) into [2^14, 2^15): computed once per weight version.
#pragma once

#include "common.h"

namespace e4b {

constexpr int kScaleThreads = 256;

E4B_DEV uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) v = max(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), o)));
  return v;
}

// One wave, row `row` of x [rows, k] (bf16, k % 8 == 0): row_exp[row] = the row's largest biased
// exponent, and x16[row] = fp16(x[row] * 2^exp_shift(row_exp[row])) (exact; see
// bf16x2_to_f16x2), a GEMM operand staged once instead of once per output tile. The row's pieces
// stay in registers between the two passes when k <= 64 * 8 * RP. x16 may be x (in place): the
// wave reads every piece of its row for the maximum before it writes any, and writes each piece
// after reading it. RP (16-byte pieces per lane held across the passes) follows the row length
// (row_exp_pieces): a fixed 8 made a 768-value h row issue 8 loads per lane for its 96 pieces, 5
// in 6 of them clamped re-reads. No barrier: a kernel may hand any wave any row.
template <int RP>
E4B_DEV void row_exp_row(const uint16_t* x, int64_t row, int64_t k, int32_t* __restrict__ row_exp, uint16_t* x16) {
  const int lane = threadIdx.x & (kWave - 1);
  const uint4* xr = reinterpret_cast<const uint4*>(x + row * k);
  uint4* yr = reinterpret_cast<uint4*>(x16 + row * k);
  const int64_t pieces = k / 8;
  uint32_t m = 0;
  uint4 v[RP];
#pragma unroll
  for (int j = 0; j < RP; ++j) {
    const int64_t i = lane + int64_t(j) * kWave;
    v[j] = xr[i < pieces ? i : 0];
    m = max(m, bf16_exp_max(v[j]));
  }
  for (int64_t i = lane + int64_t(RP) * kWave; i < pieces; i += kWave) m = max(m, bf16_exp_max(xr[i]));
  m = wave_max_u32(m);
  if (lane == 0) row_exp[row] = static_cast<int32_t>(m >> 7);
  const int d = exp_shift(static_cast<int>(m >> 7));
  auto conv = [&](const uint4& a) {
    return make_uint4(bf16x2_to_f16x2(a.x, d), bf16x2_to_f16x2(a.y, d), bf16x2_to_f16x2(a.z, d),
                      bf16x2_to_f16x2(a.w, d));
  };
#pragma unroll
  for (int j = 0; j < RP; ++j) {
    const int64_t i = lane + int64_t(j) * kWave;
    if (i < pieces) yr[i] = conv(v[j]);
  }
  for (int64_t i = lane + int64_t(RP) * kWave; i < pieces; i += kWave) yr[i] = conv(xr[i]);
}

// row_exp_row over every row, one wave per row (rows / 4 blocks of 256 threads), and zero[0 ..
// nzero) = 0 (grid-stride).
template <int RP>
__global__ void __launch_bounds__(kScaleThreads) row_exp_kernel(const uint16_t* x, int64_t rows,
                                                                int64_t k, int32_t* __restrict__ row_exp,
                                                                uint16_t* x16,
                                                                int32_t* __restrict__ zero, int64_t nzero) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < nzero; i += int64_t(gridDim.x) * blockDim.x)
    zero[i] = 0;
  const int64_t row = int64_t(blockIdx.x) * (kScaleThreads / kWave) + threadIdx.x / kWave;
  if (row >= rows) return;  // whole waves; no barrier follows
  row_exp_row<RP>(x, row, k, row_exp, x16);
}

// Pieces per lane for a row of k values: enough to hold the row (k <= 4096), rounded up to 1, 2,
// 4 or 8.
inline int row_exp_pieces(int64_t k) {
  const int64_t per = (k / 8 + kWave - 1) / kWave;
  return per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : 8;
}

inline void launch_row_exp(const uint16_t* x, int64_t rows, int64_t k, int32_t* row_exp, uint16_t* x16,
                           int32_t* zero, int64_t nzero, hipStream_t s) {
  const unsigned blocks = static_cast<unsigned>((rows + kScaleThreads / kWave - 1) / (kScaleThreads / kWave));
  switch (row_exp_pieces(k)) {
    case 1: hipLaunchKernelGGL(row_exp_kernel<1>, dim3(blocks), dim3(kScaleThreads), 0, s, x, rows, k, row_exp, x16, zero, nzero); break;
    case 2: hipLaunchKernelGGL(row_exp_kernel<2>, dim3(blocks), dim3(kScaleThreads), 0, s, x, rows, k, row_exp, x16, zero, nzero); break;
    case 4: hipLaunchKernelGGL(row_exp_kernel<4>, dim3(blocks), dim3(kScaleThreads), 0, s, x, rows, k, row_exp, x16, zero, nzero); break;
    default: hipLaunchKernelGGL(row_exp_kernel<8>, dim3(blocks), dim3(kScaleThreads), 0, s, x, rows, k, row_exp, x16, zero, nzero); break;
  }
}

// shift[e] = exp_shift(largest biased fp32 exponent of expert e's block scales), NF4 (fp32
// absmax) or NF4_DQ (decoded absmax). Grid (ceil(nb / kShiftSpan), E): each block reduces the
// exponents of kShiftSpan consecutive block scales of expert blockIdx.y (kShiftPer independent
// loads per thread in flight) and folds exp_shift of its maximum into shift[e] with an atomic
// minimum; exp_shift is non-increasing, so the minimum over blocks is exp_shift of the expert's
// maximum, whatever the order. shift must hold kShiftInit first (weight_shift_init_kernel).
// A block past an expert's scales contributes exp_shift(0) = the largest possible value.
constexpr int kShiftPer = 16;
constexpr int64_t kShiftSpan = int64_t(kScaleThreads) * kShiftPer;
constexpr int32_t kShiftInit = 0x7fffffff;

__global__ void __launch_bounds__(kScaleThreads) weight_shift_init_kernel(int32_t* __restrict__ shift, int E) {
  for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < E; e += gridDim.x * blockDim.x) shift[e] = kShiftInit;
}

template <int FMT>
__global__ void __launch_bounds__(kScaleThreads) weight_shift_kernel(e4b_qweight w, int32_t* __restrict__ shift) {
  const int e = blockIdx.y;
  const int64_t nb = w.n * (w.k / 64);
  const int64_t base = int64_t(blockIdx.x) * kShiftSpan + threadIdx.x;
  uint32_t m = 0;
#pragma unroll
  for (int j = 0; j < kShiftPer; ++j) {
    const int64_t b = base + int64_t(j) * kScaleThreads;
    const uint32_t x = (__float_as_uint(nf4_block_scale<FMT>(w, e, b < nb ? b : nb - 1)) >> 23) & 0xffu;
    m = max(m, b < nb ? x : 0u);
  }
  m = wave_max_u32(m);
  if ((threadIdx.x & (kWave - 1)) == 0) atomicMin(&shift[e], exp_shift(static_cast<int>(m)));
}

}  // namespace e4b
