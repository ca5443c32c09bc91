// Decode-path grouped GEMV: few rows per expert, HBM-bandwidth bound.
//
// Work unit: one (active expert, output column) "row slot" per G-lane group. The group streams
// the packed weight row(s) of that column -- for a gated epilogue the gate row j and the up
// row n/2 + j together -- in 16-byte chunks (32 values = half an NF4 block or one MX block),
// decodes nibbles through a per-lane replicated LDS code table (16 codes x 64 lanes: every
// lane reads its own bank, so the lookups never conflict), multiplies against the fp32
// activations of each routed row, and applies the block scale once per chunk:
//     acc += scale * sum_{32 values} code[nib] * x
// Scale factoring is exact for MXFP4 (power-of-two scales) and reassociates the fp32 sum for
// NF4; both accumulate in fp32. The G partial sums reduce with lane shuffles and lane 0 of the
// group runs the fused epilogue (bias, SwiGLU / clamped GLU) in fp32 and stores the result
// rounded once to the activation dtype, or as fp32.
#pragma once

#include "common.h"
#include "dequant.h"

namespace e4b {

struct GemmArgs {
  const uint16_t* a;  // activations [*, k]
  int gather_k;       // > 0: A row of sorted row r is a[sorted_flat[r] / gather_k]
  e4b_qweight w;
  e4b_routing rt;
  int64_t M;          // sorted rows
  int epi;
  float alpha, limit;
  void* out;          // [M, n_out] in the activation dtype, or fp32 when out_f32
  int64_t n_out;
  int out_f32;
  // fp16 matrix-core mode (MFMA kernels, bf16 activations, NF4 weights with w.shift): the A
  // rows are stored as fp16, each scaled by 2^exp_shift(a_exp[row]) (row_exp_kernel), a_exp
  // indexed like the A rows themselves (token when gather_k > 0, else sorted row); NULL selects
  // the bf16 mode.
  const int32_t* a_exp;
  // fp16 mode, down rows (epi NONE, no bias, out_f32 set): > 0 stores each row as fp16 of the
  // scaled accumulator times 2^-out_f16_shift (the operand scales left on) instead of fp32 rows;
  // the combine takes the scales off (combine_kernel's SC form)
  int out_f16_shift;
  // LoRA delta in the epilogue (the LORA instances of the fp16-mode wide and narrow kernels):
  // output column j of sorted row m gains lscale * sum_q lt[m, q] * lb[e, w_row(j), q] before the
  // epilogue, lt the fp32 t = x . A^T rows [M, lr] of the routed rows, lb B [E, w.n, lr] in lbdt.
  const float* lt;
  const void* lb;
  int lbdt, lr;
  float lscale;
};

// Store one output element: fp32, or rounded once into the activation dtype.
template <int DT>
E4B_DEV void store_elem(const GemmArgs& p, int64_t i, float v) {
  if (p.out_f32) {
    static_cast<float*>(p.out)[i] = v;
  } else {
    static_cast<uint16_t*>(p.out)[i] = from_f<DT>(v);
  }
}

constexpr int kGemvThreads = 256;
constexpr int kGemvRowsPerPass = 4;  // routed rows held in registers per weight pass

template <int FMT>
E4B_DEV float chunk_scale(const e4b_qweight& w, int e, int64_t row, int64_t c) {
  if constexpr (FMT == E4B_FMT_MXFP4) {
    const uint8_t* sc = static_cast<const uint8_t*>(w.absmax);
    return e8m0_to_f32(sc[(int64_t(e) * w.n + row) * (w.k / 32) + c]);
  } else {
    return nf4_block_scale<FMT>(w, e, row * (w.k / 64) + c / 2);
  }
}

// 16 packed bytes -> 32 unscaled codes, element order of the format.
template <int FMT>
E4B_DEV void decode_chunk(const uint4& q, const float* lut, int lane, float* v) {
  const uint32_t words[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int wi = 0; wi < 4; ++wi) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t byte = (words[wi] >> (8 * b)) & 0xffu;
      const uint32_t first = (FMT == E4B_FMT_MXFP4) ? (byte & 0xfu) : (byte >> 4);
      const uint32_t second = (FMT == E4B_FMT_MXFP4) ? (byte >> 4) : (byte & 0xfu);
      v[8 * wi + 2 * b] = lut[first * kWave + lane];
      v[8 * wi + 2 * b + 1] = lut[second * kWave + lane];
    }
  }
}

template <int DT>
E4B_DEV float dot32(const float* v, const uint16_t* xrow) {
  const uint4* xp = reinterpret_cast<const uint4*>(xrow);
  float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint4 x = xp[q];
    const uint32_t xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      s0 = fmaf(v[8 * q + 2 * p], lo_f<DT>(xs[p]), s0);
      s1 = fmaf(v[8 * q + 2 * p + 1], hi_f<DT>(xs[p]), s1);
    }
  }
  return s0 + s1;
}

template <int G>
E4B_DEV float group_sum(float v) {
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

template <int DT, int FMT, int G>
__global__ void __launch_bounds__(kGemvThreads) gemv_kernel(GemmArgs p) {
  constexpr int kSlots = kWave / G;
  __shared__ float lut[16 * kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  for (int i = threadIdx.x; i < 16 * kWave; i += kGemvThreads) {
    lut[i] = (FMT == E4B_FMT_MXFP4) ? kFp4E2M1[i / kWave] : p.w.code[i / kWave];
  }
  __syncthreads();

  const int a = blockIdx.y;
  if (a >= p.rt.meta[1]) return;
  const int e = p.rt.active[a];
  const int r0 = p.rt.offsets[e];
  const int r1 = p.rt.offsets[e + 1];
  const bool pair = is_gated(p.epi);
  const int64_t n = p.w.n;
  const int64_t k = p.w.k;
  const int gl = lane % G;
  const int64_t j = (int64_t(blockIdx.x) * (kGemvThreads / kWave) + wid) * kSlots + lane / G;
  if (j >= p.n_out) return;  // whole G-lane groups exit together

  const int64_t row_a = j;
  const int64_t row_b = pair ? j + n / 2 : j;
  const int64_t row_bytes = k / 2;
  const uint8_t* wa = p.w.packed + (int64_t(e) * n + row_a) * row_bytes;
  const uint8_t* wb = p.w.packed + (int64_t(e) * n + row_b) * row_bytes;
  const int64_t nchunk = k / 32;
  const bool has_bias = p.w.bias != nullptr;
  const uint16_t* bias = static_cast<const uint16_t*>(p.w.bias);

  for (int rb = r0; rb < r1; rb += kGemvRowsPerPass) {
    const int m = min(kGemvRowsPerPass, r1 - rb);
    const uint16_t* xrow[kGemvRowsPerPass];
#pragma unroll
    for (int mm = 0; mm < kGemvRowsPerPass; ++mm) {
      const int r = rb + min(mm, m - 1);
      const int64_t src = p.gather_k > 0 ? p.rt.sorted_flat[r] / p.gather_k : r;
      xrow[mm] = p.a + src * k;
    }
    float acc_a[kGemvRowsPerPass], acc_b[kGemvRowsPerPass];
#pragma unroll
    for (int mm = 0; mm < kGemvRowsPerPass; ++mm) acc_a[mm] = acc_b[mm] = 0.0f;

    for (int64_t c = gl; c < nchunk; c += G) {
      const uint4 qa = *reinterpret_cast<const uint4*>(wa + 16 * c);
      const float sa = chunk_scale<FMT>(p.w, e, row_a, c);
      float va[32];
      decode_chunk<FMT>(qa, lut, lane, va);
      if (pair) {
        const uint4 qb = *reinterpret_cast<const uint4*>(wb + 16 * c);
        const float sb = chunk_scale<FMT>(p.w, e, row_b, c);
        float vb[32];
        decode_chunk<FMT>(qb, lut, lane, vb);
#pragma unroll
        for (int mm = 0; mm < kGemvRowsPerPass; ++mm) {
          if (mm < m) {
            acc_a[mm] = fmaf(dot32<DT>(va, xrow[mm] + 32 * c), sa, acc_a[mm]);
            acc_b[mm] = fmaf(dot32<DT>(vb, xrow[mm] + 32 * c), sb, acc_b[mm]);
          }
        }
      } else {
#pragma unroll
        for (int mm = 0; mm < kGemvRowsPerPass; ++mm) {
          if (mm < m) acc_a[mm] = fmaf(dot32<DT>(va, xrow[mm] + 32 * c), sa, acc_a[mm]);
        }
      }
    }
#pragma unroll
    for (int mm = 0; mm < kGemvRowsPerPass; ++mm) {
      acc_a[mm] = group_sum<G>(acc_a[mm]);
      if (pair) acc_b[mm] = group_sum<G>(acc_b[mm]);
    }
    if (gl == 0) {
#pragma unroll
      for (int mm = 0; mm < kGemvRowsPerPass; ++mm) {
        if (mm >= m) continue;
        float v;
        if (pair) {
          const float bg = has_bias ? to_f<DT>(bias[int64_t(e) * n + row_a]) : 0.0f;
          const float bu = has_bias ? to_f<DT>(bias[int64_t(e) * n + row_b]) : 0.0f;
          v = gated(p.epi, acc_a[mm], acc_b[mm], p.alpha, p.limit, bg, bu);
        } else {
          const float b = has_bias ? to_f<DT>(bias[int64_t(e) * n + row_a]) : 0.0f;
          v = single(p.epi, acc_a[mm], b);
        }
        store_elem<DT>(p, int64_t(rb + mm) * p.n_out + j, v);
      }
    }
  }
}

}  // namespace e4b
