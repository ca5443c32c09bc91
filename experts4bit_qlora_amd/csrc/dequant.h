// Standalone bit-exact dequantization (the parity anchor for the in-GEMM decode).
//
// NF4: W = out_t(code[nib] * absmax[block]) -- one fp32 product, one RNE rounding
//      (bitsandbytes dequantize_4bit as called by _vendor/experts.py:447-457;
//      cold_engine.py:104-115 for the nibble order: element 2j is the HIGH nibble of byte j).
// MXFP4: W = out_t(FP4[nib] * 2^(s-127)), element 2j is the LOW nibble (formats/mxfp4.py:95-97).
//
// One thread decodes one 32-bit word (8 values); a 64-element NF4 block or a 32-element MX
// block never splits a word, so each word has exactly one scale.
#pragma once

#include "common.h"

namespace e4b {

__constant__ float kFp4E2M1[16] = {0.0f, 0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                                   -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

template <int FMT, int OUT>
__global__ void __launch_bounds__(256) dequant_kernel(e4b_qweight w, int expert_begin, int64_t words,
                                                      void* __restrict__ out) {
  const int64_t words_per_expert = w.n * w.k / 8;
  const uint32_t* packed =
      reinterpret_cast<const uint32_t*>(w.packed) + static_cast<int64_t>(expert_begin) * words_per_expert;
  __shared__ float code_s[16];
  if (threadIdx.x < 16) {
    code_s[threadIdx.x] = (FMT == E4B_FMT_MXFP4) ? kFp4E2M1[threadIdx.x] : w.code[threadIdx.x];
  }
  __syncthreads();
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < words;
       i += int64_t(gridDim.x) * blockDim.x) {
    const uint32_t v = packed[i];
    const int e = expert_begin + static_cast<int>(i / words_per_expert);
    const int64_t wi = i % words_per_expert;  // word within this expert
    float scale;
    if constexpr (FMT == E4B_FMT_MXFP4) {
      const uint8_t* sc = static_cast<const uint8_t*>(w.absmax) + int64_t(e) * (w.n * w.k / 32);
      scale = e8m0_to_f32(sc[wi / 4]);  // 8 values per word, 32 per scale
    } else {
      scale = nf4_block_scale<FMT>(w, e, wi / 8);  // 64 values per block
    }
    float vals[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t byte = (v >> (8 * j)) & 0xffu;
      const uint32_t first = (FMT == E4B_FMT_MXFP4) ? (byte & 0xfu) : (byte >> 4);
      const uint32_t second = (FMT == E4B_FMT_MXFP4) ? (byte >> 4) : (byte & 0xfu);
      vals[2 * j] = mul_f32(code_s[first], scale);
      vals[2 * j + 1] = mul_f32(code_s[second], scale);
    }
    if constexpr (OUT == E4B_FP32) {
      float4* o = reinterpret_cast<float4*>(out) + 2 * i;
      o[0] = make_float4(vals[0], vals[1], vals[2], vals[3]);
      o[1] = make_float4(vals[4], vals[5], vals[6], vals[7]);
    } else {
      uint4 o;
      o.x = pack2(from_f<OUT>(vals[0]), from_f<OUT>(vals[1]));
      o.y = pack2(from_f<OUT>(vals[2]), from_f<OUT>(vals[3]));
      o.z = pack2(from_f<OUT>(vals[4]), from_f<OUT>(vals[5]));
      o.w = pack2(from_f<OUT>(vals[6]), from_f<OUT>(vals[7]));
      reinterpret_cast<uint4*>(out)[i] = o;
    }
  }
}

}  // namespace e4b
