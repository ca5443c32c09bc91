// Shared device helpers for the gfx950 frozen-expert MoE kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/e4b_amd.h"

#define E4B_DEV __device__ __forceinline__

namespace e4b {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------------- dtypes
// Activations travel as raw 16-bit patterns; DT selects bf16 (0) or fp16 (1).
template <int DT>
E4B_DEV float to_f(uint16_t v);
template <>
E4B_DEV float to_f<E4B_BF16>(uint16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}
template <>
E4B_DEV float to_f<E4B_FP16>(uint16_t v) {
  return static_cast<float>(__builtin_bit_cast(_Float16, v));
}

// fp32 -> 16-bit, round to nearest even (the rounding torch's .to(dtype) performs).
template <int DT>
E4B_DEV uint16_t from_f(float f);
template <>
E4B_DEV uint16_t from_f<E4B_BF16>(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
template <>
E4B_DEV uint16_t from_f<E4B_FP16>(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

template <int DT>
E4B_DEV float rnd(float f) {
  return to_f<DT>(from_f<DT>(f));
}

// Low / high 16-bit halves of a packed pair of activations as fp32.
template <int DT>
E4B_DEV float lo_f(uint32_t p) {
  return to_f<DT>(static_cast<uint16_t>(p & 0xffffu));
}
template <int DT>
E4B_DEV float hi_f(uint32_t p) {
  return to_f<DT>(static_cast<uint16_t>(p >> 16));
}
template <>
E4B_DEV float lo_f<E4B_BF16>(uint32_t p) {
  return __uint_as_float(p << 16);
}
template <>
E4B_DEV float hi_f<E4B_BF16>(uint32_t p) {
  return __uint_as_float(p & 0xffff0000u);
}

E4B_DEV uint32_t pack2(uint16_t lo, uint16_t hi) {
  return static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
}

// ------------------------------------------------------------- fp16 operands of bf16 data
// Power-of-two shift that puts values whose largest biased exponent (fp32 / bf16 field) is e
// into [2^14, 2^15): below fp16's largest finite value, with fp16's 11 significant bits for
// everything down to 2^-28 of that maximum. Exponents below 20 (|v| < 2^-107) count as 20, so
// the shift and its inverse stay normal fp32 powers of two.
__host__ __device__ inline int exp_shift(int e) { return 141 - (e > 20 ? e : 20); }

// Largest biased exponent among the 8 bf16 values of a 16-byte piece, in bits 7..14.
E4B_DEV uint32_t bf16_exp_max(const uint4& v) {
  auto m2 = [](uint32_t w) { return max(w & 0x7f80u, (w >> 16) & 0x7f80u); };
  return max(max(m2(v.x), m2(v.y)), max(m2(v.z), m2(v.w)));
}

// Two bf16 values times 2^d as an fp16 pair: exact for results of at least 2^-14 (bf16's 8
// significant bits fit fp16's 11) when the results stay below 2^15, which exp_shift of their
// row's (or chunk's) largest exponent guarantees. Round-toward-zero only touches results below
// 2^-14 (at least 2^-28 under the row maximum).
E4B_DEV uint32_t bf16x2_to_f16x2(uint32_t w, int d) {
  const float lo = __builtin_amdgcn_ldexpf(__uint_as_float(w << 16), d);
  const float hi = __builtin_amdgcn_ldexpf(__uint_as_float(w & 0xffff0000u), d);
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
}

// ------------------------------------------------------------------------------ epilogues
// sigmoid(x) = 1 / (1 + 2^(-x log2 e)) on the hardware exp2 and reciprocal (each within 1 ulp):
// a few ulp of fp32 error, far below the bf16 / fp16 rounding every result goes through, for a
// handful of instructions instead of a correctly rounded expf and an IEEE division.
E4B_DEV float sigmoid_f32(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}
E4B_DEV float silu_f32(float x) { return x * sigmoid_f32(x); }

// fp32 product rounded to fp32 before any later conversion. The empty asm hides the product
// from instruction selection, which would otherwise fold a multiply followed by an fp16
// conversion into one v_fma_mix (a single rounding of the exact product) -- the reference
// rounds to fp32 first (code[idx] * absmax), then to the output dtype.
E4B_DEV float mul_f32(float a, float b) {
  float p = a * b;
  asm volatile("" : "+v"(p));
  return p;
}

// Gated activation of one (gate, up) pair, evaluated in fp32 on the fp32 GEMM sums; the
// caller rounds the result once into the activation dtype. The reference rounds at every
// torch op of its epilogue (lora.py:125-127, hot_residency.py:72-80); keeping the fused
// epilogue in registers at fp32 removes those intermediate roundings.
//   SWIGLU        silu(g) * u
//   CLAMP_SWIGLU  silu(min(g, L)) * clamp(u, -L, L)        (L <= 0: no clamp)
//   GPTOSS        g += bg, u += bu, g = min(g, L), u = clamp(u, -L, L),
//                 (u + 1) * (g * sigmoid(alpha * g))
E4B_DEV float gated(int epi, float g, float u, float alpha, float limit, float bg, float bu) {
  if (epi == E4B_EPI_GPTOSS) {
    g = fminf(g + bg, limit);
    u = fminf(fmaxf(u + bu, -limit), limit);
    return (u + 1.0f) * (g * sigmoid_f32(alpha * g));
  }
  if (epi == E4B_EPI_CLAMP_SWIGLU && limit > 0.0f) {
    g = fminf(g, limit);
    u = fminf(fmaxf(u, -limit), limit);
  }
  return silu_f32(g) * u;
}

// Single-output epilogue in fp32: NONE (+ bias, gpt-oss down_proj) or ACT (silu).
E4B_DEV float single(int epi, float p, float b) {
  p = p + b;
  return epi == E4B_EPI_ACT ? silu_f32(p) : p;
}

__host__ __device__ inline bool is_gated(int epi) {
  return epi == E4B_EPI_SWIGLU || epi == E4B_EPI_CLAMP_SWIGLU || epi == E4B_EPI_GPTOSS;
}

// ------------------------------------------------------------------------------ weights
// Per-(expert, row, 64-element block) scale of the NF4 formats.
template <int FMT>
E4B_DEV float nf4_block_scale(const e4b_qweight& w, int e, int64_t block) {
  const int64_t nb = w.n * (w.k / 64);
  if constexpr (FMT == E4B_FMT_NF4) {
    return static_cast<const float*>(w.absmax)[e * nb + block];
  } else {
    const uint8_t q = static_cast<const uint8_t*>(w.absmax)[e * nb + block];
    const int64_t nb2 = (nb + 255) / 256;
    // fp32(fp32(code2[q] * absmax2) + offset): two separately rounded operations.
    const float p = mul_f32(w.code2[q], w.absmax2[e * nb2 + block / 256]);
    return __fadd_rn(p, w.offset[e]);
  }
}

// 2^(s - 127) for an e8m0 byte, exact (s = 0 is the subnormal 2^-127, s = 255 is +inf).
E4B_DEV float e8m0_to_f32(uint32_t s) {
  return s == 0 ? __uint_as_float(0x00400000u) : __uint_as_float(s << 23);
}

}  // namespace e4b
