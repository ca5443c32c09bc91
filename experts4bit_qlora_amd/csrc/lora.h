// Low-rank (LoRA) delta on the expert-sorted rows of a grouped projection, on the device.
//
// For sorted row m of expert e (offsets[e] <= m < offsets[e + 1]) and output column n:
//   out[m, n] += odt( scaling * sum_j t[m, j] * B[e, n, j] ),  t[m, j] = sum_c x_m[c] * A[e, j, c]
// where x_m is the row's input (token row sorted_flat[m] / gather_k of x when gather_k > 0, else
// row m), A is [E, r, in], B is [E, out, r] (adapter dtype bf16, fp16 or fp32), t and the sums
// are fp32, and odt is the compute dtype the delta is rounded to before it is added -- the
// `(scaling * F.linear(F.linear(x, A), B)).to(x.dtype)` of lora.py:251-256 applied per expert
// group as fast.py:229-233 / 249-253 do, in one pass over all groups: no group sizes on the host.
//
//   lora_a_kernel      one wave per sorted row: the r dot products of length `in`, 8 values per
//                      lane per step, then one wave reduction per rank.
//   lora_b_add_kernel  one thread per (row, output column): r multiply-adds, rounded once, added.
#pragma once

#include "common.h"

namespace e4b {

constexpr int kLoraMaxRank = 64;
constexpr int kLoraThreads = 256;

// Expert of sorted row m: the last e with offsets[e] <= m (offsets staged in LDS).
E4B_DEV int row_expert(const int* offs, int E, int m) {
  int lo = 0, hi = E;  // offs[lo] <= m < offs[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (offs[mid] <= m) lo = mid;
    else hi = mid;
  }
  return lo;
}

// Eight consecutive values of a row in dtype ADT starting at element c (c a multiple of 8).
template <int ADT>
E4B_DEV void load8(const void* base, int64_t c, float (&v)[8]) {
  if constexpr (ADT == E4B_FP32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + c);
    const float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + c);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = lo_f<ADT>(w[i]);
      v[2 * i + 1] = hi_f<ADT>(w[i]);
    }
  }
}

E4B_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// t[m, :r] for every sorted row m < offsets[E] (rows past it, dropped ids, are left alone).
// `in` is a multiple of 8.
template <int XDT, int ADT>
__global__ void __launch_bounds__(kLoraThreads) lora_a_kernel(const uint16_t* __restrict__ x, int gather_k,
                                                              const int32_t* __restrict__ sorted_flat,
                                                              const int32_t* __restrict__ offsets, int E,
                                                              const void* __restrict__ A, int r, int64_t in,
                                                              float* __restrict__ t, int64_t M) {
  __shared__ int offs[1025];
  for (int i = threadIdx.x; i <= E; i += blockDim.x) offs[i] = offsets[i];
  __syncthreads();
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t m = int64_t(blockIdx.x) * (kLoraThreads / kWave) + threadIdx.x / kWave;
  if (m >= M || m >= offs[E]) return;  // whole wave; no barrier follows
  const int e = row_expert(offs, E, static_cast<int>(m));
  const int64_t src = gather_k > 0 ? sorted_flat[m] / gather_k : m;
  const uint16_t* xr = x + src * in;
  const int64_t a_row = in;  // elements per rank row of A
  const char* Ae = static_cast<const char*>(A) + int64_t(e) * r * in * (ADT == E4B_FP32 ? 4 : 2);
  float acc[kLoraMaxRank];
#pragma unroll
  for (int j = 0; j < kLoraMaxRank; ++j) acc[j] = 0.0f;
  for (int64_t c = int64_t(lane) * 8; c < in; c += kWave * 8) {
    float xv[8];
    load8<XDT>(xr, c, xv);
#pragma unroll
    for (int j = 0; j < kLoraMaxRank; ++j) {
      if (j < r) {
        float av[8];
        load8<ADT>(Ae + j * a_row * (ADT == E4B_FP32 ? 4 : 2), c, av);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[j] = __builtin_fmaf(xv[i], av[i], acc[j]);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < kLoraMaxRank; ++j) {
    if (j < r) {
      const float s = wave_sum(acc[j]);
      if (lane == 0) t[m * r + j] = s;
    }
  }
}

// out[m, n] += odt(scaling * t[m, :] . B[e, n, :]) for the sorted rows m = m0 + blockIdx.y below
// offsets[E]; t and out point at row m0, and `rows` bounds this launch's rows.
template <int ADT, int ODT>
__global__ void __launch_bounds__(kLoraThreads) lora_b_add_kernel(const float* __restrict__ t,
                                                                  const int32_t* __restrict__ offsets, int E,
                                                                  const void* __restrict__ B, int r, int64_t nout,
                                                                  float scaling, float* __restrict__ out,
                                                                  int64_t rows, int64_t m0) {
  __shared__ int offs[1025];
  for (int i = threadIdx.x; i <= E; i += blockDim.x) offs[i] = offsets[i];
  __syncthreads();
  const int64_t ml = blockIdx.y;
  const int64_t m = m0 + ml;
  const int64_t n = int64_t(blockIdx.x) * kLoraThreads + threadIdx.x;
  if (ml >= rows || m >= offs[E] || n >= nout) return;
  const int e = row_expert(offs, E, static_cast<int>(m));
  const float* tm = t + ml * r;
  float s = 0.0f;
  if constexpr (ADT == E4B_FP32) {
    const float* b = static_cast<const float*>(B) + (int64_t(e) * nout + n) * r;
    for (int j = 0; j < r; ++j) s = __builtin_fmaf(tm[j], b[j], s);
  } else {
    const uint16_t* b = static_cast<const uint16_t*>(B) + (int64_t(e) * nout + n) * r;
    for (int j = 0; j < r; ++j) s = __builtin_fmaf(tm[j], to_f<ADT>(b[j]), s);
  }
  float d = scaling * s;
  if constexpr (ODT != E4B_FP32) d = rnd<ODT>(d);  // the delta's own rounding, then the fp32 add
  out[ml * nout + n] += d;
}

}  // namespace e4b
