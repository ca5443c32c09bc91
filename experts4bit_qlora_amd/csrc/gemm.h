// Prefill / large-batch grouped GEMM on the bf16 (fp16) matrix cores of gfx950.
//
// One workgroup (4 waves) computes a 64-row x 128-weight-row tile of one expert. Tiles come
// from the route kernel's (expert, first sorted row) list, so skewed expert sizes cost at most
// one partial tile per expert and the grid never depends on host-side counts.
// Per 64-deep K step:
//   * A: 64 routed rows x 64 activations, gathered through sorted_flat when gather_k > 0
//     (the index_select of fast.py:135 fused into the loads) -> LDS;
//   * W: 128 packed rows x 32 bytes -> each thread decodes 32 nibbles with ONE fp32 product
//     code[nib] * scale and one RNE rounding (bit-identical to the reference's dequantized
//     bf16 weight) -> LDS;
//   * 2 x (2 x 4) v_mfma_f32_16x16x32_{bf16,f16} per wave, fp32 accumulators.
// Gated epilogues pair gate row j with up row n/2 + j in the same tile: LDS rows 0..63 hold
// the gate rows of 64 output columns and rows 64..127 their up rows, and a wave's gate and up
// accumulators sit in the same lanes, so SwiGLU runs on registers (fp32) before the only store.
#pragma once

#include "common.h"
#include "dequant.h"
#include "gemv.h"

namespace e4b {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kTileM = 64;
constexpr int kTileNW = 128;  // weight rows per tile
constexpr int kTileK = 64;
constexpr int kLdsPitch = kTileK + 8;  // elements; 144-byte rows keep 16-byte alignment
constexpr int kGemmThreads = 256;

template <int DT>
E4B_DEV f32x4_t mfma_16x16x32(const uint4& a, const uint4& b, const f32x4_t& c) {
  if constexpr (DT == E4B_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
}

template <int DT, int FMT>
__global__ void __launch_bounds__(kGemmThreads) gemm_mfma_kernel(GemmArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t As[kTileM * kLdsPitch];
  __shared__ __attribute__((aligned(16))) uint16_t Ws[kTileNW * kLdsPitch];
  __shared__ float lut[16];

  const int tile = blockIdx.x;
  if (tile >= p.rt.meta[0]) return;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wid = tid / kWave;
  const int wave_m = wid & 1;
  const int wave_n = wid >> 1;
  const int e = p.rt.tiles[2 * tile];
  const int row0 = p.rt.tiles[2 * tile + 1];
  const int row_end = min(row0 + kTileM, p.rt.offsets[e + 1]);
  const bool pair = is_gated(p.epi);
  const int64_t n = p.w.n;
  const int64_t k = p.w.k;
  const int64_t col0 = int64_t(blockIdx.y) * (pair ? kTileNW / 2 : kTileNW);
  if (col0 >= p.n_out) return;

  if (tid < 16) lut[tid] = (FMT == E4B_FMT_MXFP4) ? kFp4E2M1[tid] : p.w.code[tid];

  // A-load assignment: row tid/4, 16 activations at column (tid%4)*16.
  const int ar = tid >> 2;
  const int aseg = (tid & 3) * 16;
  const int r = row0 + ar;
  const bool avalid = r < row_end;
  const int64_t src = avalid ? (p.gather_k > 0 ? p.rt.sorted_flat[r] / p.gather_k : r) : 0;
  const uint16_t* aptr = p.a + src * k + aseg;

  // W-load assignment: LDS row tid/2 (0..127), 32 values of the 64-deep step at (tid%2)*32.
  const int lrow = tid >> 1;
  const int half = tid & 1;
  int64_t grow;
  bool wvalid;
  if (pair) {
    const int64_t jj = col0 + (lrow & 63);
    wvalid = jj < p.n_out;
    grow = (lrow < 64) ? jj : n / 2 + jj;
  } else {
    grow = col0 + lrow;
    wvalid = grow < p.n_out;
  }
  if (!wvalid) grow = 0;
  const uint8_t* wptr = p.w.packed + (int64_t(e) * n + grow) * (k / 2) + half * 16;

  f32x4_t acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  int nbase[4];
#pragma unroll
  for (int ns = 0; ns < 4; ++ns) {
    nbase[ns] = pair ? ((ns < 2) ? wave_n * 32 + ns * 16 : 64 + wave_n * 32 + (ns - 2) * 16)
                     : wave_n * 64 + ns * 16;
  }
  __syncthreads();

  const int64_t ksteps = k / kTileK;
  for (int64_t kb = 0; kb < ksteps; ++kb) {
    uint4 a0 = make_uint4(0, 0, 0, 0), a1 = make_uint4(0, 0, 0, 0);
    if (avalid) {
      const uint4* ap = reinterpret_cast<const uint4*>(aptr + kb * kTileK);
      a0 = ap[0];
      a1 = ap[1];
    }
    uint4 q = make_uint4(0, 0, 0, 0);
    float scale = 0.0f;
    if (wvalid) {
      q = *reinterpret_cast<const uint4*>(wptr + kb * 32);
      if constexpr (FMT == E4B_FMT_MXFP4) {
        const uint8_t* sc = static_cast<const uint8_t*>(p.w.absmax);
        scale = e8m0_to_f32(sc[(int64_t(e) * n + grow) * (k / 32) + kb * 2 + half]);
      } else {
        scale = nf4_block_scale<FMT>(p.w, e, grow * (k / 64) + kb);
      }
    }
    // decode 32 values -> exact DT weights
    uint32_t wv[16];
    const uint32_t words[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int wi = 0; wi < 4; ++wi) {
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t byte = (words[wi] >> (8 * b)) & 0xffu;
        const uint32_t first = (FMT == E4B_FMT_MXFP4) ? (byte & 0xfu) : (byte >> 4);
        const uint32_t second = (FMT == E4B_FMT_MXFP4) ? (byte >> 4) : (byte & 0xfu);
        wv[4 * wi + b] = pack2(from_f<DT>(mul_f32(lut[first], scale)),
                               from_f<DT>(mul_f32(lut[second], scale)));
      }
    }
    uint4* ws = reinterpret_cast<uint4*>(Ws + lrow * kLdsPitch + half * 32);
    ws[0] = make_uint4(wv[0], wv[1], wv[2], wv[3]);
    ws[1] = make_uint4(wv[4], wv[5], wv[6], wv[7]);
    ws[2] = make_uint4(wv[8], wv[9], wv[10], wv[11]);
    ws[3] = make_uint4(wv[12], wv[13], wv[14], wv[15]);
    uint4* as = reinterpret_cast<uint4*>(As + ar * kLdsPitch + aseg);
    as[0] = a0;
    as[1] = a1;
    __syncthreads();

#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int kcol = ks * 32 + (lane >> 4) * 8;
      uint4 av[2], bv[4];
#pragma unroll
      for (int ms = 0; ms < 2; ++ms) {
        av[ms] = *reinterpret_cast<const uint4*>(As + (wave_m * 32 + ms * 16 + (lane & 15)) * kLdsPitch + kcol);
      }
#pragma unroll
      for (int ns = 0; ns < 4; ++ns) {
        bv[ns] = *reinterpret_cast<const uint4*>(Ws + (nbase[ns] + (lane & 15)) * kLdsPitch + kcol);
      }
#pragma unroll
      for (int ms = 0; ms < 2; ++ms)
#pragma unroll
        for (int ns = 0; ns < 4; ++ns) acc[ms][ns] = mfma_16x16x32<DT>(av[ms], bv[ns], acc[ms][ns]);
    }
    __syncthreads();
  }

  // Epilogue: lane holds D[4*(lane/16) + i][lane % 16] of each 16x16 sub-tile.
  const bool has_bias = p.w.bias != nullptr;
  const uint16_t* bias = static_cast<const uint16_t*>(p.w.bias);
#pragma unroll
  for (int ms = 0; ms < 2; ++ms) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rr = row0 + wave_m * 32 + ms * 16 + 4 * (lane >> 4) + i;
      if (rr >= row_end) continue;
      const int64_t orow = int64_t(rr) * p.n_out;
      if (pair) {
#pragma unroll
        for (int ns = 0; ns < 2; ++ns) {
          const int64_t jj = col0 + wave_n * 32 + ns * 16 + (lane & 15);
          if (jj >= p.n_out) continue;
          const float bg = has_bias ? to_f<DT>(bias[int64_t(e) * n + jj]) : 0.0f;
          const float bu = has_bias ? to_f<DT>(bias[int64_t(e) * n + n / 2 + jj]) : 0.0f;
          store_elem<DT>(p, orow + jj, gated(p.epi, acc[ms][ns][i], acc[ms][ns + 2][i], p.alpha, p.limit, bg, bu));
        }
      } else {
#pragma unroll
        for (int ns = 0; ns < 4; ++ns) {
          const int64_t nn = col0 + wave_n * 64 + ns * 16 + (lane & 15);
          if (nn >= p.n_out) continue;
          const float b = has_bias ? to_f<DT>(bias[int64_t(e) * n + nn]) : 0.0f;
          store_elem<DT>(p, orow + nn, single(p.epi, acc[ms][ns][i], b));
        }
      }
    }
  }
}

}  // namespace e4b
