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
//   lora_a_kernel      tiles of 1 or 8 sorted rows x 16 ranks per block: each A value loaded is
//                      used for every row of the tile that shares its expert.
//   lora_b_add_kernel  tiles of up to 32 rows x 256 output columns per block: t rows in LDS, the
//                      column's B slice in registers, r multiply-adds, rounded once, added.
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

// Wave sums of N per-lane values (N a power of two, <= 64) in N - 1 + log2(64 / N) shuffles:
// each step folds the half of the values that lane bit BIT does not keep into the partner lane's
// kept half. Afterwards v[0] of lane l is the wave sum of value l >> (6 - log2 N).
template <int N, int BIT>
struct WaveFold {
  static E4B_DEV void run(float* v, int lane) {
    if constexpr (N > 1) {
      constexpr int H = N / 2;
      const bool hi = (lane & BIT) != 0;
#pragma unroll
      for (int k = 0; k < H; ++k) {
        const float mine = hi ? v[k + H] : v[k];
        const float other = hi ? v[k] : v[k + H];
        v[k] = mine + __shfl_xor(other, BIT);
      }
      WaveFold<H, BIT / 2>::run(v, lane);
    } else if constexpr (BIT >= 1) {
      v[0] += __shfl_xor(v[0], BIT);
      WaveFold<1, BIT / 2>::run(v, lane);
    }
  }
};

template <int N>
constexpr int ilog2() { return N <= 1 ? 0 : 1 + ilog2<N / 2>(); }

// Rows of one launch tile that share an expert form a segment; sorted rows make every segment
// one contiguous run, found from the LDS-staged offsets: [s, end) with end = min(tile end,
// offsets[e + 1]).
E4B_DEV int64_t segment_end(const int* offs, int e, int64_t mend) {
  return offs[e + 1] < mend ? static_cast<int64_t>(offs[e + 1]) : mend;
}

constexpr int kLoraRanksPerWave = 4;
constexpr int kLoraRanksPerBlock = kLoraRanksPerWave * (kLoraThreads / kWave);  // 16

// t[m, :r] for every sorted row m < offsets[E] (rows past it, dropped ids, are left alone).
// Block b covers rank group b % rgroups (16 ranks, 4 per wave) of the TR-row tile b / rgroups.
// Per segment, each lane loads 8 values of each of its wave's 4 rank rows of A[e] once per
// step and applies them to every row of the segment, so A is read once per tile, not per row;
// the `in` dimension is spread over the 64 lanes (8 values each, coalesced) and reduced across
// the wave at the end. `in` is a multiple of 8.
template <int XDT, int ADT, int TR>
__global__ void __launch_bounds__(kLoraThreads) lora_a_kernel(const uint16_t* __restrict__ x, int gather_k,
                                                              const int32_t* __restrict__ sorted_flat,
                                                              const int32_t* __restrict__ offsets, int E,
                                                              const void* __restrict__ A, int r, int64_t in,
                                                              float* __restrict__ t, int64_t M, int rgroups) {
  __shared__ int offs[1025];
  for (int i = threadIdx.x; i <= E; i += blockDim.x) offs[i] = offsets[i];
  __syncthreads();
  constexpr int kEs = ADT == E4B_FP32 ? 4 : 2;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t tile = blockIdx.x / rgroups;
  const int j0 = static_cast<int>(blockIdx.x % rgroups) * kLoraRanksPerBlock +
                 static_cast<int>(threadIdx.x / kWave) * kLoraRanksPerWave;
  if (j0 >= r) return;  // whole wave; no barrier follows
  const int64_t mbeg = tile * TR;
  int64_t mend = mbeg + TR < M ? mbeg + TR : M;
  if (offs[E] < mend) mend = offs[E];
  for (int64_t s = mbeg; s < mend;) {
    const int e = row_expert(offs, E, static_cast<int>(s));
    const int64_t send = segment_end(offs, e, mend);
    const int nr = static_cast<int>(send - s);  // 1..TR, uniform
    const uint16_t* xr[TR];
#pragma unroll
    for (int i = 0; i < TR; ++i) {
      const int64_t m = s + (i < nr ? i : nr - 1);
      xr[i] = x + (gather_k > 0 ? static_cast<int64_t>(sorted_flat[m] / gather_k) : m) * in;
    }
    const char* Ae = static_cast<const char*>(A) + (int64_t(e) * r + j0) * in * kEs;
    constexpr int kN = TR * kLoraRanksPerWave;  // value i * 4 + q: row i, rank j0 + q
    float acc[kN];
#pragma unroll
    for (int f = 0; f < kN; ++f) acc[f] = 0.0f;
#pragma unroll 2
    for (int64_t c = int64_t(lane) * 8; c < in; c += kWave * 8) {
      float av[kLoraRanksPerWave][8];
#pragma unroll
      for (int q = 0; q < kLoraRanksPerWave; ++q) {
        if (j0 + q < r) {
          load8<ADT>(Ae + int64_t(q) * in * kEs, c, av[q]);
        } else {
#pragma unroll
          for (int u = 0; u < 8; ++u) av[q][u] = 0.0f;
        }
      }
#pragma unroll
      for (int i = 0; i < TR; ++i) {
        if (i < nr) {
          float xv[8];
          load8<XDT>(xr[i], c, xv);
#pragma unroll
          for (int q = 0; q < kLoraRanksPerWave; ++q)
#pragma unroll
            for (int u = 0; u < 8; ++u)
              acc[i * kLoraRanksPerWave + q] = __builtin_fmaf(xv[u], av[q][u], acc[i * kLoraRanksPerWave + q]);
        }
      }
    }
    WaveFold<kN, kWave / 2>::run(acc, lane);
    constexpr int kSh = 6 - ilog2<kN>();
    if ((lane & ((1 << kSh) - 1)) == 0) {
      const int f = lane >> kSh, i = f / kLoraRanksPerWave, q = f % kLoraRanksPerWave;
      if (i < nr && j0 + q < r) t[(s + i) * r + j0 + q] = acc[0];
    }
    s = send;
  }
}

// t[f, j] = sum_c x_f[c] * A[e_f, j, c] over the flat rows f of the decode path, in flat order
// (no routing tables): e_f = ids[f], x_f = row f / gather_k of x (gather_k > 0) or row f; a row
// whose id is outside [0, E) gets t = 0. Block (f, rank quad): wave w takes rank
// 4 * blockIdx.y + w, its lanes spread over `in` 8 values at a time (coalesced), and the wave
// sums at the end. The decode GEMVs add t . B[e, n, :] to their fp32 sums themselves.
template <int XDT, int ADT>
__global__ void __launch_bounds__(kLoraThreads) lora_t_rows_kernel(const uint16_t* __restrict__ x, int gather_k,
                                                                   const int64_t* __restrict__ ids, int E,
                                                                   const void* __restrict__ A, int r, int64_t in,
                                                                   float* __restrict__ t) {
  constexpr int kEs = ADT == E4B_FP32 ? 4 : 2;
  const int f = static_cast<int>(blockIdx.x);
  const int j = static_cast<int>(blockIdx.y) * (kLoraThreads / kWave) + static_cast<int>(threadIdx.x / kWave);
  if (j >= r) return;  // whole wave; no barrier follows
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t id = ids[f];
  float acc = 0.0f;
  if (id >= 0 && id < E) {
    const char* Ar = static_cast<const char*>(A) + (id * r + j) * in * kEs;
    const uint16_t* xr = x + (gather_k > 0 ? f / gather_k : f) * in;
#pragma unroll 4
    for (int64_t c = int64_t(lane) * 8; c < in; c += kWave * 8) {
      float av[8], xv[8];
      load8<ADT>(Ar, c, av);
      load8<XDT>(xr, c, xv);
#pragma unroll
      for (int u = 0; u < 8; ++u) acc = __builtin_fmaf(xv[u], av[u], acc);
    }
  }
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
  if (lane == 0) t[int64_t(f) * r + j] = acc;
}

constexpr int kLoraMaxTileRows = 32;
constexpr int kLoraRowBatch = 8;

// out[m, n] += odt(scaling * t[m, :] . B[e, n, :]) for the sorted rows below offsets[E].
// Block b covers the 256 output columns of column block b % ncb over the `tile_rows` rows of
// tile b / ncb: the tile's t rows are staged in LDS (zero-padded to RB ranks), and per segment
// each thread holds its column's B[e, n, :r] in registers and applies it to every row, so B is
// read once per tile and every access to `out` is coalesced. The rank sum runs in rank order.
template <int ADT, int ODT, int RB>
__global__ void __launch_bounds__(kLoraThreads) lora_b_add_kernel(const float* __restrict__ t,
                                                                  const int32_t* __restrict__ offsets, int E,
                                                                  const void* __restrict__ B, int r, int64_t nout,
                                                                  float scaling, float* __restrict__ out, int64_t M,
                                                                  int tile_rows, int64_t ncb) {
  __shared__ int offs[1025];
  __shared__ float4 ts[kLoraMaxTileRows][RB / 4];
  for (int i = threadIdx.x; i <= E; i += blockDim.x) offs[i] = offsets[i];
  const int64_t tile = blockIdx.x / ncb;
  const int64_t n = (blockIdx.x % ncb) * kLoraThreads + threadIdx.x;
  const int64_t mbeg = tile * tile_rows;
  float* tsf = reinterpret_cast<float*>(&ts[0][0]);
  for (int i = threadIdx.x; i < tile_rows * RB; i += blockDim.x) {
    const int row = i / RB, j = i % RB;
    const int64_t m = mbeg + row;
    tsf[i] = (m < M && j < r) ? t[m * r + j] : 0.0f;
  }
  __syncthreads();
  int64_t mend = mbeg + tile_rows < M ? mbeg + tile_rows : M;
  if (offs[E] < mend) mend = offs[E];
  if (n >= nout) return;  // no barrier follows
  for (int64_t s = mbeg; s < mend;) {
    const int e = row_expert(offs, E, static_cast<int>(s));
    const int64_t send = segment_end(offs, e, mend);
    float bv[RB];
    const int64_t bo = (int64_t(e) * nout + n) * r;
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      if (j < r) {
        if constexpr (ADT == E4B_FP32) bv[j] = static_cast<const float*>(B)[bo + j];
        else bv[j] = to_f<ADT>(static_cast<const uint16_t*>(B)[bo + j]);
      } else {
        bv[j] = 0.0f;
      }
    }
    auto delta = [&](int64_t m) {
      const float4* tr = ts[m - mbeg];
      float acc = 0.0f;
#pragma unroll
      for (int q = 0; q < RB / 4; ++q) {
        const float4 tv = tr[q];
        acc = __builtin_fmaf(tv.x, bv[4 * q], acc);
        acc = __builtin_fmaf(tv.y, bv[4 * q + 1], acc);
        acc = __builtin_fmaf(tv.z, bv[4 * q + 2], acc);
        acc = __builtin_fmaf(tv.w, bv[4 * q + 3], acc);
      }
      float d = scaling * acc;
      if constexpr (ODT != E4B_FP32) d = rnd<ODT>(d);  // the delta's own rounding, then the fp32 add
      return d;
    };
    int64_t m = s;
    for (; m + kLoraRowBatch <= send; m += kLoraRowBatch) {  // the batch's loads go out together
      float o[kLoraRowBatch];
#pragma unroll
      for (int u = 0; u < kLoraRowBatch; ++u) o[u] = out[(m + u) * nout + n];
#pragma unroll
      for (int u = 0; u < kLoraRowBatch; ++u) out[(m + u) * nout + n] = o[u] + delta(m + u);
    }
    for (; m < send; ++m) out[m * nout + n] += delta(m);
    s = send;
  }
}

// The gate_up projection's delta fused with the activation: for the sorted rows below
// offsets[E], g = proj[m, n] + odt(delta[m, n]) and, when gated, u = proj[m, n + nh] +
// odt(delta[m, n + nh]) (the two halves of lora.py's `_epilogue`, `proj.chunk(2, -1)`), then
// h[m, n] = hdt(gated(epi, g, u) or single(epi, g)) for the nh = h columns. Same tiling as
// lora_b_add_kernel; the fp32 projection is read once and never written back.
template <int ADT, int ODT, int HDT, int RB, bool GATED>
__global__ void __launch_bounds__(kLoraThreads) lora_b_epilogue_kernel(
    const float* __restrict__ t, const int32_t* __restrict__ offsets, int E, const void* __restrict__ B, int r,
    int64_t nh, int64_t nout, float scaling, const float* __restrict__ proj, int epi, float limit,
    uint16_t* __restrict__ h, int64_t M, int tile_rows, int64_t ncb) {
  __shared__ int offs[1025];
  __shared__ float4 ts[kLoraMaxTileRows][RB / 4];
  for (int i = threadIdx.x; i <= E; i += blockDim.x) offs[i] = offsets[i];
  const int64_t tile = blockIdx.x / ncb;
  const int64_t n = (blockIdx.x % ncb) * kLoraThreads + threadIdx.x;
  const int64_t mbeg = tile * tile_rows;
  float* tsf = reinterpret_cast<float*>(&ts[0][0]);
  for (int i = threadIdx.x; i < tile_rows * RB; i += blockDim.x) {
    const int row = i / RB, j = i % RB;
    const int64_t m = mbeg + row;
    tsf[i] = (m < M && j < r) ? t[m * r + j] : 0.0f;
  }
  __syncthreads();
  int64_t mend = mbeg + tile_rows < M ? mbeg + tile_rows : M;
  if (offs[E] < mend) mend = offs[E];
  if (n >= nh) return;  // no barrier follows
  constexpr int kHalves = GATED ? 2 : 1;
  for (int64_t s = mbeg; s < mend;) {
    const int e = row_expert(offs, E, static_cast<int>(s));
    const int64_t send = segment_end(offs, e, mend);
    float bv[kHalves][RB];
#pragma unroll
    for (int hf = 0; hf < kHalves; ++hf) {
      const int64_t bo = (int64_t(e) * nout + n + hf * nh) * r;
#pragma unroll
      for (int j = 0; j < RB; ++j) {
        if (j < r) {
          if constexpr (ADT == E4B_FP32) bv[hf][j] = static_cast<const float*>(B)[bo + j];
          else bv[hf][j] = to_f<ADT>(static_cast<const uint16_t*>(B)[bo + j]);
        } else {
          bv[hf][j] = 0.0f;
        }
      }
    }
    for (int64_t m = s; m < send; ++m) {
      const float4* tr = ts[m - mbeg];
      float v[kHalves];
#pragma unroll
      for (int hf = 0; hf < kHalves; ++hf) {
        float acc = 0.0f;
#pragma unroll
        for (int q = 0; q < RB / 4; ++q) {
          const float4 tv = tr[q];
          acc = __builtin_fmaf(tv.x, bv[hf][4 * q], acc);
          acc = __builtin_fmaf(tv.y, bv[hf][4 * q + 1], acc);
          acc = __builtin_fmaf(tv.z, bv[hf][4 * q + 2], acc);
          acc = __builtin_fmaf(tv.w, bv[hf][4 * q + 3], acc);
        }
        float d = scaling * acc;
        if constexpr (ODT != E4B_FP32) d = rnd<ODT>(d);
        v[hf] = proj[m * nout + n + hf * nh] + d;
      }
      float o;
      if constexpr (GATED) o = gated(epi, v[0], v[1], 1.0f, limit, 0.0f, 0.0f);
      else o = single(epi, v[0], 0.0f);
      h[m * nh + n] = from_f<HDT>(o);
    }
    s = send;
  }
}

}  // namespace e4b
