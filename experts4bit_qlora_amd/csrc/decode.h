// Decode path (few tokens): the whole MoE layer in two launches, no routing round trip.
//
//   decode_up_kernel    routing of this block's expert in LDS, then gate_up GEMV with the
//                       fused epilogue; writes h[flat, :] (flat = token * k + slot).
//   decode_down_kernel  full routing in LDS, down GEMV over every routed row for a block of
//                       output columns, then the deterministic k-slot combine of those
//                       columns in slot order -- the combine never leaves the block.
//
// Both recompute the (tiny) routing from top_k_index instead of reading a route kernel's
// output, so a layer costs two dependent global round trips per kernel: the ids, then the
// weights and activations.
//
// Weight decode. A 64 KB LDS table holds, for every byte value b, the two codes the byte
// encodes as activation-dtype pairs -- hi = dt(code) and lo = dt(code - hi) -- so hi + lo
// carries the fp32 code to ~16 significant bits; the table is replicated 32 times and a lane
// reads copy (lane % 32), so 32 lanes touch 64 distinct banks. A byte's table address is one
// v_perm_b32 (byte -> bits 8..15, lane copy -> bits 3..7), and each element pair costs one
// ds_read_b64 plus two v_dot2 (hi, lo) against the packed activation pair, which is used as
// loaded (no conversion). The block scale multiplies the fp32 chunk sum once per 32 values.
#pragma once

#include "common.h"
#include "dequant.h"
#include "gemv.h"

namespace e4b {

constexpr int kDecThreads = 256;
constexpr int kDecMaxRows = 512;     // tokens * top_k handled by the decode path
constexpr int kDecMaxExperts = 256;
constexpr int kLutCopies = 32;
constexpr int kDownCols = 4;         // output columns per decode_down block

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

template <int DT>
E4B_DEV float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (DT == E4B_BF16) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c,
                                           false);
  } else {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b), c, false);
  }
}

struct DecodeArgs {
  const uint16_t* x;          // gate_up: hidden [T, K1]; down: h [T*k, K2] (flat rows)
  const int64_t* topk;        // [T, k]
  const void* topk_w;         // [T, k] router weights (down only)
  int wdt;                    // router weight dtype
  int tokens, k, E;
  e4b_qweight w;
  int epi;
  float alpha, limit;
  void* out;                  // gate_up: h [T*k, n_out] act dtype; down: out [T, n] in odt
  int odt;
  int64_t n_out;
};

// LDS pair table: entry (byte, copy) at byte offset byte * 256 + copy * 8. The 16 codes are
// staged in LDS first, so building the 64 KB table costs one global round trip, not one per
// entry.
template <int DT, int FMT>
E4B_DEV void build_pair_table(uint2* lut, const float* codes_s) {
  for (int i = threadIdx.x; i < 256 * kLutCopies; i += blockDim.x) {
    const uint32_t b = static_cast<uint32_t>(i) / kLutCopies;
    const uint32_t first = (FMT == E4B_FMT_MXFP4) ? (b & 0xfu) : (b >> 4);
    const uint32_t second = (FMT == E4B_FMT_MXFP4) ? (b >> 4) : (b & 0xfu);
    const float v1 = codes_s[first];
    const float v2 = codes_s[second];
    const uint16_t h1 = from_f<DT>(v1), h2 = from_f<DT>(v2);
    const uint16_t l1 = from_f<DT>(v1 - to_f<DT>(h1)), l2 = from_f<DT>(v2 - to_f<DT>(h2));
    lut[i] = make_uint2(pack2(h1, h2), pack2(l1, l2));
  }
}

// Codes (and, for double-quant, the 256-entry second-level code) into LDS.
template <int FMT>
E4B_DEV void stage_codes(const e4b_qweight& w, float* codes_s, float* code2_s) {
  if (threadIdx.x < 16) codes_s[threadIdx.x] = (FMT == E4B_FMT_MXFP4) ? kFp4E2M1[threadIdx.x] : w.code[threadIdx.x];
  if constexpr (FMT == E4B_FMT_NF4_DQ) {
    for (int i = threadIdx.x; i < 256; i += blockDim.x) code2_s[i] = w.code2[i];
  }
}

// Scale of the chunk c (32 values) of weight row `row` of expert e; double-quant codes come
// from the LDS copy of code2.
template <int FMT>
E4B_DEV float dec_scale(const e4b_qweight& w, int e, int64_t row, int c, const float* code2_s) {
  if constexpr (FMT == E4B_FMT_MXFP4) {
    const uint8_t* sc = static_cast<const uint8_t*>(w.absmax);
    return e8m0_to_f32(sc[(int64_t(e) * w.n + row) * (w.k / 32) + c]);
  } else if constexpr (FMT == E4B_FMT_NF4) {
    return static_cast<const float*>(w.absmax)[(int64_t(e) * w.n + row) * (w.k / 64) + c / 2];
  } else {
    const int64_t nb = w.n * (w.k / 64);
    const int64_t blk = row * (w.k / 64) + c / 2;
    const uint8_t q = static_cast<const uint8_t*>(w.absmax)[e * nb + blk];
    const int64_t nb2 = (nb + 255) / 256;
    return __fadd_rn(mul_f32(code2_s[q], w.absmax2[e * nb2 + blk / 256]), w.offset[e]);
  }
}

// sum over one 16-byte chunk (32 values) of code * x, unscaled, fp32.
template <int DT, int FMT>
E4B_DEV float chunk_dot(const uint4& q, const uint4* xq, const char* lut_bytes, uint32_t lane_off) {
  const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
  float acc = 0.0f;
#pragma unroll
  for (int wi = 0; wi < 4; ++wi) {
    const uint4 xv = xq[wi];
    const uint32_t xs[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      // address = (byte b of the word) << 8 | lane_off
      const uint32_t addr = __builtin_amdgcn_perm(lane_off, qw[wi], 0x0c0c0004u | (static_cast<uint32_t>(b) << 8));
      const uint2 e = *reinterpret_cast<const uint2*>(lut_bytes + addr);
      acc = dot2<DT>(e.x, xs[b], acc);
      if constexpr (FMT != E4B_FMT_MXFP4) acc = dot2<DT>(e.y, xs[b], acc);  // e2m1 codes are exact: lo == 0
    }
  }
  return acc;
}

template <int G>
E4B_DEV float group_reduce(float v) {
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// One lane's share (CPL chunks, stride G) of the dot products of one activation row with one
// or two weight rows. Every global load of the share is issued before the first use.
template <int DT, int FMT, int G, int CPL, bool PAIR>
E4B_DEV void row_dots(const e4b_qweight& w, int e, int64_t row_a, int64_t row_b, const uint16_t* xr, int gl,
                      const char* lut_bytes, uint32_t lane_off, const float* code2_s, float& acc_a, float& acc_b) {
  const int nchunk = static_cast<int>(w.k / 32);
  const uint8_t* wa = w.packed + (int64_t(e) * w.n + row_a) * (w.k / 2);
  const uint8_t* wb = w.packed + (int64_t(e) * w.n + row_b) * (w.k / 2);
  uint4 qa[CPL], qb[CPL], xv[CPL][4];
  float sa[CPL], sb[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = gl + i * G;
    if (c < nchunk) {
      qa[i] = *reinterpret_cast<const uint4*>(wa + 16 * c);
      if (PAIR) qb[i] = *reinterpret_cast<const uint4*>(wb + 16 * c);
      const uint4* xp = reinterpret_cast<const uint4*>(xr + 32 * c);
#pragma unroll
      for (int q = 0; q < 4; ++q) xv[i][q] = xp[q];
    }
  }
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = gl + i * G;
    if (c < nchunk) {
      sa[i] = dec_scale<FMT>(w, e, row_a, c, code2_s);
      if (PAIR) sb[i] = dec_scale<FMT>(w, e, row_b, c, code2_s);
    }
  }
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = gl + i * G;
    if (c < nchunk) {
      acc_a = fmaf(chunk_dot<DT, FMT>(qa[i], xv[i], lut_bytes, lane_off), sa[i], acc_a);
      if (PAIR) acc_b = fmaf(chunk_dot<DT, FMT>(qb[i], xv[i], lut_bytes, lane_off), sb[i], acc_b);
    }
  }
}

// Routing ids of this launch into LDS: ids[i] = expert of flat row i, or -1 when out of range.
E4B_DEV void load_ids(const DecodeArgs& p, int* ids) {
  const int M = p.tokens * p.k;
  for (int i = threadIdx.x; i < M; i += blockDim.x) {
    const int64_t v = p.topk[i];
    ids[i] = (v >= 0 && v < p.E) ? static_cast<int>(v) : -1;
  }
}

// Wave 0: the a-th active expert (ascending) and its rows in flat order. Returns via LDS.
E4B_DEV void find_expert_rows(const int* ids, int M, int E, int a, int* present, int* sel, int* rows) {
  const int lane = threadIdx.x & (kWave - 1);
  if (threadIdx.x >= kWave) return;
  for (int e = lane; e < E; e += kWave) present[e] = 0;
  __builtin_amdgcn_wave_barrier();
  for (int i = lane; i < M; i += kWave) {
    const int e = ids[i];
    if (e >= 0) present[e] = 1;
  }
  __builtin_amdgcn_wave_barrier();
  int expert = -1, seen = 0;
  for (int base = 0; base < E && expert < 0; base += kWave) {
    const int e = base + lane;
    const unsigned long long m = __ballot(e < E && present[e] != 0);
    const int c = __popcll(m);
    if (a < seen + c) {
      unsigned long long mm = m;  // drop the lowest (a - seen) set bits
      for (int s = 0; s < a - seen; ++s) mm &= mm - 1;
      expert = base + __ffsll(static_cast<long long>(mm)) - 1;
    }
    seen += c;
  }
  int n = 0;
  if (expert >= 0) {
    const unsigned long long below = (lane == 0) ? 0ull : ((~0ull) >> (kWave - lane));
    for (int base = 0; base < M; base += kWave) {
      const int i = base + lane;
      const bool hit = i < M && ids[i] == expert;
      const unsigned long long m = __ballot(hit);
      if (hit) rows[n + __popcll(m & below)] = i;
      n += __popcll(m);
    }
  }
  if (lane == 0) {
    sel[0] = expert;
    sel[1] = n;
  }
}

// gate_up GEMV + fused epilogue for the a-th active expert (blockIdx.y), G lanes per column.
template <int DT, int FMT, int G, int CPL>
__global__ void __launch_bounds__(kDecThreads) decode_up_kernel(DecodeArgs p) {
  __shared__ uint2 lut[256 * kLutCopies];
  __shared__ int ids[kDecMaxRows];
  __shared__ int present[kDecMaxExperts];
  __shared__ int rows[kDecMaxRows];
  __shared__ float codes_s[16];
  __shared__ float code2_s[(FMT == E4B_FMT_NF4_DQ) ? 256 : 1];
  __shared__ int sel[2];
  const int M = p.tokens * p.k;
  load_ids(p, ids);
  stage_codes<FMT>(p.w, codes_s, code2_s);
  __syncthreads();
  build_pair_table<DT, FMT>(lut, codes_s);
  find_expert_rows(ids, M, p.E, blockIdx.y, present, sel, rows);
  __syncthreads();
  const int e = sel[0];
  const int nrows = sel[1];
  if (e < 0) return;

  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  const int gl = lane % G;
  const uint32_t lane_off = static_cast<uint32_t>(lane % kLutCopies) * 8u;
  const char* lut_bytes = reinterpret_cast<const char*>(lut);
  const bool pair = is_gated(p.epi);
  const int64_t n = p.w.n, k = p.w.k;
  const int64_t j = (int64_t(blockIdx.x) * (kDecThreads / kWave) + wid) * (kWave / G) + lane / G;
  if (j >= p.n_out) return;  // whole G-lane groups exit together
  const int64_t row_a = j, row_b = pair ? j + n / 2 : j;
  const bool has_bias = p.w.bias != nullptr;
  const uint16_t* bias = static_cast<const uint16_t*>(p.w.bias);
  const float bg = has_bias ? to_f<DT>(bias[int64_t(e) * n + row_a]) : 0.0f;
  const float bu = has_bias ? to_f<DT>(bias[int64_t(e) * n + row_b]) : 0.0f;

  for (int ri = 0; ri < nrows; ++ri) {
    const int f = rows[ri];
    const uint16_t* xr = p.x + int64_t(f / p.k) * k;
    float acc_a = 0.0f, acc_b = 0.0f;
    if (pair) {
      row_dots<DT, FMT, G, CPL, true>(p.w, e, row_a, row_b, xr, gl, lut_bytes, lane_off, code2_s, acc_a, acc_b);
    } else {
      row_dots<DT, FMT, G, CPL, false>(p.w, e, row_a, row_b, xr, gl, lut_bytes, lane_off, code2_s, acc_a, acc_b);
    }
    acc_a = group_reduce<G>(acc_a);
    if (pair) acc_b = group_reduce<G>(acc_b);
    if (gl == 0) {
      const float v = pair ? gated(p.epi, acc_a, acc_b, p.alpha, p.limit, bg, bu) : single(p.epi, acc_a, bg);
      static_cast<uint16_t*>(p.out)[int64_t(f) * p.n_out + j] = from_f<DT>(v);
    }
  }
}

// down GEMV over every routed row for kDownCols output columns, then the k-slot combine.
template <int DT, int FMT, int G, int CPL>
__global__ void __launch_bounds__(kDecThreads) decode_down_kernel(DecodeArgs p) {
  __shared__ uint2 lut[256 * kLutCopies];
  __shared__ int ids[kDecMaxRows];
  __shared__ int cnt[kDecMaxExperts];
  __shared__ int order[kDecMaxRows];   // flat rows grouped by expert, flat order within
  __shared__ int active[kDecMaxExperts];
  __shared__ int ebeg[kDecMaxExperts + 1];
  __shared__ float res[kDecMaxRows * kDownCols];
  __shared__ float codes_s[16];
  __shared__ float code2_s[(FMT == E4B_FMT_NF4_DQ) ? 256 : 1];
  __shared__ int nact;
  const int M = p.tokens * p.k;
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  load_ids(p, ids);
  stage_codes<FMT>(p.w, codes_s, code2_s);
  for (int e = threadIdx.x; e < p.E; e += blockDim.x) cnt[e] = 0;
  __syncthreads();
  build_pair_table<DT, FMT>(lut, codes_s);
  for (int i = threadIdx.x; i < M; i += blockDim.x) {
    if (ids[i] >= 0) atomicAdd(&cnt[ids[i]], 1);
  }
  __syncthreads();
  if (wid == 0) {
    // active experts ascending + row offsets, then a stable placement of the rows
    int run = 0, na = 0;
    for (int base = 0; base < p.E; base += kWave) {
      const int e = base + lane;
      const int c = e < p.E ? cnt[e] : 0;
      int x = c;  // inclusive scans (row counts, active flags) within the wave
      int act = c > 0;
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) {
        const int y = __shfl_up(x, o);
        const int z = __shfl_up(act, o);
        if (lane >= o) {
          x += y;
          act += z;
        }
      }
      if (e < p.E) ebeg[e] = run + x - c;
      if (c > 0) active[na + act - 1] = e;
      run += __shfl(x, kWave - 1);
      na += __shfl(act, kWave - 1);
    }
    if (lane == 0) {
      ebeg[p.E] = run;
      nact = na;
    }
    __builtin_amdgcn_wave_barrier();
    for (int e = lane; e < p.E; e += kWave) cnt[e] = ebeg[e];  // cursors
    __builtin_amdgcn_wave_barrier();
    const unsigned long long below = (lane == 0) ? 0ull : ((~0ull) >> (kWave - lane));
    for (int base = 0; base < M; base += kWave) {
      const int i = base + lane;
      const int e = i < M ? ids[i] : -1;
      unsigned long long pending = __ballot(e >= 0);
      while (pending) {
        const int leader = __ffsll(static_cast<long long>(pending)) - 1;
        const int e0 = __shfl(e, leader);
        const unsigned long long m = __ballot(e == e0);
        const int c0 = cnt[e0];
        if (e == e0) order[c0 + __popcll(m & below)] = i;
        if (lane == leader) cnt[e0] = c0 + __popcll(m);
        pending &= ~m;
      }
    }
  }
  __syncthreads();

  const int gl = lane % G;
  const uint32_t lane_off = static_cast<uint32_t>(lane % kLutCopies) * 8u;
  const char* lut_bytes = reinterpret_cast<const char*>(lut);
  const int64_t n = p.w.n, k = p.w.k;
  const int64_t col0 = int64_t(blockIdx.x) * kDownCols;
  const bool has_bias = p.w.bias != nullptr;
  const uint16_t* bias = static_cast<const uint16_t*>(p.w.bias);
  const int groups = kDecThreads / G;
  const int group = threadIdx.x / G;
  const int jobs = nact * kDownCols;
  for (int job = group; job < jobs; job += groups) {
    const int ai = job / kDownCols;
    const int cl = job % kDownCols;
    const int64_t col = col0 + cl;
    if (col >= n) continue;  // whole group skips together
    const int e = active[ai];
    const float b = has_bias ? to_f<DT>(bias[int64_t(e) * n + col]) : 0.0f;
    for (int ri = ebeg[e]; ri < ebeg[e + 1]; ++ri) {
      const int f = order[ri];
      float acc = 0.0f, unused = 0.0f;
      row_dots<DT, FMT, G, CPL, false>(p.w, e, col, col, p.x + int64_t(f) * k, gl, lut_bytes, lane_off, code2_s,
                                       acc, unused);
      acc = group_reduce<G>(acc);
      if (gl == 0) res[f * kDownCols + cl] = acc + b;
    }
  }
  __syncthreads();

  // combine: out[t, col] = sum_s res[t*k+s][col] * w[t, s], slots in order, fp32
  for (int i = threadIdx.x; i < p.tokens * kDownCols; i += blockDim.x) {
    const int t = i / kDownCols;
    const int cl = i % kDownCols;
    const int64_t col = col0 + cl;
    if (col >= n) continue;
    float acc = 0.0f;
    for (int s = 0; s < p.k; ++s) {
      const int f = t * p.k + s;
      if (ids[f] < 0) continue;
      float w;
      if (p.wdt == E4B_FP32) w = static_cast<const float*>(p.topk_w)[f];
      else if (p.wdt == E4B_BF16) w = to_f<E4B_BF16>(static_cast<const uint16_t*>(p.topk_w)[f]);
      else w = to_f<E4B_FP16>(static_cast<const uint16_t*>(p.topk_w)[f]);
      acc = __fadd_rn(acc, mul_f32(res[f * kDownCols + cl], w));
    }
    const int64_t o = int64_t(t) * n + col;
    if (p.odt == E4B_FP32) static_cast<float*>(p.out)[o] = acc;
    else if (p.odt == E4B_BF16) static_cast<uint16_t*>(p.out)[o] = from_f<E4B_BF16>(acc);
    else static_cast<uint16_t*>(p.out)[o] = from_f<E4B_FP16>(acc);
  }
}

}  // namespace e4b
