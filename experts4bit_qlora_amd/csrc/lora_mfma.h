// The LoRA delta of a grouped GEMM tile, on the matrix cores, in the tile's fp32 accumulators
// (the LORA instances of gemm_wide_kernel and gemm_narrow_kernel):
//
//   acc[m, j] += lscale * sum_q t[m, q] * B[e, row(j), q]
//
// a rank-r product of the tile's t rows (t = x . A^T, fp32, from lora_a_kernel) and the B rows of
// the tile's weight rows. Both operands are split into bf16 pairs, v = hi + lo with hi = bf16(v)
// and lo = bf16(v - hi) (the subtraction is exact), and the product is formed as hi.hi + lo.hi +
// hi.lo on bf16 MFMAs with fp32 accumulation: every bf16 x bf16 product is exact in fp32 and the
// dropped lo.lo term is below 2^-16 of |t||B|, so the delta carries about 16 significant bits
// (bf16 adapters have lo = 0 and skip the third product). The extra MFMAs are r / 16 x 3 per
// 32 x 32 block (about 2 % of a 256 x 256 gate_up tile's at rank 16): the delta costs no pass
// over the GEMM's output rows. Operands come straight from global memory, once per tile, at the
// tile's start (the accumulators begin as the scaled delta).
#pragma once

#include "gemm.h"

namespace e4b {

// 8 fp32 values -> their bf16 hi and lo halves as two MFMA operand pieces (value 2i in the low
// half of word i).
E4B_DEV void split_bf16x8(const float (&v)[8], uint4& hi, uint4& lo) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    h[i] = cvt_pair<E4B_BF16>(v[2 * i], v[2 * i + 1]);
    l[i] = cvt_pair<E4B_BF16>(v[2 * i] - lo_f<E4B_BF16>(h[i]), v[2 * i + 1] - hi_f<E4B_BF16>(h[i]));
  }
  hi = make_uint4(h[0], h[1], h[2], h[3]);
  lo = make_uint4(l[0], l[1], l[2], l[3]);
}

// 2^e * lscale * t[m, q0 + i] (0 past the rank), i = 0..7, split. With the rank a multiple of 8
// the eight values are two 16-byte loads, else eight element loads.
E4B_DEV void lora_t_piece(const GemmArgs& p, int64_t m, int q0, int e2, uint4& hi, uint4& lo) {
  float v[8];
  const float* t = p.lt + m * p.lr;
  if ((p.lr & 7) == 0) {
    const float4 a = *reinterpret_cast<const float4*>(t + (q0 < p.lr ? q0 : 0));
    const float4 b = *reinterpret_cast<const float4*>(t + (q0 < p.lr ? q0 : 0) + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = t[q0 + i < p.lr ? q0 + i : 0];
  }
  const float sc = __builtin_amdgcn_ldexpf(p.lscale, e2);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = q0 + i < p.lr ? v[i] * sc : 0.0f;
  split_bf16x8(v, hi, lo);
}

// 2^e * B[e, row, q0 + i] (0 past the rank), i = 0..7, from the adapter dtype, split.
E4B_DEV void lora_b_piece(const GemmArgs& p, int ex, int64_t row, int q0, int e2, uint4& hi, uint4& lo) {
  float v[8];
  const int64_t base = (int64_t(ex) * p.w.n + row) * p.lr;
  const int64_t q0c = q0 < p.lr ? q0 : 0;
  if ((p.lr & 7) == 0 && p.lbdt == E4B_FP32) {
    const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(p.lb) + base + q0c);
    const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(p.lb) + base + q0c + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else if ((p.lr & 7) == 0) {
    const uint4 a = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.lb) + base + q0c);
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t l = static_cast<uint16_t>(w[i]), h = static_cast<uint16_t>(w[i] >> 16);
      v[2 * i] = p.lbdt == E4B_BF16 ? to_f<E4B_BF16>(l) : to_f<E4B_FP16>(l);
      v[2 * i + 1] = p.lbdt == E4B_BF16 ? to_f<E4B_BF16>(h) : to_f<E4B_FP16>(h);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t o = base + (q0 + i < p.lr ? q0 + i : 0);
      if (p.lbdt == E4B_FP32) v[i] = static_cast<const float*>(p.lb)[o];
      else if (p.lbdt == E4B_BF16) v[i] = to_f<E4B_BF16>(static_cast<const uint16_t*>(p.lb)[o]);
      else v[i] = to_f<E4B_FP16>(static_cast<const uint16_t*>(p.lb)[o]);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = q0 + i < p.lr ? __builtin_amdgcn_ldexpf(v[i], e2) : 0.0f;
  split_bf16x8(v, hi, lo);
}

// The delta of 32 x 32 accumulator blocks (v_mfma_f32_32x32x16: lane l supplies row / column
// l % 32 and the eight ranks 8 (l / 32) .. of each 16-rank step), scaled like the fp16 mode's
// products: t row of block row ms = min(arow0 + 32 ms, arow_last), times 2^ashift(ms) (its
// activation row's shift, exact); B rows brow[ns], times 2^bshift (the expert's weight shift). Run
// on zeroed accumulators before a tile's main loop, where its loads overlap the tile's first loads
// and few registers are live; the epilogue then removes the scales from the sum.
template <int MS, int NS, class AS>
E4B_DEV void lora_delta_32x32(const GemmArgs& p, f32x16_t (&acc)[MS][NS], int e, int64_t arow0, int64_t arow_last,
                              AS&& ashift, int bshift, const int64_t (&brow)[NS], int lane) {
  const int g8 = 8 * (lane >> 5);
  const bool b_lo = p.lbdt != E4B_BF16;  // a bf16 B has no lo half
  for (int q0 = 0; q0 < p.lr; q0 += 16) {
    uint4 bh[NS], bl[NS];
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) lora_b_piece(p, e, brow[ns], q0 + g8, bshift, bh[ns], bl[ns]);
    static_for<MS>([&](auto ms) {
      uint4 ah, al;
      lora_t_piece(p, min(arow0 + 32 * int(ms), arow_last), q0 + g8, ashift(int(ms)), ah, al);
      static_for<NS>([&](auto ns) {
        acc[ms][ns] = mfma_32x32x16<E4B_BF16>(ah, bh[ns], acc[ms][ns]);
        acc[ms][ns] = mfma_32x32x16<E4B_BF16>(al, bh[ns], acc[ms][ns]);
        if (b_lo) acc[ms][ns] = mfma_32x32x16<E4B_BF16>(ah, bl[ns], acc[ms][ns]);
      });
    });
  }
}

// 16 x 16 accumulator blocks (v_mfma_f32_16x16x32: lane l supplies row / column l % 16 and the
// eight ranks 8 (l / 16) .. of each 32-rank step); t row of block row ms: min(arow0 + 16 ms,
// arow_last); scales as above.
template <int MS, int NS, class AS>
E4B_DEV void lora_delta_16x16(const GemmArgs& p, f32x4_t (&acc)[MS][NS], int e, int64_t arow0, int64_t arow_last,
                              AS&& ashift, int bshift, const int64_t (&brow)[NS], int lane) {
  const int g8 = 8 * (lane >> 4);
  const bool b_lo = p.lbdt != E4B_BF16;
  for (int q0 = 0; q0 < p.lr; q0 += 32) {
    uint4 bh[NS], bl[NS];
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) lora_b_piece(p, e, brow[ns], q0 + g8, bshift, bh[ns], bl[ns]);
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
      uint4 ah, al;
      lora_t_piece(p, min(arow0 + 16 * ms, arow_last), q0 + g8, ashift(ms), ah, al);
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) {
        acc[ms][ns] = mfma_16x16x32<E4B_BF16>(ah, bh[ns], acc[ms][ns]);
        acc[ms][ns] = mfma_16x16x32<E4B_BF16>(al, bh[ns], acc[ms][ns]);
        if (b_lo) acc[ms][ns] = mfma_16x16x32<E4B_BF16>(ah, bl[ns], acc[ms][ns]);
      }
    }
  }
}

}  // namespace e4b

namespace e4b {

// t[m, q] = sum_c x_m[c] * A[e, q, c] for the sorted rows m of every routing tile (one expert per
// tile), on the matrix cores: the t of the fp16-mode LoRA path (rows past the routed ones are not
// written). One workgroup per BM-row part of a tile, one wave per 16 rows, each wave all ranks of
// its rows (NSM 16-rank blocks) on v_mfma_f32_16x16x32_bf16. x rows are bf16 (exact operands); A
// (bf16, fp16 or fp32) is staged per 64-deep chunk in LDS as bf16 hi / lo halves (lo = bf16(a -
// hi), the split of split_bf16x8), so t carries about 16 significant bits of each product of an
// fp32 or fp16 adapter and every product of a bf16 one exactly. The chunks are double-buffered:
// chunk c + 1's A is loaded into registers and its x fragments are loaded while chunk c's MFMAs
// run, one barrier per chunk. The LDS is 8 KB per rank block (4 KB without lo halves), so many
// workgroups share a CU and keep enough x loads in flight.
constexpr int kLoraTK = 64;  // K per chunk
constexpr int kLoraTGroups = kLoraTK / 8;

// LDS element offset of the 16-byte group holding columns 8 g .. 8 g + 7 of rank row q: 128-byte
// rows with the groups XOR-swizzled by q % 8, so the fragment reads of 16 consecutive ranks at one
// group spread over all banks.
E4B_DEV int lora_t_at(int q, int g) { return q * kLoraTK + (((g ^ q) & 7) << 3); }

template <int ADT, int BM, int NSM>
__global__ void __launch_bounds__(BM / 16 * kWave) lora_t_mfma_kernel(const uint16_t* __restrict__ x, int gather_k,
                                                                      e4b_routing rt, const void* __restrict__ A,
                                                                      int rank, int64_t in, float* __restrict__ t) {
  constexpr int NT = BM / 16 * kWave;
  constexpr bool LO = ADT != E4B_BF16;  // bf16 adapters have no lo half
  constexpr int NSTAGE = 16 * NSM * kLoraTGroups;  // 16-byte groups per chunk
  constexpr int SPT = (NSTAGE + NT - 1) / NT;      // staging groups per thread
  __shared__ __align__(16) uint16_t ah[2][16 * NSM * kLoraTK];
  __shared__ __align__(16) uint16_t al[LO ? 2 : 1][LO ? 16 * NSM * kLoraTK : 8];
  const int sub = rt.tile_m / BM;
  const int tile = static_cast<int>(blockIdx.x) / sub;
  if (tile >= rt.meta[0]) return;  // uniform
  const int e = rt.tiles[2 * tile];
  const int row0 = rt.tiles[2 * tile + 1] + (static_cast<int>(blockIdx.x) % sub) * BM;
  const int rows = min(BM, rt.offsets[e + 1] - row0);
  if (rows <= 0) return;  // uniform: a part past the end of its expert's last tile
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & (kWave - 1), w = tid / kWave;
  const int l16 = lane & 15, g = lane >> 4;
  // the lane's x row (clamped to the part's rows; only real rows are stored)
  const int rr = row0 + min(16 * w + l16, rows - 1);
  const int64_t src = gather_k > 0 ? rt.sorted_flat[rr] / gather_k : rr;
  const uint16_t* xr = x + src * in;
  const int nchunks = static_cast<int>(in / kLoraTK);

  // staging: thread tid takes groups j = tid + NT i of the chunk's [16 NSM ranks][8 groups]
  float sv[SPT][8];
  auto load_a = [&](int c) {
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
      const int j = tid + NT * i;
      if (NSTAGE % NT != 0 && j >= NSTAGE) break;
      const int q = min(j / kLoraTGroups, rank - 1), gg = j % kLoraTGroups;
      const int64_t o = (int64_t(e) * rank + q) * in + int64_t(c) * kLoraTK + 8 * gg;
      if constexpr (ADT == E4B_FP32) {
        const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(A) + o);
        const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(A) + o + 4);
        sv[i][0] = a.x; sv[i][1] = a.y; sv[i][2] = a.z; sv[i][3] = a.w;
        sv[i][4] = b.x; sv[i][5] = b.y; sv[i][6] = b.z; sv[i][7] = b.w;
      } else {
        const uint4 a = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(A) + o);
        const uint32_t wv[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          sv[i][2 * h] = to_f<ADT>(static_cast<uint16_t>(wv[h]));
          sv[i][2 * h + 1] = to_f<ADT>(static_cast<uint16_t>(wv[h] >> 16));
        }
      }
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
      const int j = tid + NT * i;
      if (NSTAGE % NT != 0 && j >= NSTAGE) break;
      const int q = j / kLoraTGroups, gg = j % kLoraTGroups;
      float v[8];
#pragma unroll
      for (int h = 0; h < 8; ++h) v[h] = q < rank ? sv[i][h] : 0.0f;
      uint4 hi, lo;
      split_bf16x8(v, hi, lo);
      *reinterpret_cast<uint4*>(&ah[buf][lora_t_at(q, gg)]) = hi;
      if constexpr (LO) *reinterpret_cast<uint4*>(&al[buf][lora_t_at(q, gg)]) = lo;
    }
  };
  // x fragments of a chunk: 32-deep step s takes columns 32 s + 8 g .. + 7
  auto load_x = [&](uint4 (&xf)[2], int c) {
#pragma unroll
    for (int s = 0; s < 2; ++s)
      xf[s] = *reinterpret_cast<const uint4*>(xr + int64_t(c) * kLoraTK + 32 * s + 8 * g);
  };

  f32x4_t acc[NSM];
#pragma unroll
  for (int i = 0; i < NSM; ++i) acc[i] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  // chunk c from LDS buffer c % 2 and x fragments xc, with chunk c + 1 loaded meanwhile
  auto step = [&](int c, const uint4 (&xc)[2], uint4 (&xn)[2]) {
    const int cur = c & 1;
    const int nc = min(c + 1, nchunks - 1);  // past the last chunk: a cached re-read, never used
    load_a(nc);
    load_x(xn, nc);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
      for (int ns = 0; ns < NSM; ++ns) {
        const int at = lora_t_at(16 * ns + l16, 4 * s + g);
        const uint4 bh = *reinterpret_cast<const uint4*>(&ah[cur][at]);
        acc[ns] = mfma_16x16x32<E4B_BF16>(xc[s], bh, acc[ns]);
        if constexpr (LO) {
          const uint4 bl = *reinterpret_cast<const uint4*>(&al[cur][at]);
          acc[ns] = mfma_16x16x32<E4B_BF16>(xc[s], bl, acc[ns]);
        }
      }
    }
    store_a(cur ^ 1);  // the other buffer: its last readers passed the previous barrier
    __syncthreads();
  };
  uint4 xa[2], xb[2];
  load_a(0);
  load_x(xa, 0);
  store_a(0);
  __syncthreads();
  for (int c = 0; c < nchunks; c += 2) {  // two chunks per trip: the fragment sets stay in registers
    step(c, xa, xb);
    if (c + 1 < nchunks) step(c + 1, xb, xa);
  }
  // lane holds t[row 16 w + 4 g + i][rank 16 ns + l16]
#pragma unroll
  for (int ns = 0; ns < NSM; ++ns) {
    const int q = 16 * ns + l16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * w + 4 * g + i;
      if (q < rank && r < rows) t[int64_t(row0 + r) * rank + q] = acc[ns][i];
    }
  }
}

}  // namespace e4b
