// Training-lane kernels over expert-sorted rows (routing tables from route.h, no host-side group
// sizes): the frozen projection's input gradient and the LoRA weight gradients.
//
//   dgrad_mfma_kernel  out[m, :] = g[m, :] . deq(W[e_m]) -- g the gradient of the projection's
//                      output [M, n], W [E, n, k] the frozen 4-bit weights, out [M, k] fp32. The
//                      reduction runs over the weight's OUTPUT features, so the weights are read
//                      along their rows' k axis and transposed while they are decoded into LDS:
//                      each thread decodes a 4 (n) x 8 (k) block -- 4 row words of packed bytes,
//                      one scale per row, in registers -- pairs its rows per k column with
//                      v_perm, and stores it as 8 k-rows of 4 n-values, the layout
//                      the MFMA B fragments read (k-rows of 64 reduction values, the same XOR
//                      swizzle as the forward GEMM). Every weight is dt(fp32(code * scale)), the
//                      forward's dequantized value; the gradient rows are the A operand as loaded;
//                      v_mfma_f32_16x16x32 with fp32 accumulators; two register stages of global
//                      loads ahead of the MFMAs, double-buffered LDS, one barrier per 64-deep step,
//                      the decode of step s + 1 interleaved with the MFMAs of step s.
//   lora_wgrad_kernel  out[e, j, c] = scale * sum over expert e's rows m of u[m, j] * a_m[c] (in
//                      row order): dL/dA = scaling * (g . B)^T . x and dL/dB^T = scaling * t^T . g
//                      of a LoRA projection, per expert. Block (expert, 256 columns); the rows'
//                      u entries are staged in LDS 32 at a time and broadcast to the block.
#pragma once

#include <type_traits>

#include "common.h"
#include "gemm.h"

namespace e4b {

struct DgradArgs {
  const uint16_t* g;  // [M, w.n] sorted rows, activation dtype
  e4b_qweight w;      // [E, n, k]
  e4b_routing rt;     // tiles of rt.tile_m rows
  float* out;         // [M, w.k]
};

constexpr int dgrad_threads(int bm) { return bm >= kTileM ? 512 : 256; }
constexpr int dgrad_cols(int bm) { return bm >= kTileM ? 256 : 128; }

template <int DT, int FMT, int BM>
__global__ void __launch_bounds__(dgrad_threads(BM)) dgrad_mfma_kernel(DgradArgs p) {
  static_assert(FMT != E4B_FMT_MXFP4, "the LoRA bases are NF4");
  constexpr int NT = dgrad_threads(BM);
  constexpr int BC = dgrad_cols(BM);           // output columns (weight k) per tile
  constexpr int WAVES = NT / kWave;
  constexpr int WAVES_M = BM / 32;
  constexpr int WAVES_C = WAVES / WAVES_M;
  constexpr int WC = BC / WAVES_C;             // output columns per wave
  constexpr int MS = 2, NS = WC / 16;          // 16x16 sub-tiles per wave: 32 rows x WC columns
  constexpr int TPR = NT / BM;                 // threads per gradient row
  constexpr int AV = kTileK / TPR / 8;         // uint4 of gradient per thread per step
  constexpr int NQ = kTileK / 4;               // 4-row weight blocks per 64-deep step
  static_assert(NT == NQ * (BC / 8) && AV >= 1 && NS >= 1, "one 4 x 8 weight block per thread");
  constexpr int ST = 2;
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * kTileK];
  __shared__ __attribute__((aligned(16))) uint16_t Ws[2][BC * kTileK];
  __shared__ float code2_s[(FMT == E4B_FMT_NF4_DQ) ? 256 : 1];

  // XCD-aware order, as the forward GEMM: XCD x takes a contiguous run of row tiles and sweeps
  // all column tiles of one row tile before the next (the gradient tile stays in its L2).
  const int num_tiles = p.rt.meta[0];
  const int64_t K = p.w.k, n = p.w.n;
  const int c_tiles = static_cast<int>((K + BC - 1) / BC);
  const int xcd = static_cast<int>(blockIdx.x % kXcds);
  const int q = static_cast<int>(blockIdx.x / kXcds);
  const int chunk = (num_tiles + kXcds - 1) / kXcds;
  const int m_local = q / c_tiles;
  const int tile = xcd * chunk + m_local;
  if (m_local >= chunk || tile >= num_tiles) return;
  const int64_t c0 = int64_t(q % c_tiles) * BC;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wid = tid / kWave;
  const int wave_m = wid % WAVES_M;
  const int wave_c = wid / WAVES_M;
  const int e = p.rt.tiles[2 * tile];
  const int row0 = p.rt.tiles[2 * tile + 1];
  const int row_end = min(row0 + BM, p.rt.offsets[e + 1]);

  float code[16];  // the same in every lane
#pragma unroll
  for (int i = 0; i < 16; ++i) code[i] = p.w.code[i];
  if constexpr (FMT == E4B_FMT_NF4_DQ) {
    if (tid < 256) code2_s[tid] = p.w.code2[tid];
  }

  // gradient rows: row tid / TPR, AV * 8 values at (tid % TPR) * AV * 8 of the step; tile rows
  // past the expert's end read the tile's first row (never stored)
  const int ar = tid / TPR;
  const int aseg = (tid % TPR) * AV * 8;
  const int64_t src = (row0 + ar < row_end) ? row0 + ar : row0;
  const uint16_t* aptr = p.g + src * n + aseg;

  // weight block: rows 4 * nq .. 4 * nq + 3 of the step, columns c0 + 8 * cg .. + 7 (one packed
  // word per row, inside one 64-column scale block); columns past k read column 0 (never stored)
  // lane l of wave w: column group (l & 7) + 8 * (w % CGW), row quad (l >> 3) + 8 * (w / CGW), so a
  // load instruction reads 32 contiguous bytes of each of 8 rows
  constexpr int CGW = BC / 64;  // waves across the column groups
  const int cg = (lane & 7) + 8 * (wid % CGW);
  const int nq = (lane >> 3) + 8 * (wid / CGW);
  const int64_t cc = (c0 + 8 * cg < K) ? c0 + 8 * cg : 0;
  const uint8_t* wbase = p.w.packed + int64_t(e) * n * (K / 2) + cc / 2;
  const int64_t nb = n * (K / 64);  // scale blocks per expert
  const int64_t cblk = cc / 64;
  const float offset = (FMT == E4B_FMT_NF4_DQ) ? p.w.offset[e] : 0.0f;
  // The weight tile's LDS layout: k-rows of 64 n values, the 16-byte group of n-group ng stored
  // at ng ^ (row & 7) ^ ((row >> 3) & 7). The extra term makes the staging stores -- eight
  // column groups of one n-quad, rows 8 apart -- land in distinct banks, and the fragment reads
  // (16 consecutive rows) stay conflict-free.
  auto w_at = [](int row, int ng) { return row * kTileK + (((ng ^ row ^ (row >> 3)) & 7) << 3); };

  f32x4_t acc[MS][NS];
#pragma unroll
  for (int i = 0; i < MS; ++i)
#pragma unroll
    for (int j = 0; j < NS; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  u32x4_t areg[ST][AV];
  uint32_t wq[ST][4];
  float sa[ST][4];
  uint32_t sq[ST][4];
  // every load unconditional (indices clamped instead), so the waits count exactly
  auto load_step = [&](int set, int64_t s) {
    const u32x4_t* ap = reinterpret_cast<const u32x4_t*>(aptr + s * kTileK);
#pragma unroll
    for (int i = 0; i < AV; ++i) areg[set][i] = ap[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t nn = s * kTileK + 4 * nq + i;
      wq[set][i] = *reinterpret_cast<const uint32_t*>(wbase + nn * (K / 2));
      const int64_t blk = nn * (K / 64) + cblk;  // the row's scale block, within the expert
      if constexpr (FMT == E4B_FMT_NF4) {
        sa[set][i] = static_cast<const float*>(p.w.absmax)[int64_t(e) * nb + blk];
      } else {
        sq[set][i] = static_cast<const uint8_t*>(p.w.absmax)[int64_t(e) * nb + blk];
        sa[set][i] = p.w.absmax2[int64_t(e) * ((nb + 255) / 256) + blk / 256];
      }
    }
  };
  auto stage = [&](int set, int buf) {
    int arow = ar, wrow = 8 * cg;
    asm volatile("" : "+v"(arow), "+v"(wrow));
#pragma unroll
    for (int i = 0; i < AV; ++i)
      *reinterpret_cast<u32x4_t*>(&As[buf][lds_at(arow, aseg + 8 * i)]) = areg[set][i];
    float sc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (FMT == E4B_FMT_NF4) {
        sc[i] = sa[set][i];
      } else {
        const float prod = code2_s[sq[set][i]] * sa[set][i];
        sc[i] = prod + offset;
      }
    }
    // each row word decoded in registers (the forward's byte-plane decode: dt(fp32(code *
    // scale)), pairs of consecutive k), then rows paired per k column by v_perm: k column 2b
    // and 2b + 1 of the block take the low / high halves of byte b's pairs of rows (0, 1) and
    // (2, 3), one 8-byte store each into the k-row's four n values
    uint32_t wv[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t word[1] = {wq[set][i]};
      dequant_bytes<DT, FMT, 4>(word, code, sc[i], wv[i]);
    }
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t lo01 = __builtin_amdgcn_perm(wv[1][b], wv[0][b], 0x05040100u);
      const uint32_t hi01 = __builtin_amdgcn_perm(wv[1][b], wv[0][b], 0x07060302u);
      const uint32_t lo23 = __builtin_amdgcn_perm(wv[3][b], wv[2][b], 0x05040100u);
      const uint32_t hi23 = __builtin_amdgcn_perm(wv[3][b], wv[2][b], 0x07060302u);
      const int r0 = wrow + 2 * b, r1 = r0 + 1;
      const int g = 4 * (nq & 1);
      *reinterpret_cast<uint2*>(&Ws[buf][w_at(r0, nq >> 1) + g]) = make_uint2(lo01, lo23);
      *reinterpret_cast<uint2*>(&Ws[buf][w_at(r1, nq >> 1) + g]) = make_uint2(hi01, hi23);
    }
  };
  const int fcol0 = ((lane >> 4) ^ (lane & 7)) << 3;
  const int a_frag = (wave_m * 32 + (lane & 15)) * kTileK;
  // B fragment rows wave_c * WC + 16 * ns + (lane & 15): the swizzle term of row r is
  // g ^ (r & 7) ^ ((r >> 3) & 7), and (r >> 3) & 7 = g1 ^ (2 * ns & 7) with the lane's
  // g1 = ((wave_c * WC) / 8 + (lane & 15) / 8) & 7: for these tile shapes (WC a multiple of 32)
  // g1 has no bit 1 and 2 * ns no bit 0, so their sum mod 8 is their XOR (a carry out of bit 2
  // is dropped) -- four XOR terms per half step, not one address per fragment.
  static_assert(WC % 32 == 0, "fragment swizzle terms");
  const int w_frag = (wave_c * WC + (lane & 15)) * kTileK;
  const int g1 = (((wave_c * WC) >> 3) + ((lane & 15) >> 3)) & 7;
  // fragments of one 32-deep half step (ks) of LDS buffer buf, and the MFMAs on them
  auto read_frags = [&](int buf, int ks, uint4 (&av)[MS], uint4 (&bv)[NS]) {
    const int fcol = ks ? fcol0 ^ 32 : fcol0;
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
      av[ms] = *reinterpret_cast<const uint4*>(&As[buf][a_frag + ms * 16 * kTileK + fcol]);
#pragma unroll
    for (int ns = 0; ns < NS; ++ns)
      bv[ns] = *reinterpret_cast<const uint4*>(
          &Ws[buf][w_frag + ns * 16 * kTileK + ((((lane >> 4) + 4 * ks) ^ (lane & 7) ^ g1 ^ ((2 * ns) & 7)) << 3)]);
  };
  auto mfmas = [&](const uint4 (&av)[MS], const uint4 (&bv)[NS]) {
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) acc[ms][ns] = mfma_16x16x32<DT>(av[ms], bv[ns], acc[ms][ns]);
  };

  // Step s (LDS buffer and register set u = s % 2, both compile-time in the unrolled loop), in
  // two scheduling blocks around its one barrier, as the forward GEMM: the MFMAs of half step 0
  // with the decode and staging of step s + 1 (into the other buffer) and the refill of set u
  // with step s + 2 spread between them; after the barrier, the MFMAs of half step 1 while step
  // s + 1's first fragments are read. Step indices past the last are clamped (unused re-reads).
  const int64_t steps = n / kTileK;
  const int64_t last = steps - 1;
  constexpr int kMf = MS * NS;
  constexpr int kDsRead = (MS + NS + kMf - 1) / kMf;  // fragment reads per MFMA
  constexpr int kValu = 240 / kMf;
  uint4 fa0[MS], fb0[NS], fa1[MS], fb1[NS];
  load_step(0, 0);
  load_step(1, min<int64_t>(1, last));
  __syncthreads();  // code2 table
  stage(0, 0);
  __syncthreads();
  read_frags(0, 0, fa0, fb0);
  auto iteration = [&](auto uc, int64_t s) __attribute__((always_inline)) {
    constexpr int u = decltype(uc)::value;
    read_frags(u, 1, fa1, fb1);
    mfmas(fa0, fb0);
    stage(u ^ 1, u ^ 1);
#pragma unroll
    for (int i = 0; i < kMf; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);        // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, kDsRead, 0);  // LDS reads
      __builtin_amdgcn_sched_group_barrier(0x002, kValu, 0);    // VALU
    }
    load_step(u, min<int64_t>(s + 2, last));
    __syncthreads();
    read_frags(u ^ 1, 0, fa0, fb0);
    mfmas(fa1, fb1);
#pragma unroll
    for (int i = 0; i < kMf; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  int64_t s = 0;
  for (; s + 2 <= steps; s += 2) {
    iteration(std::integral_constant<int, 0>{}, s);
    iteration(std::integral_constant<int, 1>{}, s + 1);
  }
  if (s < steps) iteration(std::integral_constant<int, 0>{}, s);

  // lane holds D[4 * (lane / 16) + i][lane % 16] of each 16 x 16 sub-tile
  const int64_t cbase = c0 + wave_c * WC + (lane & 15);
#pragma unroll
  for (int ms = 0; ms < MS; ++ms)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rr = row0 + wave_m * 32 + ms * 16 + 4 * (lane >> 4) + i;
      float* const orow = p.out + int64_t(rr) * K + cbase;
#pragma unroll
      for (int ns = 0; ns < NS; ++ns)
        if (rr < row_end && cbase + ns * 16 < K) orow[ns * 16] = acc[ms][ns][i];
    }
}

constexpr int kWgradThreads = 256;
constexpr int kWgradRows = 32;  // u rows staged per round

// out[e, j, c] = scale * sum_{m in expert e's rows, in order} u[m, j] * a_m[c], for j < r,
// c < cols; zero for an expert without rows. Block = (expert blockIdx.y, columns 256 *
// blockIdx.x ..); a_m = row sorted_flat[m] / gather_k of a (gather_k > 0) or row m.
template <int XDT, int RB>
__global__ void __launch_bounds__(kWgradThreads) lora_wgrad_kernel(const float* __restrict__ u, int r,
                                                                   const uint16_t* __restrict__ a, int gather_k,
                                                                   const int32_t* __restrict__ sorted_flat,
                                                                   const int32_t* __restrict__ offsets, int64_t cols,
                                                                   float scale, float* __restrict__ out) {
  __shared__ float4 us[kWgradRows][RB / 4];
  const int e = static_cast<int>(blockIdx.y);
  const int64_t c = int64_t(blockIdx.x) * kWgradThreads + threadIdx.x;
  const int beg = offsets[e], end = offsets[e + 1];
  float acc[RB];
#pragma unroll
  for (int j = 0; j < RB; ++j) acc[j] = 0.0f;
  const int64_t cl = c < cols ? c : 0;  // columns past the end read column 0 (never stored)
  float* usf = reinterpret_cast<float*>(&us[0][0]);
  for (int m0 = beg; m0 < end; m0 += kWgradRows) {
    const int nr = min(kWgradRows, end - m0);
    __syncthreads();  // the previous round's reads are done
    for (int i = threadIdx.x; i < kWgradRows * RB; i += kWgradThreads) {
      const int row = i / RB, j = i % RB;
      usf[i] = (row < nr && j < r) ? u[int64_t(m0 + row) * r + j] : 0.0f;
    }
    __syncthreads();
    for (int i0 = 0; i0 < nr; i0 += 8) {
      float av[8];
#pragma unroll
      for (int b = 0; b < 8; ++b) {  // the batch's loads go out together
        const int m = m0 + min(i0 + b, nr - 1);
        const int64_t row = gather_k > 0 ? static_cast<int64_t>(sorted_flat[m] / gather_k) : m;
        av[b] = to_f<XDT>(a[row * cols + cl]);
      }
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        if (i0 + b < nr) {
          const float4* ur = us[i0 + b];
#pragma unroll
          for (int q4 = 0; q4 < RB / 4; ++q4) {
            const float4 uv = ur[q4];
            acc[4 * q4] = __builtin_fmaf(uv.x, av[b], acc[4 * q4]);
            acc[4 * q4 + 1] = __builtin_fmaf(uv.y, av[b], acc[4 * q4 + 1]);
            acc[4 * q4 + 2] = __builtin_fmaf(uv.z, av[b], acc[4 * q4 + 2]);
            acc[4 * q4 + 3] = __builtin_fmaf(uv.w, av[b], acc[4 * q4 + 3]);
          }
        }
      }
    }
  }
  if (c >= cols) return;
#pragma unroll
  for (int j = 0; j < RB; ++j)
    if (j < r) out[(int64_t(e) * r + j) * cols + c] = scale * acc[j];
}

}  // namespace e4b
