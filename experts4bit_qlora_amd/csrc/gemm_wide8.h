// Prefill grouped GEMM, wide tiles with two waves per SIMD: 256 sorted rows x 256 weight rows
// per workgroup, eight waves of 128 x 64 each on 32 x 32 x 16 MFMAs. Two weight formats: in the
// fp16 matrix-core mode (F16C: bf16 activations stored as scaled fp16 rows, NF4 / double-quant
// NF4 weights decoded through the LDS code-pair table, v_mfma_f32_32x32x16_f16), and MXFP4 with
// bf16 activations (e2m1 bytes converted in registers by v_cvt_scalef32_pk_bf16_fp4, exact in
// bf16, v_mfma_f32_32x32x16_bf16; a thread's 32 values of a step are one e8m0 scale block).
//
// gemm_wide_kernel runs the same tile with four waves of 128 x 128, one per SIMD: nothing covers
// a stall of its wave, so its loop is laid out by hand, and still a 64-deep step takes ~3x its
// MFMA time (no single part bounds it: with half its MFMAs, no table lookups, or every load an
// L2 hit, the gate_up launch is only 3-8 % faster). Here every SIMD holds two waves of one
// workgroup, each with half the accumulators (128 registers), and issues from whichever is ready:
// the schedule is left to the compiler and the hardware. Per 64-deep step and CU the fragment
// reads grow from 128 to 192 KB of LDS (a wave's B fragments feed 2 accumulator columns, not 4),
// still below the step's MFMA time; each weight is still decoded once for all 256 rows (thread
// t stages half of weight row t / 2: four packed words, four lookups and four v_pk_mul_f16 each).
//
// Pipeline: step s computes from LDS buffer s % 2 while step s + 1 is staged from registers into
// the other buffer (its activation pieces and decoded weight words spread over the four 16-deep
// sub-steps), then the register set step s + 1 used is refilled with the global loads of step
// s + 3; one barrier per step. A step's loads are thus issued two steps before its staging.
//
// Output layout of a 32 x 32 MFMA: lane l holds column l % 32 of rows
// 8 * (i / 4) + 4 * (l / 32) + i % 4, i = 0..15, of its tile.
#pragma once

#include "gemm.h"
#include "gemm_wide.h"
#include "lora_mfma.h"

namespace e4b {

constexpr int kWide8Threads = 512;

// A tile's record and its rows' sources, loaded by the kernel in the round trip after the tile's
// (beside the code tables' loads): the expert, its first sorted row and the expert's row end, and
// in the fp16 mode, for thread t, the sources of tile rows 64 i + t / 8 (i < 4: its activation
// pieces) and t % 256 (its row shift) -- sorted_flat at each row clamped to the last one with a
// gather, the row itself without. Sources of rows past the expert's end are dropped where they
// are used.
struct Wide8Rows {
  int e, row0, end;
  int sf[5];
};

// One tile. HALF: a tile of at most 128 rows as 128 rows x 256 weight rows (waves of 64 x 64).
template <int DT, int FMT, bool F16C, bool HALF, bool LORA, bool H16>
E4B_DEV void wide8_tile(const GemmArgs& p, const Wide8Rows& tr, int n_tile, uint16_t (&As)[2][kWideTileM * kTileK],
                        uint16_t (&Ws)[2][kWideTileN * kTileK], const float* code2_s, int* row_shift_s,
                        const uint32_t* ptab) {
  constexpr int CT = F16C ? E4B_FP16 : DT;
  constexpr int BM = HALF ? kWideTileM / 2 : kWideTileM, BN = kWideTileN;
  constexpr int MS = BM / 64;  // 32-row MFMA tiles per wave (each wave: BM / 2 rows)
  constexpr int NS = 2;        // 32-column MFMA tiles per wave
  constexpr int NT = kWide8Threads;
  constexpr int AP = BM * kTileK / 8 / NT;  // 16-byte activation pieces per thread and step
  constexpr int RS = 2;                     // register sets of global loads
  const bool pair = is_gated(p.epi);
  const int cols = pair ? BN / 2 : BN;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wid = __builtin_amdgcn_readfirstlane(tid) / kWave;
  const int wave_m = wid & 1;
  const int wave_n = wid >> 1;
  const int e = tr.e;
  const int row0 = tr.row0;
  const int row_end = min(row0 + BM, tr.end);
  const int64_t n = p.w.n;
  const int64_t k = p.w.k;
  const int64_t col0 = int64_t(n_tile) * cols;
  if (col0 >= p.n_out) return;

  // activation piece i of thread t: tile row 64 i + t / 8, columns 8 (t % 8) .. + 7 (eight lanes
  // read one row's 128 contiguous bytes); aoff[i]: that piece of step 0 in 16-byte units of p.a
  const int apart = tid & 7;
  const bool gather = p.gather_k > 0;
  auto row_src = [&](int r, int s) -> int64_t { return r < row_end ? (gather ? s / p.gather_k : s) : 0; };
  uint32_t aoff[AP];
#pragma unroll
  for (int i = 0; i < AP; ++i) {
    const int r = row0 + 64 * i + (tid >> 3);
    if constexpr (F16C) {
      aoff[i] = static_cast<uint32_t>((row_src(r, tr.sf[i]) * k) / 8 + apart);
    } else {
      // bf16 activations (MXFP4): each source loaded here behind its row test, which measured
      // ~1 % faster for the gpt-oss prefill than the sources loaded ahead by the kernel
      const int64_t src = (r < row_end) ? (gather ? p.rt.sorted_flat[r] / p.gather_k : r) : 0;
      aoff[i] = static_cast<uint32_t>((src * k) / 8 + apart);
    }
  }
  const int wsh = F16C ? p.w.shift[e] : 0;
  // the exponent of tile row t (t < BM), stored to row_shift_s (the epilogue's shifts) once the
  // first steps' loads are out
  const int a_exp_row = F16C ? p.a_exp[row_src(row0 + (tid & (kWideTileM - 1)), tr.sf[4])] : 0;
  // weights: thread t stages half wh = t % 2 of LDS weight row wr = t / 2 (for a gated epilogue
  // rows 0..127 are the gate rows of the tile's 128 output columns, 128..255 their up rows); rows
  // past n_out read weight row 0 and feed only columns that are never stored
  const int wr = tid >> 1, wh = tid & 1;
  int64_t grow;
  if (pair) {
    const int64_t jj = col0 + (wr & (BN / 2 - 1));
    grow = jj < p.n_out ? ((wr < BN / 2) ? jj : n / 2 + jj) : 0;
  } else {
    grow = col0 + wr < p.n_out ? col0 + wr : 0;
  }
  const uint8_t* wptr = p.w.packed + (int64_t(e) * n + grow) * (k / 2) + 16 * wh;
  const int64_t nb = n * (k / 64);
  const float offset = (FMT == E4B_FMT_NF4_DQ) ? p.w.offset[e] : 0.0f;

  f32x16_t acc[MS][NS];
  static_for<MS>([&](auto ms) { static_for<NS>([&](auto ns) { acc[ms][ns] = f32x16_t{}; }); });

  u32x4_t areg[RS][AP];
  uint4 wq[RS];
  float sa[RS];
  uint32_t sq[RS];  // double quant: code index; MXFP4: the e8m0 scale of the thread's 32 values
  auto load_a = [&](int set, int64_t kb) {
#pragma unroll
    for (int i = 0; i < AP; ++i) areg[set][i] = (reinterpret_cast<const u32x4_t*>(p.a) + kb * (kTileK / 8))[aoff[i]];
  };
  auto load_w = [&](int set, int64_t kb) {
    wq[set] = *reinterpret_cast<const uint4*>(wptr + kb * 32);
    if constexpr (FMT == E4B_FMT_MXFP4) {
      sq[set] = static_cast<const uint8_t*>(p.w.absmax)[(int64_t(e) * n + grow) * (k / 32) + 2 * kb + wh];
    } else if constexpr (FMT == E4B_FMT_NF4) {
      sa[set] = static_cast<const float*>(p.w.absmax)[e * nb + grow * (k / 64) + kb];
    } else {
      const int64_t blk = grow * (k / 64) + kb;
      sq[set] = static_cast<const uint8_t*>(p.w.absmax)[e * nb + blk];
      sa[set] = p.w.absmax2[e * ((nb + 255) / 256) + blk / 256];
    }
  };
  // the block scale of a staged step: as an fp16 pair with 2^shift applied (exact) for the
  // table decode, as the fp32 scale for the e2m1 conversion
  auto scale_pair = [&](int set) -> uint32_t {
    if constexpr (FMT == E4B_FMT_MXFP4) return sq[set];
    float scale;
    if constexpr (FMT == E4B_FMT_NF4) {
      scale = sa[set];
    } else {
      const float prod = code2_s[sq[set]] * sa[set];
      scale = prod + offset;
    }
    scale = __builtin_amdgcn_ldexpf(scale, wsh);
    return cvt_pair<E4B_FP16>(scale, scale);
  };
  auto store_a = [&](int set, int buf, int i) {
    *reinterpret_cast<u32x4_t*>(&As[buf][lds_at_w(64 * i + (tid >> 3), 8 * apart)]) = areg[set][i];
  };
  // weight word wi (values 32 wh + 8 wi .. + 7 of the row's step): byte b's code pair from the
  // lane's table copy, times the scale pair, one 16-byte store
  const uint32_t* tab = ptab + (lane & (kPairCopies - 1));
  auto store_w = [&](int set, int buf, int wi, uint32_t sc) {
    const uint32_t w = wi == 0 ? wq[set].x : wi == 1 ? wq[set].y : wi == 2 ? wq[set].z : wq[set].w;
    uint32_t o[4];
    if constexpr (FMT == E4B_FMT_MXFP4) {
      fp4_word<CT>(w, e8m0_to_f32(sc), o);
    } else {
#pragma unroll
      for (int b = 0; b < 4; ++b) o[b] = pk_mul_f16(tab[((w >> (8 * b)) & 0xffu) * kPairCopies], sc);
    }
    *reinterpret_cast<uint4*>(&Ws[buf][lds_at_w(wr, 32 * wh + 8 * wi)]) = make_uint4(o[0], o[1], o[2], o[3]);
  };

  // fragments of sub-step ks (k = 16 ks .. + 15): lane l reads row (base + l % 32), the eight
  // values at k = 16 ks + 8 (l / 32); every base is a multiple of 32, so the row's swizzle term
  // is (l & 7) ^ ((l >> 3) & 3) ^ 4 (base / 32 & 1)
  int nbase[NS], bpar[NS];
#pragma unroll
  for (int ns = 0; ns < NS; ++ns) {
    nbase[ns] = pair ? (ns == 0 ? 32 * wave_n : BN / 2 + 32 * wave_n) : 64 * wave_n + 32 * ns;
    bpar[ns] = ((nbase[ns] >> 5) & 1) << 5;
  }
  const int a_frag = (wave_m * (BM / 2) + (lane & 31)) * kTileK;
  const int w_frag = (lane & 31) * kTileK;
  auto sub_step = [&](int buf, int ks) {
    const int fcol = (((2 * ks + (lane >> 5)) ^ lane ^ ((lane >> 3) & 3)) & 7) << 3;
    uint4 bv[NS];
#pragma unroll
    for (int ns = 0; ns < NS; ++ns)
      bv[ns] = *reinterpret_cast<const uint4*>(&Ws[buf][w_frag + nbase[ns] * kTileK + (fcol ^ bpar[ns])]);
    static_for<MS>([&](auto ms) {
      const uint4 av = *reinterpret_cast<const uint4*>(&As[buf][a_frag + ms * 32 * kTileK + (fcol ^ ((ms & 1) << 5))]);
      static_for<NS>([&](auto ns) { acc[ms][ns] = mfma_32x32x16<CT>(av, bv[ns], acc[ms][ns]); });
    });
  };

  const int64_t ksteps = k / kTileK;
  const int64_t klast = ksteps - 1;
  load_a(0, 0);
  load_w(0, 0);
  load_a(1, min<int64_t>(1, klast));
  load_w(1, min<int64_t>(1, klast));
  if (F16C && tid < BM) row_shift_s[tid] = exp_shift(a_exp_row);
  __syncthreads();  // code2 table, code-pair table, row shifts
  if constexpr (LORA) {
    // the accumulators start as the tile's LoRA delta, scaled like the products (lora_mfma.h):
    // the lane's t rows (clamped to the expert's rows: the rest is never stored) times their
    // activation shifts, the B rows of its columns (weight row 0 past n_out) times the expert's
    // weight shift
    int64_t brow[NS];
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) {
      const int tr = nbase[ns] + (lane & 31);
      if (pair) {
        const int64_t jj = col0 + (tr & (BN / 2 - 1));
        brow[ns] = jj < p.n_out ? (tr < BN / 2 ? jj : n / 2 + jj) : 0;
      } else {
        brow[ns] = col0 + tr < p.n_out ? col0 + tr : 0;
      }
    }
    const int arow = wave_m * (BM / 2) + (lane & 31);
    lora_delta_32x32<MS, NS>(p, acc, e, row0 + arow, row_end - 1,
                             [&](int ms) { return row_shift_s[arow + 32 * ms]; }, wsh, brow, lane);
  }
  {  // step 0 into buffer 0; its register set takes step 2
    const uint32_t sc = scale_pair(0);
#pragma unroll
    for (int i = 0; i < AP; ++i) store_a(0, 0, i);
#pragma unroll
    for (int wi = 0; wi < 4; ++wi) store_w(0, 0, wi, sc);
  }
  load_a(0, min<int64_t>(2, klast));
  load_w(0, min<int64_t>(2, klast));
  __syncthreads();

  // step kb: sub-steps from buffer kb % 2, step kb + 1 (register set (kb + 1) % 2) staged into the
  // other buffer, one activation piece group and one weight word per sub-step; then that set
  // takes step kb + 3. (Past the last step the loads re-read the last step and the staging fills
  // a buffer no later step reads.)
  auto iteration = [&](auto uc, int64_t kb) __attribute__((always_inline)) {
    constexpr int nset = (decltype(uc)::value + 1) % RS;
    const int cur = static_cast<int>(kb & 1);
    const uint32_t sc = scale_pair(nset);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      sub_step(cur, ks);
#pragma unroll
      for (int i = 0; i < AP; ++i)
        if (i == ks) store_a(nset, cur ^ 1, i);
      store_w(nset, cur ^ 1, ks, sc);
    }
    load_a(nset, min<int64_t>(kb + 3, klast));
    load_w(nset, min<int64_t>(kb + 3, klast));
    __syncthreads();
  };
  const int64_t kmain = ksteps - ksteps % RS;
  for (int64_t kb0 = 0; kb0 < kmain; kb0 += RS) {
    iteration(std::integral_constant<int, 0>{}, kb0);
    iteration(std::integral_constant<int, 1>{}, kb0 + 1);
  }
  if (kmain < ksteps) iteration(std::integral_constant<int, 0>{}, kmain);

  // epilogue: the operand scales come off (2^-(row shift + expert shift), exact), then the
  // gated or plain store; the lane index is formed again here (v_mbcnt) so nothing from before
  // the loop stays live across it
  const int lane_e = static_cast<int>(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)));
  auto row_of = [&](int ms, int i) {
    return wave_m * (BM / 2) + ms * 32 + 8 * (i >> 2) + 4 * (lane_e >> 5) + (i & 3);
  };
  if constexpr (F16C) {
    static_for<MS>([&](auto ms) {
      static_for<16>([&](auto i) {
        const int d = H16 ? -p.out_f16_shift : -(row_shift_s[row_of(ms, i)] + wsh);
        static_for<NS>([&](auto ns) { acc[ms][ns][int(i)] = __builtin_amdgcn_ldexpf(acc[ms][ns][int(i)], d); });
      });
    });
  }
  const bool has_bias = p.w.bias != nullptr;
  const uint16_t* bias = static_cast<const uint16_t*>(p.w.bias);
  if (pair && p.epi == E4B_EPI_SWIGLU && !has_bias && !p.out_f32) {  // gate_up: silu(g) * u -> bf16
    uint16_t* const out = static_cast<uint16_t*>(p.out);
    const int64_t cc = col0 + 32 * wave_n + (lane_e & 31);
    if (cc < p.n_out) {
      static_for<MS>([&](auto ms) {
        static_for<16>([&](auto i) {
          const int rr = row0 + row_of(ms, i);
          const float v = silu_f32(acc[ms][0][int(i)]) * acc[ms][1][int(i)];
          if (rr < row_end) out[int64_t(rr) * p.n_out + cc] = from_f<DT>(v);
        });
      });
    }
    return;
  }
  if constexpr (H16) {  // down: fp16 rows, the operand scales left on (the host checks the form)
    uint16_t* const out = static_cast<uint16_t*>(p.out);
    const int64_t cbase = col0 + 64 * wave_n + (lane_e & 31);
    static_for<MS>([&](auto ms) {
      static_for<16>([&](auto i) {
        const int rr = row0 + row_of(ms, i);
        uint16_t* const orow = out + int64_t(rr) * p.n_out + cbase;
        static_for<NS>([&](auto ns) {
          if (rr < row_end && cbase + ns * 32 < p.n_out) orow[ns * 32] = from_f<E4B_FP16>(acc[ms][ns][int(i)]);
        });
      });
    });
    return;
  }
  if (!pair && p.epi == E4B_EPI_NONE && !has_bias && p.out_f32) {  // down: fp32 rows
    float* const out = static_cast<float*>(p.out);
    const int64_t cbase = col0 + 64 * wave_n + (lane_e & 31);
    static_for<MS>([&](auto ms) {
      static_for<16>([&](auto i) {
        const int rr = row0 + row_of(ms, i);
        float* const orow = out + int64_t(rr) * p.n_out + cbase;
        static_for<NS>([&](auto ns) {
          if (rr < row_end && cbase + ns * 32 < p.n_out) orow[ns * 32] = acc[ms][ns][int(i)];
        });
      });
    });
    return;
  }
  // general path
  static_for<MS>([&](auto ms) {
    static_for<16>([&](auto i) {
      const int rr = row0 + row_of(ms, i);
      if (rr < row_end) {
        const int64_t orow = int64_t(rr) * p.n_out;
        if (pair) {
          const int64_t jj = col0 + 32 * wave_n + (lane_e & 31);
          if (jj < p.n_out) {
            const float bg = has_bias ? to_f<DT>(bias[int64_t(e) * n + jj]) : 0.0f;
            const float bu = has_bias ? to_f<DT>(bias[int64_t(e) * n + n / 2 + jj]) : 0.0f;
            store_elem<DT>(p, orow + jj, gated(p.epi, acc[ms][0][int(i)], acc[ms][1][int(i)], p.alpha, p.limit, bg, bu));
          }
        } else {
          static_for<NS>([&](auto ns) {
            const int64_t nn = col0 + 64 * wave_n + ns * 32 + (lane_e & 31);
            if (nn < p.n_out) {
              const float b = has_bias ? to_f<DT>(bias[int64_t(e) * n + nn]) : 0.0f;
              store_elem<DT>(p, orow + nn, single(p.epi, acc[ms][ns][int(i)], b));
            }
          });
        }
      }
    });
  });
}

// H16: the down rows as fp16 with the operand scales left on (GemmArgs::out_f16_shift).
template <int DT, int FMT, bool F16C, bool LORA = false, bool H16 = false>
__global__ void __launch_bounds__(kWide8Threads) gemm_wide8_kernel(GemmArgs p) {
  static_assert(F16C ? (DT == E4B_BF16 && FMT != E4B_FMT_MXFP4) : (DT == E4B_BF16 && FMT == E4B_FMT_MXFP4),
                "fp16 mode with NF4 weights, or bf16 activations with MXFP4 weights");
  static_assert(!LORA || F16C, "the LoRA epilogue runs in the fp16 mode");
  static_assert(!H16 || (F16C && !LORA), "fp16 down rows: the fp16 mode without LoRA");
  constexpr int BM = kWideTileM, BN = kWideTileN;
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * kTileK];
  __shared__ __attribute__((aligned(16))) uint16_t Ws[2][BN * kTileK];
  __shared__ float code2_s[(FMT == E4B_FMT_NF4_DQ) ? 256 : 1];
  __shared__ int row_shift_s[F16C ? BM : 1];
  __shared__ uint32_t ptab[F16C ? 256 * kPairCopies : 1];
  const int cols = is_gated(p.epi) ? BN / 2 : BN;
  const int n_tiles = static_cast<int>((p.n_out + cols - 1) / cols);
  const TileItem item = tile_item(p.rt, n_tiles);
  if (!item.ok) return;
  const int n_tile = item.n_tile;
  Wide8Rows tr;
#pragma unroll
  for (int i = 0; i < 5; ++i) tr.sf[i] = 0;
  tr.e = item.e;
  tr.row0 = item.row0;
  tr.end = p.rt.offsets[item.e + 1];
  {
    const int mlast = static_cast<int>(p.M) - 1;
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < (F16C ? 5 : 0); ++i) {  // the fp16 mode (MXFP4 loads its sources in the tile)
      const int r = min(item.row0 + (i < 4 ? 64 * i + (tid >> 3) : (tid & (kWideTileM - 1))), mlast);
      const int v = p.rt.sorted_flat[r];
      tr.sf[i] = p.gather_k > 0 ? v : r;
    }
  }
  if constexpr (F16C) {
    if (threadIdx.x < 256) {
      // the table of code pairs: pass j fills entries 16 j .. 16 j + 15, all copies; entry
      // 16 j + t / 16 of copy t % 16 (high nibble j, low nibble t / 16)
      static_assert(256 == 16 * kPairCopies, "table fill");
      const float lo = p.w.code[threadIdx.x / kPairCopies];
#pragma unroll
      for (int j = 0; j < 16; ++j) ptab[j * 256 + threadIdx.x] = cvt_pair<E4B_FP16>(p.w.code[j], lo);
      if constexpr (FMT == E4B_FMT_NF4_DQ) code2_s[threadIdx.x] = p.w.code2[threadIdx.x];
    }
  }
  const int rows = tr.end - tr.row0;  // the tile's rows, capped at BM below
  if (rows <= BM / 2) wide8_tile<DT, FMT, F16C, true, LORA, H16>(p, tr, n_tile, As, Ws, code2_s, row_shift_s, ptab);
  else wide8_tile<DT, FMT, F16C, false, LORA, H16>(p, tr, n_tile, As, Ws, code2_s, row_shift_s, ptab);
}

}  // namespace e4b
