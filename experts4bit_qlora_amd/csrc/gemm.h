// Prefill / large-batch grouped GEMM on the bf16 (fp16) matrix cores of gfx950.
//
// One workgroup computes a BM-row x BN-weight-row tile of one expert: 128 x 256 (8 waves) for
// prefill-sized groups, 32 x 128 (4 waves) for mid-size batches where experts get few rows,
// 256 x 128 (8 waves) for full 256-row runs. Every dequantized weight feeds BM rows, so the
// decode work per MFMA falls as BM grows, and every activation tile feeds BN weight rows: its
// global (L2) reads repeat once per N tile, so the prefill tile is wide. Tiles come from
// the route kernel's (expert, first sorted row) list, so skewed expert sizes cost at most one
// partial tile per expert and the grid never depends on host-side counts.
//
// Pipeline, per 64-deep K step (one NF4 absmax block per weight row):
//   * global -> registers runs ST steps ahead (A rows gathered through sorted_flat when
//     gather_k > 0, the index_select of fast.py:135 fused into the loads; 16 packed bytes +
//     the scale of each weight half-row), in ST rotating register sets, so several
//     global round trips overlap the MFMAs of step s, which read LDS buffer s % 2;
//   * after the MFMAs, step s+1's registers are written to the other LDS buffer: activations as
//     loaded, weights decoded with ONE fp32 product code[nib] * scale and one RNE rounding --
//     bit-identical to the reference's dequantized bf16 (fp16) weight. Codes come from a
//     16-entry fp32 LDS table indexed by nibble: its 16 words sit in 16 different banks, so a
//     lookup never conflicts (lanes reading the same word share one broadcast);
//   * one barrier per step. Each wave runs (BM / WAVES_M / 16) x (128 / WAVES_N / 16)
//     v_mfma_f32_16x16x32_{bf16,f16} per 32-deep half step with fp32 accumulators.
// Gated epilogues pair gate row j with up row n/2 + j in the same tile: LDS rows 0..BN/2-1 hold
// the gate rows of BN/2 output columns and rows BN/2..BN-1 their up rows, and a wave's gate and up
// accumulators sit in the same lanes, so the activation runs on registers (fp32) before the
// only store.
#pragma once

#include "common.h"
#include "dequant.h"
#include "gemv.h"

namespace e4b {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kTileMBig = 256;   // rows per tile for the full 256-row runs of large experts
constexpr int kTileM = 128;      // rows per tile of the prefill-sized GEMM
constexpr int kTileMSmall = 32;  // rows per tile for mid-size batches
constexpr int kTileNW = 128;     // weight rows per tile of the 32- and 256-row shapes
constexpr int kTileNWWide = 256; // weight rows per tile of the 128-row (prefill) shape
constexpr int kTileK = 64;
constexpr int kLdsPitch = kTileK + 8;  // elements; 144-byte rows keep 16-byte alignment
// K steps of global loads in flight ahead of the MFMAs (6 for the 32-row tiles was measured:
// no change at bs=64, whose blocks are bound by their decode and LDS work, not by latency)
constexpr int gemm_stages(int) { return 3; }
constexpr int kXcds = 8;    // accelerator dies of an MI355X; blocks go round-robin over them

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

// Two fp32 values rounded to nearest even into one packed DT pair (first in the low half):
// one v_cvt_pk_{bf16,f16}_f32.
template <int DT>
E4B_DEV uint32_t cvt_pair(float a, float b) {
  typedef float f2_t __attribute__((ext_vector_type(2)));
  const f2_t v = {a, b};
  if constexpr (DT == E4B_BF16) {
    typedef __bf16 o2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, o2_t));
  } else {
    typedef _Float16 o2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, o2_t));
  }
}

// fp32 product code * scale. For fp16 the product is kept away from the conversion (mul_f32),
// which instruction selection could otherwise fuse into one rounding of the exact product.
template <int DT>
E4B_DEV float code_times_scale(float c, float s) {
  if constexpr (DT == E4B_FP16) return mul_f32(c, s);
  else return c * s;
}

// NB packed bytes (2 * NB values; byte i = elements 2i and 2i + 1, the first in the high nibble
// for NF4, in the low one for e2m1) -> NB words of DT pairs, each value dt(fp32(code * scale)).
// Table offsets are nibble * 4: bits 2..5 of byte b of (w << 2) hold its low nibble, of (w >> 2)
// its high one.
template <int DT, int FMT, int NB>
E4B_DEV void dequant_bytes(const uint32_t (&words)[NB / 4], const float* code16, float scale, uint32_t (&wv)[NB]) {
  const char* tb = reinterpret_cast<const char*>(code16);
#pragma unroll
  for (int wi = 0; wi < NB / 4; ++wi) {
    const uint32_t wl = words[wi] << 2, wh = words[wi] >> 2;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const float c_lo = *reinterpret_cast<const float*>(tb + ((wl >> (8 * b)) & 0x3cu));
      const float c_hi = *reinterpret_cast<const float*>(tb + ((wh >> (8 * b)) & 0x3cu));
      const float first = (FMT == E4B_FMT_MXFP4) ? c_lo : c_hi;
      const float second = (FMT == E4B_FMT_MXFP4) ? c_hi : c_lo;
      wv[4 * wi + b] = cvt_pair<DT>(code_times_scale<DT>(first, scale), code_times_scale<DT>(second, scale));
    }
  }
}

// Tile shapes: weight rows per tile and threads (8 waves for the 128- and 256-row tiles, else 4).
constexpr int gemm_tile_nw(int bm) { return bm == kTileM ? kTileNWWide : kTileNW; }
constexpr int gemm_threads(int bm) { return bm >= kTileM ? 512 : 256; }

template <int DT, int FMT, int BM>
__global__ void __launch_bounds__(gemm_threads(BM)) gemm_mfma_kernel(GemmArgs p) {
  constexpr int NT = gemm_threads(BM);
  constexpr int BN = gemm_tile_nw(BM);
  constexpr int WAVES = NT / kWave;
  constexpr int WAVES_M = BM >= 256 ? 4 : BM >= 128 ? 2 : 1;
  constexpr int WAVES_N = WAVES / WAVES_M;
  constexpr int WM = BM / WAVES_M;       // rows per wave
  constexpr int WN = BN / WAVES_N;       // weight rows per wave
  constexpr int MS = WM / 16, NS = WN / 16;
  constexpr int TPR = NT / BM;            // threads per A row
  constexpr int AV = kTileK / TPR / 8;    // uint4 of A per thread per step
  constexpr int TPW = NT / BN;            // threads per weight row
  constexpr int WB = kTileK / 2 / TPW;    // packed weight bytes per thread per step
  static_assert(AV >= 1 && NS % 2 == 0 && (WB == 16 || WB == 8), "tile shape");
  constexpr int ST = gemm_stages(BM);
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * kLdsPitch];
  __shared__ __attribute__((aligned(16))) uint16_t Ws[2][BN * kLdsPitch];
  __shared__ float code16[16];
  __shared__ float code2_s[(FMT == E4B_FMT_NF4_DQ) ? 256 : 1];

  // XCD-aware tile order: workgroups are dispatched round-robin over the 8 XCDs, so linear
  // block L runs on XCD L % 8. XCD x takes the contiguous run of M tiles
  // [x * chunk, (x + 1) * chunk) and sweeps all N tiles of one M tile before the next: the
  // activation tile stays in that XCD's L2 across the N sweep, and an expert's consecutive M
  // tiles (same weights) stay on one XCD as well.
  const int num_tiles = p.rt.meta[0];
  const int n_tiles = static_cast<int>((p.n_out + (is_gated(p.epi) ? BN / 2 : BN) - 1) /
                                       (is_gated(p.epi) ? BN / 2 : BN));
  const int xcd = static_cast<int>(blockIdx.x % kXcds);
  const int q = static_cast<int>(blockIdx.x / kXcds);
  const int chunk = (num_tiles + kXcds - 1) / kXcds;
  const int m_local = q / n_tiles;
  const int tile = xcd * chunk + m_local;
  if (m_local >= chunk || tile >= num_tiles) return;
  const int n_tile = q % n_tiles;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wid = tid / kWave;
  const int wave_m = wid % WAVES_M;
  const int wave_n = wid / WAVES_M;
  const int e = p.rt.tiles[2 * tile];
  const int row0 = p.rt.tiles[2 * tile + 1];
  const int row_end = min(row0 + BM, p.rt.offsets[e + 1]);
  const bool pair = is_gated(p.epi);
  const int64_t n = p.w.n;
  const int64_t k = p.w.k;
  const int64_t col0 = int64_t(n_tile) * (pair ? BN / 2 : BN);
  if (col0 >= p.n_out) return;

  // decode tables: the 16 codes, and the second-level code of double quantization
  if (tid < 16) code16[tid] = (FMT == E4B_FMT_MXFP4) ? kFp4E2M1[tid] : p.w.code[tid];
  if constexpr (FMT == E4B_FMT_NF4_DQ) {
    if (tid < 256) code2_s[tid] = p.w.code2[tid];
  }

  // A assignment: row tid / TPR, AV * 8 activations at column (tid % TPR) * AV * 8.
  const int ar = tid / TPR;
  const int aseg = (tid % TPR) * AV * 8;
  const int r = row0 + ar;
  const int64_t src = (r < row_end) ? (p.gather_k > 0 ? p.rt.sorted_flat[r] / p.gather_k : r) : 0;
  const uint16_t* aptr = p.a + src * k + aseg;

  // W assignment: LDS row tid / TPW (0..BN-1), 2 * WB values of the 64-deep step at
  // (tid % TPW) * 2 * WB.
  const int lrow = tid / TPW;
  const int half = tid % TPW;  // which WB-byte part of the row's 32 packed bytes
  int64_t grow;
  bool wvalid;
  if (pair) {
    const int64_t jj = col0 + (lrow & (BN / 2 - 1));
    wvalid = jj < p.n_out;
    grow = (lrow < BN / 2) ? jj : n / 2 + jj;
  } else {
    grow = col0 + lrow;
    wvalid = grow < p.n_out;
  }
  if (!wvalid) grow = 0;
  const uint8_t* wptr = p.w.packed + (int64_t(e) * n + grow) * (k / 2) + half * WB;
  const int64_t nb = n * (k / 64);
  const float offset = (FMT == E4B_FMT_NF4_DQ) ? p.w.offset[e] : 0.0f;

  f32x4_t acc[MS][NS];
#pragma unroll
  for (int i = 0; i < MS; ++i)
#pragma unroll
    for (int j = 0; j < NS; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  int nbase[NS];
#pragma unroll
  for (int ns = 0; ns < NS; ++ns) {
    nbase[ns] = pair ? ((ns < NS / 2) ? wave_n * (WN / 2) + ns * 16 : BN / 2 + wave_n * (WN / 2) + (ns - NS / 2) * 16)
                     : wave_n * WN + ns * 16;
  }

  // ---- step registers: ST sets, step j in set j % ST, loaded ST steps before
  // the step that writes it to LDS, so that many global round trips overlap the MFMAs
  // Every load is unconditional: tile rows past the expert's end read row 0, and weight rows
  // past n_out read weight row 0; both feed only outputs that are never stored. (A load behind
  // a branch leaves the compiler unsure how many loads are in flight, and it then waits for all
  // of them, which would cancel the prefetch.) Native vector types keep the sets in registers.
  u32x4_t areg[ST][AV];
  uint32_t wq[ST][WB / 4];
  float sa[ST];     // NF4 absmax, or double-quant absmax2
  uint32_t sq[ST];  // double-quant code, or e8m0
  auto load_step = [&](int set, int64_t kb) {
    const u32x4_t* ap = reinterpret_cast<const u32x4_t*>(aptr + kb * kTileK);
#pragma unroll
    for (int i = 0; i < AV; ++i) areg[set][i] = ap[i];
    if constexpr (WB == 16) {
      const uint4 v = *reinterpret_cast<const uint4*>(wptr + kb * 32);
      wq[set][0] = v.x; wq[set][1] = v.y; wq[set][2] = v.z; wq[set][3] = v.w;
    } else {
      const uint2 v = *reinterpret_cast<const uint2*>(wptr + kb * 32);
      wq[set][0] = v.x; wq[set][1] = v.y;
    }
    if constexpr (FMT == E4B_FMT_MXFP4) {
      sq[set] = static_cast<const uint8_t*>(p.w.absmax)[(int64_t(e) * n + grow) * (k / 32) + kb * 2 + half * WB / 16];
    } else if constexpr (FMT == E4B_FMT_NF4) {
      sa[set] = static_cast<const float*>(p.w.absmax)[e * nb + grow * (k / 64) + kb];
    } else {
      const int64_t blk = grow * (k / 64) + kb;
      sq[set] = static_cast<const uint8_t*>(p.w.absmax)[e * nb + blk];
      sa[set] = p.w.absmax2[e * ((nb + 255) / 256) + blk / 256];
    }
  };
  auto stage = [&](int set, int buf) {
    // weight rows past n_out hold row 0's bytes and feed only columns that are never stored, so
    // their scale needs no condition (a select here becomes a branch that splits the schedule)
    float scale;
    if constexpr (FMT == E4B_FMT_MXFP4) {
      scale = e8m0_to_f32(sq[set]);
    } else if constexpr (FMT == E4B_FMT_NF4) {
      scale = sa[set];
    } else {
      // fp32(fp32(code2 * absmax2) + offset): plain operators, two roundings (no contraction
      // under -ffp-contract=off); an asm fence or constrained intrinsic would split the schedule
      const float prod = code2_s[sq[set]] * sa[set];
      scale = prod + offset;
    }
    uint32_t wv[WB];
    dequant_bytes<DT, FMT, WB>(wq[set], code16, scale, wv);
    uint4* ws = reinterpret_cast<uint4*>(&Ws[buf][lrow * kLdsPitch + half * 2 * WB]);
#pragma unroll
    for (int i = 0; i < WB / 4; ++i) ws[i] = make_uint4(wv[4 * i], wv[4 * i + 1], wv[4 * i + 2], wv[4 * i + 3]);
    u32x4_t* as = reinterpret_cast<u32x4_t*>(&As[buf][ar * kLdsPitch + aseg]);
#pragma unroll
    for (int i = 0; i < AV; ++i) as[i] = areg[set][i];
  };
  auto mfma_step = [&](int buf) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int kcol = ks * 32 + (lane >> 4) * 8;
      uint4 av[MS], bv[NS];
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) {
        av[ms] = *reinterpret_cast<const uint4*>(&As[buf][(wave_m * WM + ms * 16 + (lane & 15)) * kLdsPitch + kcol]);
      }
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) {
        bv[ns] = *reinterpret_cast<const uint4*>(&Ws[buf][(nbase[ns] + (lane & 15)) * kLdsPitch + kcol]);
      }
#pragma unroll
      for (int ms = 0; ms < MS; ++ms)
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) acc[ms][ns] = mfma_16x16x32<DT>(av[ms], bv[ns], acc[ms][ns]);
    }
  };

  // Step indices past the last step are clamped (a cached re-read nobody uses), for the same
  // reason the loads carry no conditions.
  const int64_t ksteps = k / kTileK;
  const int64_t klast = ksteps - 1;
  load_step(0, 0);
  __syncthreads();  // tables
  stage(0, 0);
#pragma unroll
  for (int j = 1; j <= ST; ++j) load_step(j % ST, min<int64_t>(j, klast));
  __syncthreads();
  // step kb: its MFMAs, then stage step kb + 1 (after the last step: a stale set into the idle
  // buffer, never read) and refill that set with step kb + 1 + ST
  // The MFMAs of step kb and the decode / staging of step kb + 1 form one scheduling block;
  // the group barriers slot the decode's LDS reads and VALU work between MFMAs that are still
  // executing. (Left to itself the compiler emits them one after the other, and the per-step
  // block barrier then keeps every wave of a SIMD in the same phase, so nothing overlaps.)
  auto iteration = [&](int u, int64_t kb) __attribute__((always_inline)) {
    const int cur = static_cast<int>(kb & 1);
    mfma_step(cur);
    stage((u + 1) % ST, cur ^ 1);
#pragma unroll
    for (int i = 0; i < 2 * MS * NS; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // two LDS reads
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // four VALU
    }
    load_step((u + 1) % ST, min<int64_t>(kb + 1 + ST, klast));
    __syncthreads();
  };
  const int64_t kmain = ksteps - ksteps % ST;
  for (int64_t kb0 = 0; kb0 < kmain; kb0 += ST) {
#pragma unroll
    for (int u = 0; u < ST; ++u) iteration(u, kb0 + u);
  }
#pragma unroll
  for (int u = 0; u < ST - 1; ++u) {
    if (kmain + u < ksteps) iteration(u, kmain + u);
  }

  // Epilogue: lane holds D[4*(lane/16) + i][lane % 16] of each 16x16 sub-tile.
  const bool has_bias = p.w.bias != nullptr;
  const uint16_t* bias = static_cast<const uint16_t*>(p.w.bias);
#pragma unroll
  for (int ms = 0; ms < MS; ++ms) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rr = row0 + wave_m * WM + ms * 16 + 4 * (lane >> 4) + i;
      if (rr >= row_end) continue;
      const int64_t orow = int64_t(rr) * p.n_out;
      if (pair) {
#pragma unroll
        for (int ns = 0; ns < NS / 2; ++ns) {
          const int64_t jj = col0 + wave_n * (WN / 2) + ns * 16 + (lane & 15);
          if (jj >= p.n_out) continue;
          const float bg = has_bias ? to_f<DT>(bias[int64_t(e) * n + jj]) : 0.0f;
          const float bu = has_bias ? to_f<DT>(bias[int64_t(e) * n + n / 2 + jj]) : 0.0f;
          store_elem<DT>(p, orow + jj,
                         gated(p.epi, acc[ms][ns][i], acc[ms][ns + NS / 2][i], p.alpha, p.limit, bg, bu));
        }
      } else {
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) {
          const int64_t nn = col0 + wave_n * WN + ns * 16 + (lane & 15);
          if (nn >= p.n_out) continue;
          const float b = has_bias ? to_f<DT>(bias[int64_t(e) * n + nn]) : 0.0f;
          store_elem<DT>(p, orow + nn, single(p.epi, acc[ms][ns][i], b));
        }
      }
    }
  }
}

}  // namespace e4b
