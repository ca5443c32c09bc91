// Prefill / large-batch grouped GEMM on the bf16 (fp16) matrix cores of gfx950.
//
// One workgroup computes a BM-row x BN-weight-row tile of one expert: 128 x 256 (8 waves) for
// prefill-sized groups, 32 x 128 (4 waves) for mid-size batches where experts get few rows (the
// 256-row tiles of the fused prefill run gemm_wide_kernel). Every dequantized weight feeds BM
// rows, so the decode work per MFMA falls as BM grows, and every activation tile feeds BN weight rows: its
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
//
// fp16 mode (F16C, bf16 activations with NF4 weights): the MFMAs multiply fp16 operands. The
// weights are decoded through the LDS table of code pairs as
// fp16(fp16(code) * fp16(absmax * 2^shift[e])) -- three fp16 roundings, at most 3 * 2^-11
// relative where the bf16 weight carries 2^-8 -- and the A rows arrive as their bf16 values
// times 2^exp_shift(row exponent), exact in fp16 (row_exp_kernel). The accumulators are scaled
// back by 2^-(row shift + expert shift) before the epilogue, so the results are those of the
// exact weights to within those roundings.
#pragma once

#include <utility>

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

// LDS tile layout: 128-byte rows of 64 elements, the row's eight 16-byte groups stored in the
// order group ^ (row & 7). gfx950 serves ds_read_b128 at 256 bytes per clock and ds_write_b128
// at 128: the MFMA fragment reads (16 consecutive rows, one group each) and the staging stores
// (consecutive groups of a few rows) then fall in distinct banks, both conflict-free. (A
// 144-byte padded row costs the fragment reads a 2-way conflict, a 160-byte one the stores:
// measured with SQ_LDS_BANK_CONFLICT on single-instruction patterns.) Element offset of the
// 16-byte group holding column col (a multiple of 8) of a row:
E4B_DEV int lds_at(int row, int col) { return row * kTileK + ((((col >> 3) ^ row) & 7) << 3); }
// K steps of global loads in flight ahead of the MFMAs (6 for the 32-row tiles was measured:
// no change at bs=64, whose blocks are bound by their decode and LDS work, not by latency).
// The 128-row tiles hold two: a third set spills at their 256-register budget.
constexpr int gemm_stages(int bm) { return bm >= kTileM ? 2 : 3; }
constexpr int kXcds = 8;    // accelerator dies of an MI355X; blocks go round-robin over them

// XCD-aware, balanced block -> (M tile, N tile) map. Workgroups go round-robin over the 8 XCDs
// (block L runs on XCD L % 8). The num_tiles x n_tiles work items, in (M tile, N tile) order, are
// cut into 8 runs of equal length, run x for XCD x: every XCD gets the same number of blocks
// (to within one), and consecutive items -- the N sweep of one M tile (the same activation
// rows), an expert's consecutive M tiles (the same weights) -- share that XCD's L2. false: the
// block is past the work (the grid is sized for the routing's max_tiles).
E4B_DEV bool tile_of_block(int num_tiles, int n_tiles, int& tile, int& n_tile) {
  const int total = num_tiles * n_tiles;
  const int per = (total + kXcds - 1) / kXcds;
  const int xcd = static_cast<int>(blockIdx.x % kXcds);
  const int q = static_cast<int>(blockIdx.x / kXcds);
  const int w = xcd * per + q;
  if (q >= per || w >= total) return false;
  tile = w / n_tiles;
  n_tile = w % n_tiles;
  return true;
}

// A block's work item from its index alone: tile t runs on XCD t % 8 (workgroups go round-robin
// over the 8 XCDs: block L runs on XCD L % 8), and each XCD sweeps all N tiles of one M tile
// before its next M tile, in list order -- a tile's activation rows stay in that XCD's L2 across
// its N sweep. The grid is sized for the routing's max_tiles, so the tile may lie past the list:
// its (expert, first row) is read at an index clamped into the list's capacity, in the same round
// trip as the tile count, and the block has work iff ok. (Computing the item from the count
// instead would put one more dependent round trip ahead of every load of the block.)
struct TileItem {
  int tile, n_tile, e, row0;
  bool ok;
};
E4B_DEV TileItem tile_item(const e4b_routing& rt, int n_tiles) {
  TileItem t;
  const int xcd = static_cast<int>(blockIdx.x % kXcds);
  const int q = static_cast<int>(blockIdx.x / kXcds);
  t.tile = (q / n_tiles) * kXcds + xcd;
  t.n_tile = q % n_tiles;
  const int tc = min(t.tile, rt.max_tiles - 1);
  const int num_tiles = rt.meta[0];
  t.e = rt.tiles[2 * tc];
  t.row0 = rt.tiles[2 * tc + 1];
  // one round trip for the three loads: without this use ahead of the caller's early exit the
  // compiler sinks the tile's loads past it, behind the count's
  asm volatile("; tile %0 %1 of %2" ::"s"(t.e), "s"(t.row0), "s"(num_tiles));
  t.ok = t.tile < num_tiles;
  return t;
}

// f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>): indices known at compile
// time whatever the unroller decides, so the accumulator array never needs an address (a loop
// left rolled would put all 256 accumulators in scratch memory).
template <class F, int... I>
E4B_DEV void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
E4B_DEV void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

typedef float f32x16_t __attribute__((ext_vector_type(16)));

template <int DT>
E4B_DEV f32x16_t mfma_32x32x16(const uint4& a, const uint4& b, const f32x16_t& c) {
  if constexpr (DT == E4B_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                  c, 0, 0, 0);
  }
}

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

// fp32 product code * scale. To reproduce the dequantized fp16 weight bit for bit (REF) the
// product is kept away from the conversion (mul_f32), which instruction selection could otherwise
// fuse into one rounding of the exact product; the fp16 matrix-core mode takes that fusion (one
// rounding instead of two, and fewer instructions).
template <int DT, bool REF = true>
E4B_DEV float code_times_scale(float c, float s) {
  if constexpr (DT == E4B_FP16 && REF) return mul_f32(c, s);
  else return c * s;
}

E4B_DEV uint32_t bfi(uint32_t m, uint32_t a, uint32_t b) { return (m & a) | (~m & b); }

// NB packed bytes (2 * NB values; byte i = elements 2i and 2i + 1, the first in the high nibble
// for NF4, in the low one for e2m1) -> NB words of DT pairs, each value dt(fp32(code * scale)).
//
// All in registers, no memory lookups: the 16 possible values P[c] = dt(fp32(code[c] * scale))
// of this weight row and K step are formed once (16 products, 8 conversions) and kept as byte
// planes lo[k] / hi[k] = the low / high bytes of P[4k .. 4k+3]. Four nibbles (one per byte of a
// word) then select their entries at once: v_perm_b32 over planes 0-1 (entries 0..7) and over
// planes 2-3 (entries 8..15), merged by each nibble's bit 3 (v_bfi_b32, the byte mask made by
// one more v_perm_b32), for the low and the high bytes; four more v_perm_b32 interleave the
// bytes into the (first, second) pairs. Every
// value is the same fp32 product and rounding as a per-element decode, so the result is
// bit-identical to the dequantized weights.
//
// e2m1 (power-of-two scales): one v_cvt_scalef32_pk_{bf16,f16}_fp4 per byte forms the byte's
// two values dt(code * scale) directly.
template <int DT, int SEL>
E4B_DEV uint32_t fp4_scaled_pair(uint32_t w, float scale) {
  if constexpr (DT == E4B_BF16) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, SEL));
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, scale, SEL));
  }
}

// The 16 entries dt(fp32(code[c] * scale)) of one weight row and step as byte planes: lo[k] /
// hi[k] hold the low / high bytes of entries 4k .. 4k+3 (16 products, 8 conversions, 8 v_perm).
struct NibPlanes {
  uint32_t lo[4], hi[4];
};
template <int DT, bool REF = true>
E4B_DEV NibPlanes nib_planes(const float (&code)[16], float scale) {
  uint32_t q[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    q[i] = cvt_pair<DT>(code_times_scale<DT, REF>(code[2 * i], scale), code_times_scale<DT, REF>(code[2 * i + 1], scale));
  NibPlanes t;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    t.lo[k] = __builtin_amdgcn_perm(q[2 * k + 1], q[2 * k], 0x06040200u);
    t.hi[k] = __builtin_amdgcn_perm(q[2 * k + 1], q[2 * k], 0x07050301u);
  }
  return t;
}

// One packed word (four bytes; byte i = elements 2i and 2i + 1, the first in the high nibble for
// NF4, in the low one for e2m1) -> four words of DT pairs, looked up in the planes.
template <int FMT>
E4B_DEV void nib_word(const NibPlanes& t, uint32_t w, uint32_t (&wv)[4]) {
  // four nibbles: sel = their low three bits (one per byte), m = 0xff in each byte whose
  // nibble is 8..15 -> the low and the high bytes of their four entries
  auto look = [&](uint32_t sel, uint32_t m, uint32_t& l, uint32_t& h) {
    l = bfi(m, __builtin_amdgcn_perm(t.lo[3], t.lo[2], sel), __builtin_amdgcn_perm(t.lo[1], t.lo[0], sel));
    h = bfi(m, __builtin_amdgcn_perm(t.hi[3], t.hi[2], sel), __builtin_amdgcn_perm(t.hi[1], t.hi[0], sel));
  };
  // v_perm selectors 8..11 replicate bit 15 / 31 of either source into a whole byte; the
  // nibbles' bit 3 are shifted there: low nibbles (w bits 3, 11, 19, 27) and high nibbles
  // (w bits 7, 15, 23, 31)
  const uint32_t sel_l = w & 0x07070707u, sel_h = (w >> 4) & 0x07070707u;
  const uint32_t m_l = __builtin_amdgcn_perm(w << 4, w << 12, 0x0B090A08u);
  const uint32_t m_h = __builtin_amdgcn_perm(w, w << 8, 0x0B090A08u);
  uint32_t lf, hf, ls, hs;
  if constexpr (FMT == E4B_FMT_MXFP4) {
    look(sel_l, m_l, lf, hf);  // first elements: low nibbles
    look(sel_h, m_h, ls, hs);
  } else {
    look(sel_h, m_h, lf, hf);  // first elements: high nibbles
    look(sel_l, m_l, ls, hs);
  }
  const uint32_t f01 = __builtin_amdgcn_perm(hf, lf, 0x05010400u), f23 = __builtin_amdgcn_perm(hf, lf, 0x07030602u);
  const uint32_t s01 = __builtin_amdgcn_perm(hs, ls, 0x05010400u), s23 = __builtin_amdgcn_perm(hs, ls, 0x07030602u);
  wv[0] = __builtin_amdgcn_perm(s01, f01, 0x05040100u);
  wv[1] = __builtin_amdgcn_perm(s01, f01, 0x07060302u);
  wv[2] = __builtin_amdgcn_perm(s23, f23, 0x05040100u);
  wv[3] = __builtin_amdgcn_perm(s23, f23, 0x07060302u);
}

// e2m1: one v_cvt_scalef32_pk_{bf16,f16}_fp4 per byte forms its two values dt(code * scale).
template <int DT>
E4B_DEV void fp4_word(uint32_t w, float scale, uint32_t (&wv)[4]) {
  wv[0] = fp4_scaled_pair<DT, 0>(w, scale);
  wv[1] = fp4_scaled_pair<DT, 1>(w, scale);
  wv[2] = fp4_scaled_pair<DT, 2>(w, scale);
  wv[3] = fp4_scaled_pair<DT, 3>(w, scale);
}

template <int DT, int FMT, int NB, bool REF = true>
E4B_DEV void dequant_bytes(const uint32_t (&words)[NB / 4], const float (&code)[16], float scale, uint32_t (&wv)[NB]) {
  if constexpr (FMT == E4B_FMT_MXFP4) {
#pragma unroll
    for (int wi = 0; wi < NB / 4; ++wi) {
      uint32_t o[4];
      fp4_word<DT>(words[wi], scale, o);
#pragma unroll
      for (int j = 0; j < 4; ++j) wv[4 * wi + j] = o[j];
    }
    return;
  }
  const NibPlanes t = nib_planes<DT, REF>(code, scale);
#pragma unroll
  for (int wi = 0; wi < NB / 4; ++wi) {
    uint32_t o[4];
    nib_word<FMT>(t, words[wi], o);
#pragma unroll
    for (int j = 0; j < 4; ++j) wv[4 * wi + j] = o[j];
  }
}

// fp16 matrix-core mode of the wide tiles: packed bytes decoded through an LDS table of the 256
// byte values' code pairs, entry b = (fp16(code[b >> 4]), fp16(code[b & 15])) (the first element,
// the high nibble, in the low half), times the row's block scale as an fp16 pair (v_pk_mul_f16):
// one lookup and one multiply per two weights, where the register decode above spends about six
// VALU instructions per two. kPairCopies copies of the table, copy c in word c of each entry's
// 64 bytes, lane l reading copy l % kPairCopies. Each weight is then
// fp16(fp16(code) * fp16(absmax * 2^shift)), three fp16 roundings (relative error <= 3 * 2^-11,
// against 2^-8 for the reference's bf16 weight).
constexpr int kPairCopies = 16;
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
E4B_DEV uint32_t pk_mul_f16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, a) * __builtin_bit_cast(h2_t, b));
}

// Tile shapes: weight rows per tile and threads (8 waves for the 128- and 256-row tiles, else 4).
// (The 256-row tiles run gemm_wide_kernel: 256 weight rows, four waves.)
constexpr int gemm_tile_nw(int bm) { return bm >= kTileM ? kTileNWWide : kTileNW; }
constexpr int gemm_threads(int bm) { return bm == kTileM ? 512 : 256; }

// F16C: fp16 mode, the A rows already stored as scaled fp16 by row_exp_kernel; else the
// operands are in the activation dtype.
template <int DT, int FMT, int BM, bool F16C = false>
__global__ void __launch_bounds__(gemm_threads(BM)) gemm_mfma_kernel(GemmArgs p) {
  static_assert(!F16C || (DT == E4B_BF16 && FMT != E4B_FMT_MXFP4), "fp16 mode: bf16 activations, NF4 weights");
  constexpr int CT = F16C ? E4B_FP16 : DT;  // MFMA operand type
  constexpr int NT = gemm_threads(BM);
  constexpr int BN = gemm_tile_nw(BM);
  constexpr int WAVES = NT / kWave;
  constexpr int WAVES_M = BM >= 128 ? 2 : 1;
  constexpr int WAVES_N = WAVES / WAVES_M;
  constexpr int WM = BM / WAVES_M;       // rows per wave
  constexpr int WN = BN / WAVES_N;       // weight rows per wave
  constexpr int MS = WM / 16, NS = WN / 16;
  constexpr int TPR = NT / BM;            // threads per A row
  constexpr int AV = kTileK / TPR / 8;    // uint4 of A per thread per step
  constexpr int TPW = NT / BN;            // threads per weight row
  constexpr int WB = kTileK / 2 / TPW;    // packed weight bytes per thread per step
  static_assert(BM == kTileM || BM == kTileMSmall, "tile rows: 128 or 32 (256: gemm_wide_kernel)");
  static_assert(AV >= 1 && NS % 2 == 0 && (WB == 16 || WB == 8), "tile shape");
  constexpr int ST = gemm_stages(BM);
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * kTileK];
  __shared__ __attribute__((aligned(16))) uint16_t Ws[2][BN * kTileK];
  __shared__ float code2_s[(FMT == E4B_FMT_NF4_DQ) ? 256 : 1];
  __shared__ int row_shift_s[F16C ? BM : 1];  // fp16 mode: each tile row's activation shift
  // fp16 mode: the LDS table of code pairs (see kPairCopies), PC copies
  constexpr int PC = BM == kTileMSmall ? 8 : kPairCopies;
  __shared__ uint32_t ptab[F16C ? 256 * PC : 1];

  const int num_tiles = p.rt.meta[0];
  const int n_tiles = static_cast<int>((p.n_out + (is_gated(p.epi) ? BN / 2 : BN) - 1) /
                                       (is_gated(p.epi) ? BN / 2 : BN));
  int tile, n_tile;
  if (!tile_of_block(num_tiles, n_tiles, tile, n_tile)) return;
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

  // the 16 codes (the same in every lane), and the second-level code of double quantization
  float code[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) code[i] = (FMT == E4B_FMT_MXFP4) ? kFp4E2M1[i] : p.w.code[i];
  if constexpr (FMT == E4B_FMT_NF4_DQ) {
    if (tid < 256) code2_s[tid] = p.w.code2[tid];
  }
  if constexpr (F16C) {
    // pass j fills entries 32 j .. 32 j + 31 (all copies): this thread's entry is
    // 32 j + tid / PC, high nibble 2 j + (tid / PC) / 16, low nibble (tid / PC) % 16
    static_assert(NT / PC == 32, "table fill");
    const int t = tid / PC;
    const float lo = p.w.code[t & 15];
    const bool odd = t >= 16;
#pragma unroll
    for (int j = 0; j < 256 * PC / NT; ++j)
      ptab[j * NT + tid] = cvt_pair<E4B_FP16>(odd ? code[2 * j + 1] : code[2 * j], lo);
  }

  // A assignment: row tid / TPR, AV * 8 activations at column (tid % TPR) * AV * 8.
  const int ar = tid / TPR;
  const int aseg = (tid % TPR) * AV * 8;
  const int r = row0 + ar;
  // the row's source, loaded at a clamped index before row_end is known and dropped for rows
  // past the expert's end (a load behind the row test waits for row_end first)
  const int sfv = p.rt.sorted_flat[min(r, static_cast<int>(p.M) - 1)];
  const int64_t src = (r < row_end) ? (p.gather_k > 0 ? sfv / p.gather_k : r) : 0;
  const uint16_t* aptr = p.a + src * k + aseg;
  // fp16 mode: the tile row's activation shift (for the epilogue) and the expert's weight shift
  int wsh = 0;
  if constexpr (F16C) {
    wsh = p.w.shift[e];
    if (tid % TPR == 0) row_shift_s[ar] = exp_shift(p.a_exp[src]);
  }

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
    if constexpr (F16C) scale = __builtin_amdgcn_ldexpf(scale, wsh);  // exact: a power of two
    uint32_t wv[WB];
    if constexpr (F16C) {
      // table decode: every lookup first, then the multiplies by the scale pair
      const uint32_t s2 = cvt_pair<E4B_FP16>(scale, scale);
      const uint32_t* tab = ptab + (lane & (PC - 1));
#pragma unroll
      for (int wi = 0; wi < WB / 4; ++wi)
#pragma unroll
        for (int b = 0; b < 4; ++b) wv[4 * wi + b] = tab[((wq[set][wi] >> (8 * b)) & 0xffu) * PC];
#pragma unroll
      for (int i = 0; i < WB; ++i) wv[i] = pk_mul_f16(wv[i], s2);
    } else {
      dequant_bytes<CT, FMT, WB, !F16C>(wq[set], code, scale, wv);
    }
    // the swizzled store addresses are recomputed every step (a few integer ops): held across
    // the loop they would take registers the pipeline needs
    int wr = lrow, arow = ar;
    asm volatile("" : "+v"(wr), "+v"(arow));
#pragma unroll
    for (int i = 0; i < WB / 4; ++i)
      *reinterpret_cast<uint4*>(&Ws[buf][lds_at(wr, half * 2 * WB + 8 * i)]) =
          make_uint4(wv[4 * i], wv[4 * i + 1], wv[4 * i + 2], wv[4 * i + 3]);
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      *reinterpret_cast<u32x4_t*>(&As[buf][lds_at(arow, aseg + 8 * i)]) = areg[set][i];
    }
  };
  // MFMA operands of one 32-deep half step (ks) of LDS buffer buf, and the MFMAs on them. Every
  // fragment row is a multiple of 16 plus (lane & 15), so its swizzle term is lane & 7: the
  // lane's column offset for half step 0 is ((lane >> 4) ^ (lane & 7)) * 8 and for half step 1
  // that XOR 32 (group 4 + lane >> 4), and the rows add compile-time offsets to one base.
  const int fcol0 = ((lane >> 4) ^ (lane & 7)) << 3;
  const int a_frag = (wave_m * WM + (lane & 15)) * kTileK;
  const int w_frag = (lane & 15) * kTileK;
  auto read_frags = [&](int buf, int ks, uint4 (&av)[MS], uint4 (&bv)[NS]) {
    const int fcol = ks ? fcol0 ^ 32 : fcol0;
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
      av[ms] = *reinterpret_cast<const uint4*>(&As[buf][a_frag + ms * 16 * kTileK + fcol]);
    }
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) {
      bv[ns] = *reinterpret_cast<const uint4*>(&Ws[buf][w_frag + nbase[ns] * kTileK + fcol]);
    }
  };
  auto mfmas = [&](const uint4 (&av)[MS], const uint4 (&bv)[NS]) {
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) acc[ms][ns] = mfma_16x16x32<CT>(av[ms], bv[ns], acc[ms][ns]);
  };

  // Step indices past the last step are clamped (a cached re-read nobody uses), for the same
  // reason the loads carry no conditions.
  const int64_t ksteps = k / kTileK;
  const int64_t klast = ksteps - 1;
  load_step(0, 0);
  __syncthreads();  // code2 table
  stage(0, 0);
#pragma unroll
  for (int j = 1; j <= ST; ++j) load_step(j % ST, min<int64_t>(j, klast));
  __syncthreads();
  // Step kb, in two scheduling blocks around the step's one barrier:
  //   before: the fragments of half step 1 are read while the MFMAs of half step 0 run, with
  //           the decode and LDS staging of step kb + 1 (into the other buffer) and the refill
  //           of its register set with step kb + 1 + ST slotted between them;
  //   after:  the MFMAs of half step 1 run from registers while the fragments of step kb + 1's
  //           half step 0 are read, so the LDS latency after the barrier is hidden.
  // (After the last step the staging writes a stale set into the idle buffer and the last
  // fragment reads fetch that buffer; neither is used.) The group barriers spread the decode's
  // VALU work over the MFMAs; left to itself the compiler emits them one after the other.
  uint4 fa0[MS], fb0[NS], fa1[MS], fb1[NS];
  read_frags(0, 0, fa0, fb0);
  auto iteration = [&](int u, int64_t kb) __attribute__((always_inline)) {
    const int cur = static_cast<int>(kb & 1);
    read_frags(cur, 1, fa1, fb1);
    mfmas(fa0, fb0);
    stage((u + 1) % ST, cur ^ 1);
    constexpr int kValu = (F16C ? 48 : WB == 16 ? 200 : 136) / (MS * NS);
#pragma unroll
    for (int i = 0; i < MS * NS; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);      // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);      // one LDS read
      __builtin_amdgcn_sched_group_barrier(0x002, kValu, 0);  // VALU
    }
    load_step((u + 1) % ST, min<int64_t>(kb + 1 + ST, klast));
    __syncthreads();
    read_frags(cur ^ 1, 0, fa0, fb0);
    mfmas(fa1, fb1);
#pragma unroll
    for (int i = 0; i < MS * NS; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
    }
    __builtin_amdgcn_sched_barrier(0);  // the next step's block starts here
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
  if constexpr (F16C) {
    // the operand scales come off first: 2^-(row shift + expert shift), exact
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = -(row_shift_s[wave_m * WM + ms * 16 + 4 * (lane >> 4) + i] + wsh);
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) acc[ms][ns][i] = __builtin_amdgcn_ldexpf(acc[ms][ns][i], d);
      }
  }
  const bool has_bias = p.w.bias != nullptr;
  const uint16_t* bias = static_cast<const uint16_t*>(p.w.bias);
  // The two prefill projections take a branch-free path: epilogue kind, bias and output type
  // are kernel arguments, and the general path below tests them per element.
  if (pair && p.epi == E4B_EPI_SWIGLU && !has_bias && !p.out_f32) {  // gate_up: silu(g) * u -> dt
    uint16_t* const out = static_cast<uint16_t*>(p.out);
    const int64_t cbase = col0 + wave_n * (WN / 2) + (lane & 15);
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rr = row0 + wave_m * WM + ms * 16 + 4 * (lane >> 4) + i;
        uint16_t* const orow = out + int64_t(rr) * p.n_out + cbase;
#pragma unroll
        for (int ns = 0; ns < NS / 2; ++ns) {
          const float v = silu_f32(acc[ms][ns][i]) * acc[ms][ns + NS / 2][i];
          if (rr < row_end && cbase + ns * 16 < p.n_out) orow[ns * 16] = from_f<DT>(v);
        }
      }
    }
    return;
  }
  if (!pair && p.epi == E4B_EPI_NONE && !has_bias && p.out_f32) {  // down: fp32 rows
    float* const out = static_cast<float*>(p.out);
    const int64_t cbase = col0 + wave_n * WN + (lane & 15);
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rr = row0 + wave_m * WM + ms * 16 + 4 * (lane >> 4) + i;
        float* const orow = out + int64_t(rr) * p.n_out + cbase;
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) {
          if (rr < row_end && cbase + ns * 16 < p.n_out) orow[ns * 16] = acc[ms][ns][i];
        }
      }
    }
    return;
  }
  // general path
#pragma unroll
  for (int ms = 0; ms < MS; ++ms) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rr = row0 + wave_m * WM + ms * 16 + 4 * (lane >> 4) + i;
      if (rr < row_end) {
        const int64_t orow = int64_t(rr) * p.n_out;
        if (pair) {
#pragma unroll
          for (int ns = 0; ns < NS / 2; ++ns) {
            const int64_t jj = col0 + wave_n * (WN / 2) + ns * 16 + (lane & 15);
            if (jj >= p.n_out) continue;
            const float bg = has_bias ? to_f<DT>(bias[int64_t(e) * n + jj]) : 0.0f;
            const float bu = has_bias ? to_f<DT>(bias[int64_t(e) * n + n / 2 + jj]) : 0.0f;
            store_elem<DT>(p, orow + jj, gated(p.epi, acc[ms][ns][i], acc[ms][ns + NS / 2][i], p.alpha, p.limit, bg, bu));
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
}

}  // namespace e4b
