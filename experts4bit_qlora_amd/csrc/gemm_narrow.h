// Grouped GEMM, narrow tiles in the fp16 matrix-core mode (bf16 activations stored as scaled
// fp16 rows, NF4 / double-quant NF4 weights): 32 sorted rows x 256 weight rows per workgroup,
// four waves of 32 x 64 on v_mfma_f32_16x16x32_f16. It runs the tiles that hold few rows: an
// expert's last <= 32 rows in prefill, and every tile of a mid-size batch.
//
// With 32 rows a decoded weight feeds 64 flops, so these tiles are bound by streaming and
// decoding the weights, not by the MFMAs. gemm_mfma_kernel stages the decoded weights through
// LDS, where each is written and read back once with no reuse (one wave owns each weight row).
// Here each lane loads its weight bytes in the MFMA's operand layout and decodes them in
// registers:
//
// * K order over a pair of 128-deep steps (256 K, four absmax blocks). The MFMA takes eight
//   consecutive K slots from each lane group g = lane / 16 (operand row lane % 16). Lane group g
//   owns block g of the pair: in step t (0, 1) of the pair it loads K = 64 g + 32 t .. + 31
//   (16 contiguous packed bytes, one 16-byte load per weight row and step: the four lane groups
//   of a row read one 128-byte line per step), and MFMA j of the step takes
//   K = 64 g + 32 t + 8 j + (0..7) from group g; the activation fragments of step t hold the same
//   K. Each MFMA's 32-term sum thus runs over a permutation of the natural K order, which changes
//   only the fp32 summation order, and a lane needs one block scale per pair of steps.
//   (Every weight load reads 16 rows: the texture-address unit charges such a load by the rows
//   it touches, about 33 cycles, and it bounds these tiles, so the loads per step are kept few:
//   one scale load per weight sub-tile and pair, and the double-quant absmax2 of the row's at
//   most two groups loaded once.)
// * Decode: the LDS table of the 256 byte values' fp16 code pairs of the wide tiles
//   (fp16(code[b >> 4]) in the low half, fp16(code[b & 15]) in the high half), 64 copies, the
//   entry of byte value b for lane l at byte address 256 b + 4 (l % 64). One v_perm_b32 forms
//   that address from the packed word (the byte into bits 8..15, the lane's copy offset into
//   bits 0..7), and every lookup of a wave hits its own bank. Each weight pair is then
//   fp16(pair * fp16(absmax * 2^shift)) (v_pk_mul_f16): the products of gemm_wide_kernel's fp16
//   mode, bit for bit.
// * The activations pass through one LDS buffer (32 rows x the 128 K of a step, 8 KB, 16-byte
//   groups of row r in the order group ^ (r % 16), so that the fragment reads of 16 rows and the
//   staging stores are conflict-free): fragments read, a barrier, the next step's rows stored, a
//   barrier.
//
// 64 KB table + 8 KB activations: two workgroups per CU (two waves per SIMD); the weight bytes
// and block scales of three steps, and the activations of two, are in flight.
#pragma once

#include "gemm.h"
#include "gemm_wide.h"

namespace e4b {

constexpr int kNarrowThreads = 256;
constexpr int kNarrowN = 256;     // weight rows per tile (64 per wave)
constexpr int kNarrowK = 128;     // K per step
constexpr int kNarrowStages = 3;  // weight steps in flight
constexpr int kNarrowCopies = 64; // table copies
constexpr int kNarrowUnroll = 6;  // steps per loop pass: whole weight sets (3) and scale sets (3 pairs)

// The shapes the narrow kernel takes: K a whole number of step pairs, and (double quantization)
// a weight row's absmax blocks within two absmax2 groups.
constexpr bool narrow_fits(int64_t k) { return k > 0 && k % (2 * kNarrowK) == 0 && k <= 256 * 64; }

// LORA: the accumulators start as the tile's LoRA delta (p.lt, p.lb), scaled like the products
// (lora_mfma.h).
// H16: the down rows as fp16 with the operand scales left on (GemmArgs::out_f16_shift).
template <int FMT, bool LORA = false, bool H16 = false>
__global__ void __launch_bounds__(kNarrowThreads) __attribute__((amdgpu_waves_per_eu(2)))
gemm_narrow_kernel(GemmArgs p) {
  static_assert(FMT == E4B_FMT_NF4 || FMT == E4B_FMT_NF4_DQ, "narrow tiles: NF4 weights in fp16 mode");
  static_assert(!(H16 && LORA), "fp16 down rows without LoRA");
  constexpr int BM = kTileMSmall, BN = kNarrowN, KS = kNarrowK, ST = kNarrowStages;
  constexpr int NS = BN / (kNarrowThreads / kWave) / 16;  // 4 weight sub-tiles per wave
  static_assert(kNarrowUnroll % ST == 0 && kNarrowUnroll % 6 == 0, "unroll: whole weight sets and scale sets");
  __shared__ __attribute__((aligned(16))) uint32_t ptab[256 * kNarrowCopies];
  __shared__ __attribute__((aligned(16))) uint16_t As[BM * KS];
  __shared__ float code2_s[FMT == E4B_FMT_NF4_DQ ? 256 : 1];
  __shared__ int row_shift_s[BM];

  // every kernel argument the prologue reads, loaded in one batch: left to itself the compiler
  // loads each just before its first use, behind the early exit and the tile's loads, one
  // dependent round trip each
  asm volatile("; narrow args %0 %1 %2 %3 %4 %5" ::"s"(p.rt.tiles), "s"(p.rt.meta), "s"(p.rt.offsets),
               "s"(p.rt.sorted_flat), "s"(p.a), "s"(p.a_exp));
  asm volatile("; narrow weights %0 %1 %2 %3 %4 %5" ::"s"(p.w.packed), "s"(p.w.absmax), "s"(p.w.absmax2),
               "s"(p.w.shift), "s"(p.w.offset), "s"(p.w.code));
  asm volatile("; narrow sizes %0 %1 %2 %3 %4" ::"s"(p.rt.max_tiles), "s"(p.M), "s"(p.gather_k), "s"(p.w.n),
               "s"(p.w.k));

  const bool pair = is_gated(p.epi);
  const int cols = pair ? BN / 2 : BN;  // output columns per tile
  const int n_tiles = static_cast<int>((p.n_out + cols - 1) / cols);
  const TileItem item = tile_item(p.rt, n_tiles);
  if (!item.ok) return;
  const int n_tile = item.n_tile;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wid = tid / kWave;
  const int l16 = lane & 15, g = lane >> 4;
  const int e = item.e;
  const int row0 = item.row0;
  const int row_end = min(row0 + BM, p.rt.offsets[e + 1]);
  const int64_t n = p.w.n;
  const int64_t k = p.w.k;
  const int64_t col0 = int64_t(n_tile) * cols;
  const int steps = static_cast<int>(k / KS);
  const int last = steps - 1;

  // ---- weight rows: sub-tile ns of the wave holds rows base(ns) + lane % 16. Gated: sub-tiles
  // 0, 1 the gate rows and 2, 3 the up rows of the wave's 32 output columns. Rows past n_out
  // read row 0 (their outputs are never stored).
  // Addresses: uniform per-expert bases plus 32-bit per-lane byte offsets (one expert's
  // weights and scales stay below 4 GB), so the loads take the base in scalar registers.
  const int64_t nb = n * (k / 64);  // absmax blocks per expert
  const uint8_t* const wexp = p.w.packed + int64_t(e) * n * (k / 2);
  const char* const sexp = FMT == E4B_FMT_NF4 ? reinterpret_cast<const char*>(static_cast<const float*>(p.w.absmax) + int64_t(e) * nb)
                                              : reinterpret_cast<const char*>(static_cast<const uint8_t*>(p.w.absmax) + int64_t(e) * nb);
  const char* const s2exp = reinterpret_cast<const char*>(p.w.absmax2 + int64_t(e) * ((nb + 255) / 256));
  uint32_t woff[NS];   // the lane's weight bytes at step 0
  uint32_t blk0[NS];   // the lane's absmax block (within the expert) at pair 0
  float a2lo[NS], a2hi[NS];  // double quant: absmax2 of the row's first and last group
  uint32_t a2bound[NS];      // the first block of the second group
#pragma unroll
  for (int ns = 0; ns < NS; ++ns) {
    int64_t r;
    bool ok;
    if (pair) {
      const int64_t jj = col0 + wid * 32 + (ns & 1) * 16 + l16;
      ok = jj < p.n_out;
      r = ns < 2 ? jj : n / 2 + jj;
    } else {
      r = col0 + wid * 64 + ns * 16 + l16;
      ok = r < p.n_out;
    }
    if (!ok) r = 0;
    woff[ns] = static_cast<uint32_t>(r * (k / 2)) + g * 32u;
    const uint32_t rb = static_cast<uint32_t>(r * (k / 64));
    blk0[ns] = rb + g;
    if constexpr (FMT == E4B_FMT_NF4_DQ) {
      a2lo[ns] = *reinterpret_cast<const float*>(s2exp + (rb >> 8) * 4u);
      a2hi[ns] = *reinterpret_cast<const float*>(s2exp + ((rb + static_cast<uint32_t>(k / 64) - 1u) >> 8) * 4u);
      a2bound[ns] = ((rb >> 8) + 1u) << 8;
    }
  }
  const float offset = (FMT == E4B_FMT_NF4_DQ) ? p.w.offset[e] : 0.0f;
  const int wsh = p.w.shift[e];

  // ---- activation rows: thread t stages row t / 8, the 16-byte groups 2 c and 2 c + 1 of a
  // step (c = t % 8): K = 64 (c / 2) + 32 t + 16 (c % 2) .. + 15 of the pair, t the step in it
  const int ar = tid >> 3;
  const int ac = tid & 7;
  const int ag = ac * 2;
  const int r = row0 + ar;
  // the row's source is loaded at a clamped index before row_end is known (one round trip
  // fewer ahead of the activation loads), then dropped for rows past the expert's end
  const int rcl = min(r, static_cast<int>(p.M) - 1);
  const int64_t src_any = p.gather_k > 0 ? p.rt.sorted_flat[rcl] / p.gather_k : rcl;
  const int64_t src = (r < row_end) ? src_any : 0;
  const uint16_t* aptr = p.a + src * k + 64 * (ac >> 1) + 16 * (ac & 1);
  // the row's exponent, loaded ahead of the activation and weight loads: stored to row_shift_s
  // before the first barrier, it was the last load of the prologue, and the wait for it was a
  // wait for all of them (step 2's weights included)
  const int a_exp_row = p.a_exp[src];

  // The tile's rows as MS 16-row MFMA sub-tiles: one when the tile holds at most 16 rows (a
  // mid-size batch's experts and most prefill tails hold a few rows each), halving the MFMAs and
  // fragment reads per step. Everything from the first activation and weight loads on is
  // instantiated for both (the branch comes before those loads, so no register of one
  // instantiation is live in the other).
  auto run_tile = [&](auto MSC) {
  constexpr int MS = decltype(MSC)::value;
  // a statement that differs between the instantiations, so the compiler does not hoist their
  // identical first loads above the branch (which made their registers live in both)
  asm volatile("; %0 row sub-tiles" ::"n"(MS));
  constexpr int PS = 3;  // scale sets: pairs in use or in flight
  u32x4_t areg[2][2];
  uint4 wq[ST][NS];
  float sa[PS][NS];     // NF4 absmax
  uint32_t sq[PS][NS];  // double-quant code index
  // K offset (elements) of step s within the row: pair s / 2, step s % 2 of it
  auto kof = [](int s) { return int64_t(s >> 1) * (2 * KS) + (s & 1) * 32; };
  auto load_a = [&](int set, int s) {
    const u32x4_t* ap = reinterpret_cast<const u32x4_t*>(aptr + kof(s));
    areg[set][0] = ap[0];
    areg[set][1] = ap[1];
  };
  auto load_w = [&](int set, int s) {
#pragma unroll
    for (int ns = 0; ns < NS; ++ns)
      wq[set][ns] = *reinterpret_cast<const uint4*>(wexp + (woff[ns] + static_cast<uint32_t>(s >> 1) * KS +
                                                             static_cast<uint32_t>(s & 1) * 16u));
  };
  auto load_scales = [&](int pset, int pr) {
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) {
      const uint32_t blk = blk0[ns] + 4u * static_cast<uint32_t>(pr);
      if constexpr (FMT == E4B_FMT_NF4) sa[pset][ns] = *reinterpret_cast<const float*>(sexp + blk * 4u);
      else sq[pset][ns] = *reinterpret_cast<const uint8_t*>(sexp + blk);
    }
  };
  auto store_a = [&](int set) {
    *reinterpret_cast<u32x4_t*>(&As[ar * KS + ((ag ^ (ar & 15)) << 3)]) = areg[set][0];
    *reinterpret_cast<u32x4_t*>(&As[ar * KS + (((ag + 1) ^ (ar & 15)) << 3)]) = areg[set][1];
  };
  // loads first: their latency overlaps the table build
  load_a(0, 0);
  load_a(1, 1);
  load_scales(0, 0);
  load_w(0, 0);
  load_w(1, 1);
  load_scales(1, min(1, last >> 1));
  load_w(2, min(2, last));

  // ---- the code-pair table: thread t fills copy t % 64 of entries (t / 64) + 4 i
  {
    const int w0 = tid >> 6;
    float hi[16], lo[4];
#pragma unroll
    for (int c = 0; c < 16; ++c) hi[c] = p.w.code[c];
#pragma unroll
    for (int c = 0; c < 4; ++c) lo[c] = p.w.code[w0 + 4 * c];
#pragma unroll
    for (int i = 0; i < 256 / 4; ++i)
      ptab[(w0 + 4 * i) * kNarrowCopies + lane] = cvt_pair<E4B_FP16>(hi[i >> 2], lo[i & 3]);
  }
  if constexpr (FMT == E4B_FMT_NF4_DQ) code2_s[tid] = p.w.code2[tid];
  if ((tid & 7) == 0) row_shift_s[ar] = exp_shift(a_exp_row);
  store_a(0);
  load_a(0, min(2, last));
  __syncthreads();

  f32x4_t acc[MS][NS];
#pragma unroll
  for (int i = 0; i < MS; ++i)
#pragma unroll
    for (int j = 0; j < NS; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (LORA) {
    // the accumulators start as the tile's LoRA delta, scaled like the products (lora_mfma.h):
    // t rows of the lane's fragment rows (clamped to the expert's rows) times their activation
    // shifts, B rows of its columns as the weight loads took them (row 0 past n_out) times the
    // expert's weight shift
    int64_t brow[NS];
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) {
      if (pair) {
        const int64_t jj = col0 + wid * 32 + (ns & 1) * 16 + l16;
        brow[ns] = jj < p.n_out ? (ns < 2 ? jj : n / 2 + jj) : 0;
      } else {
        const int64_t rr = col0 + wid * 64 + ns * 16 + l16;
        brow[ns] = rr < p.n_out ? rr : 0;
      }
    }
    lora_delta_16x16<MS, NS>(p, acc, e, row0 + l16, row_end - 1,
                             [&](int ms) { return row_shift_s[ms * 16 + l16]; }, wsh, brow, lane);
  }

  // fragment group slots of the lane for MFMA j: (4 g + j) ^ (row % 16), row % 16 = lane % 16
  const int fslot = (4 * g) ^ l16;
  const int frow = l16 * KS;
  const uint32_t copy_off = static_cast<uint32_t>(lane) * 4u;
  auto lookup = [&](uint32_t w, uint32_t sel) -> uint32_t {
    const uint32_t addr = __builtin_amdgcn_perm(w, copy_off, sel);
    return *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(ptab) + addr);
  };
  auto scale_pair = [&](int pset, int ns, int pr) -> uint32_t {
    float sc;
    if constexpr (FMT == E4B_FMT_NF4) {
      sc = sa[pset][ns];
    } else {
      // fp32(fp32(code2 * absmax2) + offset): two roundings (no contraction under -ffp-contract=off)
      const float a2 = blk0[ns] + 4u * static_cast<uint32_t>(pr) < a2bound[ns] ? a2lo[ns] : a2hi[ns];
      const float prod = code2_s[sq[pset][ns]] * a2;
      sc = prod + offset;
    }
    sc = __builtin_amdgcn_ldexpf(sc, wsh);  // exact: a power of two
    return cvt_pair<E4B_FP16>(sc, sc);
  };

  uint32_t s2[NS];  // the block scale pairs of the current pair of steps
  // Table lookups of the four words (MFMA j) of each weight sub-tile: raw[j % 2], issued one
  // MFMA group ahead of their use, so that their LDS latency runs under the MFMAs.
  uint32_t raw[2][NS][4];
  auto look = [&](const uint4& wv, auto J, uint32_t (&dst)[4]) {
    constexpr int j = decltype(J)::value;
    const uint32_t w = j == 0 ? wv.x : j == 1 ? wv.y : j == 2 ? wv.z : wv.w;
    dst[0] = lookup(w, 0x0c0c0400u);
    dst[1] = lookup(w, 0x0c0c0500u);
    dst[2] = lookup(w, 0x0c0c0600u);
    dst[3] = lookup(w, 0x0c0c0700u);
  };

  // One step: the activation fragments from LDS into registers, a barrier (every wave has them),
  // the next step's activations stored into the one LDS buffer; for each MFMA group j and weight
  // sub-tile ns a chunk of four multiplies (the looked-up pairs times the block scale), the
  // lookups of group j + 1 (of the next step after j = 3) and the two MFMAs, closed by a
  // scheduling barrier; then the refill of the weight set and a barrier (the stores are in
  // place). The first barrier follows the fragment reads at once, so the waves reach it together
  // and only the second waits on the compute (a single buffer with both barriers after the
  // compute measured ~1 % slower at mid-size).
  auto step = [&](auto U, int s) __attribute__((always_inline)) {
    constexpr int u = decltype(U)::value;
    constexpr int set = u % ST;
    constexpr int nset = (u + 1) % ST;
    constexpr int aset = (u + 1) & 1;
    constexpr int pset = (u >> 1) % PS;  // this step's pair (s0 is a multiple of 2 * PS)
    uint4 fa[MS][4];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        fa[ms][j] = *reinterpret_cast<const uint4*>(&As[ms * 16 * KS + frow + ((fslot ^ j) << 3)]);
    __syncthreads();  // every wave has read this step's activations
    store_a(aset);    // step s + 1 (past the last step: a stale set, never read)
    load_a(aset, min(s + 3, last));
    if constexpr ((u & 1) == 0) {
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) s2[ns] = scale_pair(pset, ns, s >> 1);
    }
    static_for<4>([&](auto J) {
      constexpr int j = decltype(J)::value;
      static_for<NS>([&](auto NSI) {
        constexpr int ns = decltype(NSI)::value;
        uint4 bv;
        bv.x = pk_mul_f16(raw[j & 1][ns][0], s2[ns]);
        bv.y = pk_mul_f16(raw[j & 1][ns][1], s2[ns]);
        bv.z = pk_mul_f16(raw[j & 1][ns][2], s2[ns]);
        bv.w = pk_mul_f16(raw[j & 1][ns][3], s2[ns]);
        if constexpr (j < 3) look(wq[set][ns], std::integral_constant<int, j + 1>{}, raw[(j + 1) & 1][ns]);
        else look(wq[nset][ns], std::integral_constant<int, 0>{}, raw[0][ns]);
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) acc[ms][ns] = mfma_16x16x32<E4B_FP16>(fa[ms][j], bv, acc[ms][ns]);
        __builtin_amdgcn_sched_barrier(0);
      });
    });
    load_w(set, min(s + ST, last));
    // step s + 3 opens a pair when s is odd: its scales, into the set after the next pair's
    if constexpr (u & 1) load_scales(((u + 3) >> 1) % PS, min(s + 3, last) >> 1);
    __syncthreads();  // step s + 1's activations are in place
  };
  // the lookups of step 0, group 0
#pragma unroll
  for (int ns = 0; ns < NS; ++ns) look(wq[0][ns], std::integral_constant<int, 0>{}, raw[0][ns]);
  const int smain = steps - steps % kNarrowUnroll;
  for (int s0 = 0; s0 < smain; s0 += kNarrowUnroll) {
    static_for<kNarrowUnroll>([&](auto U) { step(U, s0 + decltype(U)::value); });
  }
  static_for<kNarrowUnroll - 1>([&](auto U) {
    if (smain + decltype(U)::value < steps) step(U, smain + decltype(U)::value);
  });

  // ---- epilogue: lane holds D[4 g + i][lane % 16] of each 16 x 16 sub-tile; the operand
  // scales come off first, 2^-(row shift + expert shift), exact
#pragma unroll
  for (int ms = 0; ms < MS; ++ms)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = H16 ? -p.out_f16_shift : -(row_shift_s[ms * 16 + 4 * g + i] + wsh);
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) acc[ms][ns][i] = __builtin_amdgcn_ldexpf(acc[ms][ns][i], d);
    }
  const bool has_bias = p.w.bias != nullptr;
  const uint16_t* bias = static_cast<const uint16_t*>(p.w.bias);
  if (!H16 && pair) {
    const int64_t cbase = col0 + wid * 32 + l16;
    if (p.epi == E4B_EPI_SWIGLU && !has_bias && !p.out_f32) {  // gate_up: silu(g) * u -> bf16
      uint16_t* const out = static_cast<uint16_t*>(p.out);
#pragma unroll
      for (int ms = 0; ms < MS; ++ms)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int rr = row0 + ms * 16 + 4 * g + i;
          uint16_t* const orow = out + int64_t(rr) * p.n_out + cbase;
#pragma unroll
          for (int ns = 0; ns < 2; ++ns) {
            const float v = silu_f32(acc[ms][ns][i]) * acc[ms][ns + 2][i];
            if (rr < row_end && cbase + ns * 16 < p.n_out) orow[ns * 16] = from_f<E4B_BF16>(v);
          }
        }
      return;
    }
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rr = row0 + ms * 16 + 4 * g + i;
        if (rr >= row_end) continue;
#pragma unroll
        for (int ns = 0; ns < 2; ++ns) {
          const int64_t jj = cbase + ns * 16;
          if (jj >= p.n_out) continue;
          const float bg = has_bias ? to_f<E4B_BF16>(bias[int64_t(e) * n + jj]) : 0.0f;
          const float bu = has_bias ? to_f<E4B_BF16>(bias[int64_t(e) * n + n / 2 + jj]) : 0.0f;
          store_elem<E4B_BF16>(p, int64_t(rr) * p.n_out + jj,
                               gated(p.epi, acc[ms][ns][i], acc[ms][ns + 2][i], p.alpha, p.limit, bg, bu));
        }
      }
    return;
  }
  const int64_t cbase = col0 + wid * 64 + l16;
  if constexpr (H16) {  // down: fp16 rows, the operand scales left on (the host checks the form)
    uint16_t* const out = static_cast<uint16_t*>(p.out);
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rr = row0 + ms * 16 + 4 * g + i;
        uint16_t* const orow = out + int64_t(rr) * p.n_out + cbase;
#pragma unroll
        for (int ns = 0; ns < NS; ++ns)
          if (rr < row_end && cbase + ns * 16 < p.n_out) orow[ns * 16] = from_f<E4B_FP16>(acc[ms][ns][i]);
      }
    return;
  }
  if (p.epi == E4B_EPI_NONE && !has_bias && p.out_f32) {  // down: fp32 rows
    float* const out = static_cast<float*>(p.out);
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rr = row0 + ms * 16 + 4 * g + i;
        float* const orow = out + int64_t(rr) * p.n_out + cbase;
#pragma unroll
        for (int ns = 0; ns < NS; ++ns)
          if (rr < row_end && cbase + ns * 16 < p.n_out) orow[ns * 16] = acc[ms][ns][i];
      }
    return;
  }
#pragma unroll
  for (int ms = 0; ms < MS; ++ms)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rr = row0 + ms * 16 + 4 * g + i;
      if (rr >= row_end) continue;
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) {
        const int64_t nn = cbase + ns * 16;
        if (nn >= p.n_out) continue;
        const float b = has_bias ? to_f<E4B_BF16>(bias[int64_t(e) * n + nn]) : 0.0f;
        store_elem<E4B_BF16>(p, int64_t(rr) * p.n_out + nn, single(p.epi, acc[ms][ns][i], b));
      }
    }
  };
  // (the row count is the same in every lane; readfirstlane makes the branch a scalar one)
  if (__builtin_amdgcn_readfirstlane(row_end - row0) <= 16) run_tile(std::integral_constant<int, 1>{});
  else run_tile(std::integral_constant<int, 2>{});
}

}  // namespace e4b
