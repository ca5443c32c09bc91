// Prefill grouped GEMM, wide tiles: 256 sorted rows x 256 weight rows per workgroup, four waves
// (one per SIMD) of 128 x 128 each, on v_mfma_f32_32x32x16_{bf16,f16}.
//
// The 128 x 256 tile of gemm_mfma_kernel gives each of its eight waves a 64 x 64 block: per
// 64-deep step a CU then moves 48 KB of staged operands and 128 KB of MFMA fragments through
// LDS for 2M multiply-adds, and decodes every weight for 128 rows. Here a 128 x 128 wave block
// halves the fragment bytes per multiply-add (128 KB for 4M), and every decoded weight feeds 256
// rows, half the decode work. One wave per SIMD holds 256 accumulator registers (AGPRs); the
// fragments are double-buffered per 16-deep sub-step (2 x 32 registers); global loads run two
// steps ahead in two register sets.
//
// With one wave per SIMD nothing else hides a stall, so the main loop is laid out by hand: each
// 64-deep step is four 16-deep sub-steps of sixteen MFMAs, cut into chunks of four MFMAs (one
// accumulator row) by scheduling barriers, with the staging of a later step (a weight word's
// decode, an activation store) and the global loads placed between them; an MFMA then hides
// about six VALU instructions of its own wave (measured: 32 cycles per MFMA alone, ~35 with
// four VALU, ~40 with six, ~49 with eight). Step s + 2 is staged from sub-step 3 of step s into
// the buffer step s has just released, through sub-steps 0-2 of step s + 1; the activation
// loads take 128 contiguous bytes per eight lanes (a load with one 16-byte row piece per lane
// costs the load pipeline about twice the issue time). The decode is that of gemm_mfma_kernel
// (dequant_bytes' byte-plane lookups, the fp16 matrix-core mode's row and expert shifts), so the
// two kernels form the same per-element products; only the fp32 summation order differs.
//
// The output layout of a 32 x 32 MFMA: lane l holds column l % 32 of rows
// 8 * (i / 4) + 4 * (l / 32) + i % 4, i = 0..15, of its tile.
#pragma once

#include "gemm.h"
#include "lora_mfma.h"

namespace e4b {

constexpr int kWideThreads = 256;
constexpr int kWideTileM = kTileMBig;  // sorted rows per tile
constexpr int kWideTileN = 256;  // weight rows per tile

// LDS tile layout of this kernel: 128-byte rows of 64 elements, the row's eight 16-byte groups in
// the order group ^ ((row ^ (row >> 3)) & 7). Measured with SQ_LDS_BANK_CONFLICT on the two
// access patterns: a 32 x 32 fragment read (32 consecutive rows at one group) and the staging
// stores (thread t: row t, one group per store) are both conflict-free. (group ^ (row & 7), the
// layout of gemm_mfma_kernel, costs the fragment reads a 2-way conflict, and group ^ ((row >> 1)
// & 7) the stores.)
E4B_DEV int lds_at_w(int row, int col) { return row * kTileK + ((((col >> 3) ^ row ^ (row >> 3)) & 7) << 3); }

// One tile. HALF: a tile of at most 128 rows (an expert's last, partial tile) as 128 rows x 256
// weight rows, each wave 128 x 64 (two 32 x 32 MFMA columns), instead of padding it to 256 rows.
// LORA: the accumulators start as the tile's LoRA delta (p.lt, p.lb), scaled like the products
// (lora_mfma.h).
template <int DT, int FMT, bool F16C, bool HALF, bool LORA>
E4B_DEV void wide_tile(const GemmArgs& p, int tile, int n_tile, uint16_t (&As)[2][kWideTileM * kTileK],
                       uint16_t (&Ws)[2][kWideTileN * kTileK], float* code2_s, int* row_shift_s,
                       const uint32_t* ptab) {
  constexpr bool PTAB = F16C;  // fp16 mode: weights decoded through the LDS table of code pairs
  constexpr int CT = F16C ? E4B_FP16 : DT;
  constexpr int BM = kWideTileM, BN = kWideTileN;
  constexpr int MS = 4, NS = HALF ? 2 : 4;  // 32 x 32 MFMA tiles per wave: 128 x 32 NS
  constexpr int WCOL = 32 * NS;             // weight rows per wave
  constexpr int AP = HALF ? 4 : 8;          // activation pieces per thread and step
  constexpr int ST = 2;                     // register sets of global loads in flight
  const bool pair = is_gated(p.epi);
  const int cols = pair ? BN / 2 : BN;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wid = __builtin_amdgcn_readfirstlane(tid) / kWave;  // wave-uniform: a scalar register
  const int wave_m = HALF ? 0 : (wid & 1);
  const int wave_n = HALF ? wid : (wid >> 1);
  const int e = p.rt.tiles[2 * tile];
  const int row0 = p.rt.tiles[2 * tile + 1];
  const int row_end = min(row0 + BM, p.rt.offsets[e + 1]);
  const int64_t n = p.w.n;
  const int64_t k = p.w.k;
  const int64_t col0 = int64_t(n_tile) * cols;
  if (col0 >= p.n_out) return;

  float code[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) code[i] = (FMT == E4B_FMT_MXFP4) ? kFp4E2M1[i] : p.w.code[i];
  if constexpr (FMT == E4B_FMT_NF4_DQ) code2_s[tid] = p.w.code2[tid];

  // A: a step's 256 x 64 tile is 2048 16-byte pieces; load i (0..7) of thread t takes tile row
  // 32 i + t / 8, columns 8 (t % 8) .. + 7, so eight lanes read one row's 128 contiguous bytes
  // (one lane per row, 16 bytes from each of 64 rows per load, costs the load pipeline about
  // twice the issue time). aoff[i]: that piece of step 0, in 16-byte units of p.a.
  // The rows' sources (and tile row t's, for the row shifts) are loaded together at clamped
  // indices, before row_end is known, and dropped for rows past the expert's end: a load behind
  // the row test, divided inside that branch, was waited on alone, one round trip per piece.
  const int apart = tid & 7;
  const bool gather = p.gather_k > 0;
  const int mlast = static_cast<int>(p.M) - 1;
  int sf[AP + 1];
#pragma unroll
  for (int i = 0; i <= AP; ++i) {
    const int r = min(row0 + (i < AP ? 32 * i + (tid >> 3) : tid), mlast);
    const int v = p.rt.sorted_flat[r];
    sf[i] = gather ? v : r;
  }
  auto row_src = [&](int r, int s) -> int64_t { return r < row_end ? (gather ? s / p.gather_k : s) : 0; };
  uint32_t aoff[AP];
#pragma unroll
  for (int i = 0; i < AP; ++i)
    aoff[i] = static_cast<uint32_t>((row_src(row0 + 32 * i + (tid >> 3), sf[i]) * k) / 8 + apart);
  int wsh = 0;
  if constexpr (F16C) {
    wsh = p.w.shift[e];
    // row_shift_s: the shift of tile row tid, for the epilogue
    row_shift_s[tid] = exp_shift(p.a_exp[row_src(row0 + tid, sf[AP])]);
  }
  // W: thread tid stages LDS weight row tid (for a gated epilogue rows 0..127 are the gate rows
  // of the tile's 128 output columns and rows 128..255 their up rows); rows past n_out read
  // weight row 0 and feed only columns that are never stored
  int64_t grow;
  if (pair) {
    const int64_t jj = col0 + (tid & (BN / 2 - 1));
    grow = jj < p.n_out ? ((tid < BN / 2) ? jj : n / 2 + jj) : 0;
  } else {
    grow = col0 + tid < p.n_out ? col0 + tid : 0;
  }
  const uint8_t* wptr = p.w.packed + (int64_t(e) * n + grow) * (k / 2);
  const int64_t nb = n * (k / 64);
  const float offset = (FMT == E4B_FMT_NF4_DQ) ? p.w.offset[e] : 0.0f;

  f32x16_t acc[MS][NS];
  static_for<MS>([&](auto ms) { static_for<NS>([&](auto ns) { acc[ms][ns] = f32x16_t{}; }); });

  u32x4_t areg[AP];  // one set: a step's activations are loaded and staged within one step
  uint32_t wq[ST][8];
  float sa[ST];
  uint32_t sq[ST];
  // the global loads of a step: activation piece i, and the weight row's bytes and scales
  auto load_a = [&](int64_t kb, int i) {
    if (i >= AP) return;  // (i is a constant at every call)
    areg[i] = (reinterpret_cast<const u32x4_t*>(p.a) + kb * (kTileK / 8))[aoff[i]];
  };
  auto load_w = [&](int set, int64_t kb) {
    const uint4 v0 = *reinterpret_cast<const uint4*>(wptr + kb * 32);
    const uint4 v1 = *reinterpret_cast<const uint4*>(wptr + kb * 32 + 16);
    wq[set][0] = v0.x; wq[set][1] = v0.y; wq[set][2] = v0.z; wq[set][3] = v0.w;
    wq[set][4] = v1.x; wq[set][5] = v1.y; wq[set][6] = v1.z; wq[set][7] = v1.w;
    if constexpr (FMT == E4B_FMT_MXFP4) {  // both e8m0 scales of the step (k % 64 == 0: aligned)
      sq[set] = reinterpret_cast<const uint16_t*>(p.w.absmax)[((int64_t(e) * n + grow) * (k / 32) + kb * 2) / 2];
    } else if constexpr (FMT == E4B_FMT_NF4) {
      sa[set] = static_cast<const float*>(p.w.absmax)[e * nb + grow * (k / 64) + kb];
    } else {
      const int64_t blk = grow * (k / 64) + kb;
      sq[set] = static_cast<const uint8_t*>(p.w.absmax)[e * nb + blk];
      sa[set] = p.w.absmax2[e * ((nb + 255) / 256) + blk / 256];
    }
  };
  auto load_a_all = [&](int64_t kb) {
#pragma unroll
    for (int i = 0; i < AP; ++i) load_a(kb, i);
  };
  // The NF4 block scale of a staged step, formed one sub-step ahead of its staging: the
  // double-quant scale reads code2 from LDS, and a wait for that read in the staging would also
  // wait for every fragment read issued before it, holding the decode back behind the MFMAs.
  auto block_scale = [&](int set) {
    float scale = 0.0f;
    if constexpr (FMT == E4B_FMT_NF4) {
      scale = sa[set];
    } else if constexpr (FMT == E4B_FMT_NF4_DQ) {
      const float prod = code2_s[sq[set]] * sa[set];
      scale = prod + offset;
    }
    if constexpr (F16C) scale = __builtin_amdgcn_ldexpf(scale, wsh);
    return scale;
  };
  // Staging of one step, in pieces the main loop spreads over the MFMAs: the activation row
  // (eight 16-byte stores; converted to scaled fp16 in fp16 mode 1) and the weight row, one
  // packed word (eight values, one 16-byte store) at a time.
  auto store_a = [&](int buf, int i) {
    if (i >= AP) return;  // (i is a constant at every call)
    *reinterpret_cast<u32x4_t*>(&As[buf][lds_at_w(32 * i + (tid >> 3), 8 * apart)]) = areg[i];
  };
  // A weight word in two halves, so the table lookups of the fp16 mode can be issued a chunk
  // before the multiplies that wait for them: fetch_w leaves in r the looked-up code pairs
  // (fp16 mode) or the decoded values, put_w applies the scale pair t.lo[0] (fp16 mode) and
  // stores the word's eight values.
  auto fetch_w = [&](int set, int wi, const NibPlanes& t, uint32_t (&r)[4]) {
    if constexpr (FMT == E4B_FMT_MXFP4) {  // words 0-3: the first 32-value block, 4-7: the second
      fp4_word<CT>(wq[set][wi], e8m0_to_f32(wi < 4 ? (sq[set] & 0xffu) : (sq[set] >> 8)), r);
    } else if constexpr (PTAB) {  // byte b's code pair from the lane's table copy
      const uint32_t* tab = ptab + (lane & (kPairCopies - 1));
      const uint32_t w = wq[set][wi];
#pragma unroll
      for (int b = 0; b < 4; ++b) r[b] = tab[((w >> (8 * b)) & 0xffu) * kPairCopies];
    } else {
      nib_word<FMT>(t, wq[set][wi], r);
    }
  };
  auto put_w = [&](int buf, int wi, const NibPlanes& t, const uint32_t (&r)[4]) {
    uint32_t o[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) o[b] = PTAB ? pk_mul_f16(r[b], t.lo[0]) : r[b];
    *reinterpret_cast<uint4*>(&Ws[buf][lds_at_w(tid, 8 * wi)]) = make_uint4(o[0], o[1], o[2], o[3]);
  };
  auto store_w = [&](int set, int buf, int wi, const NibPlanes& t) {
    uint32_t r[4];
    fetch_w(set, wi, t, r);
    put_w(buf, wi, t, r);
  };
  auto planes = [&](float scale) {
    if constexpr (FMT == E4B_FMT_MXFP4) {
      return NibPlanes{};
    } else if constexpr (PTAB) {  // the table decode needs only the scale, as an fp16 pair
      NibPlanes t{};
      t.lo[0] = cvt_pair<E4B_FP16>(scale, scale);
      return t;
    } else {
      return nib_planes<CT, !F16C>(code, scale);
    }
  };
  auto stage = [&](int set, int buf, float scale) {
    const NibPlanes t = planes(scale);
#pragma unroll
    for (int i = 0; i < AP; ++i) store_a(buf, i);
#pragma unroll
    for (int wi = 0; wi < 8; ++wi) store_w(set, buf, wi, t);
  };
  // Fragments of sub-step ks (k = 16 ks .. 16 ks + 15): lane l reads row (base + l % 32), the
  // eight values at k = 16 ks + 8 (l / 32). Every base is a multiple of 32, so the row's swizzle
  // term is (l & 7) ^ ((l >> 3) & 3) ^ 4 (base / 32 & 1): bpar[ns] for the weight fragments,
  // ms & 1 for the activation ones (whose bases are ms * 32 past a multiple of 64).
  int nbase[NS], bpar[NS];
#pragma unroll
  for (int ns = 0; ns < NS; ++ns) {
    nbase[ns] = pair ? ((ns < NS / 2) ? wave_n * (WCOL / 2) + ns * 32 : BN / 2 + wave_n * (WCOL / 2) + (ns - NS / 2) * 32)
                     : wave_n * WCOL + ns * 32;
    bpar[ns] = ((nbase[ns] >> 5) & 1) << 5;
  }
  const int a_frag = (wave_m * 128 + (lane & 31)) * kTileK;
  const int w_frag = (lane & 31) * kTileK;
  auto read_frags = [&](int buf, int ks, uint4 (&av)[MS], uint4 (&bv)[NS]) {
    const int fcol = (((2 * ks + (lane >> 5)) ^ lane ^ ((lane >> 3) & 3)) & 7) << 3;
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
      av[ms] = *reinterpret_cast<const uint4*>(&As[buf][a_frag + ms * 32 * kTileK + (fcol ^ ((ms & 1) << 5))]);
#pragma unroll
    for (int ns = 0; ns < NS; ++ns)
      bv[ns] = *reinterpret_cast<const uint4*>(&Ws[buf][w_frag + nbase[ns] * kTileK + (fcol ^ bpar[ns])]);
  };
  auto mfma_row = [&](int ms, const uint4 (&av)[MS], const uint4 (&bv)[NS]) {
    static_for<NS>([&](auto ns) { acc[ms][ns] = mfma_32x32x16<CT>(av[ms], bv[ns], acc[ms][ns]); });
  };
  auto mfmas = [&](const uint4 (&av)[MS], const uint4 (&bv)[NS]) {
    static_for<MS>([&](auto ms) {
      static_for<NS>([&](auto ns) { acc[ms][ns] = mfma_32x32x16<CT>(av[ms], bv[ns], acc[ms][ns]); });
    });
  };

  const int64_t ksteps = k / kTileK;
  const int64_t klast = ksteps - 1;
  // Prologue: step 0 staged whole into buffer 0; of step 1, the part an iteration's sub-step 3
  // stages (the weight row's code planes, its first two words, the activation row).
  static_assert(ST == 2, "step s lives in weight register set s % 2");
  load_a_all(0);
  load_w(0, 0);
  load_w(1, min<int64_t>(1, klast));
  __syncthreads();  // code2 table, row shifts
  if constexpr (LORA) {
    // the accumulators start as the tile's LoRA delta, scaled like the products (lora_mfma.h):
    // the lane's t rows (clamped to the expert's rows: the rest is never stored) times their
    // activation shifts, the B rows of its columns (weight row 0 past n_out) times the expert's
    // weight shift
    const int la = lane;
    int64_t brow[NS];
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) {
      const int tr = nbase[ns] + (la & 31);
      if (pair) {
        const int64_t jj = col0 + (tr & (BN / 2 - 1));
        brow[ns] = jj < p.n_out ? (tr < BN / 2 ? jj : n / 2 + jj) : 0;
      } else {
        brow[ns] = col0 + tr < p.n_out ? col0 + tr : 0;
      }
    }
    const int arow = wave_m * 128 + (la & 31);
    lora_delta_32x32<MS, NS>(p, acc, e, row0 + arow, row_end - 1,
                             [&](int ms) { return row_shift_s[arow + 32 * ms]; }, wsh, brow, la);
  }
  stage(0, 0, block_scale(0));
  load_a_all(min<int64_t>(1, klast));
  load_w(0, min<int64_t>(2, klast));
  NibPlanes tp = planes(block_scale(1));
#pragma unroll
  for (int i = 0; i < AP; ++i) store_a(1, i);
  store_w(1, 1, 0, tp);
  store_w(1, 1, 1, tp);
  uint32_t lk[4];  // a word's fetched half, carried to the next chunk
  fetch_w(1, 2, tp, lk);
  __syncthreads();
  uint4 fa0[MS], fb0[NS], fa1[MS], fb1[NS];
  read_frags(0, 0, fa0, fb0);
  // Step kb in sixteen chunks of four MFMAs (one accumulator row), each closed by a scheduling
  // barrier so the staging pieces stay between them: a weight word's decode (about 26 VALU
  // instructions) next to four 32-cycle MFMAs. The staging of a step is spread over four
  // sub-steps: step kb + 2 starts in sub-step 3 of step kb, into buffer kb % 2 (free once the
  // barrier has passed: its last fragments were read before it), and ends in sub-steps 0-2 of
  // step kb + 1, whose sub-step 2 then reloads its register set with step kb + 3. Each sub-step
  // reads the next one's fragments at its start. (The compiler left to itself puts the MFMAs
  // ahead of the decode, and with one wave per SIMD the matrix core then idles through it.)
  auto iteration = [&](auto uc, int64_t kb) __attribute__((always_inline)) {
    constexpr int u = decltype(uc)::value;
    constexpr int sS = (u + 1) % ST;  // register set of step kb + 1, whose staging ends here
    constexpr int sT = u;             // register set of step kb + 2, whose staging starts here
    const int cur = static_cast<int>(kb & 1);
    // sub-step 0 (the activation registers were staged in the previous sub-step 3: the loads of
    // step kb + 2's activations go out here, two per chunk, and are staged in sub-step 3)
    const int64_t knext = min<int64_t>(kb + 1 + ST, klast);
    const int64_t ka = min<int64_t>(kb + 2, klast);
    read_frags(cur, 1, fa1, fb1);
    mfma_row(0, fa0, fb0);
    put_w(cur ^ 1, 2, tp, lk);
    fetch_w(sS, 3, tp, lk);
    load_a(ka, 0);
    load_a(ka, 1);
    __builtin_amdgcn_sched_barrier(0);
    mfma_row(1, fa0, fb0);
    load_a(ka, 2);
    load_a(ka, 3);
    __builtin_amdgcn_sched_barrier(0);
    mfma_row(2, fa0, fb0);
    put_w(cur ^ 1, 3, tp, lk);
    fetch_w(sS, 4, tp, lk);
    __builtin_amdgcn_sched_barrier(0);
    mfma_row(3, fa0, fb0);
    load_a(ka, 4);
    load_a(ka, 5);
    __builtin_amdgcn_sched_barrier(0);
    // sub-step 1 (with the block scale of step kb + 2, whose set sT was loaded a step ago: its
    // code2 read is then long done when sub-step 3 stages the step)
    read_frags(cur, 2, fa0, fb0);
    mfma_row(0, fa1, fb1);
    put_w(cur ^ 1, 4, tp, lk);
    fetch_w(sS, 5, tp, lk);
    __builtin_amdgcn_sched_barrier(0);
    mfma_row(1, fa1, fb1);
    load_a(ka, 6);
    load_a(ka, 7);
    const float sc = block_scale(sT);
    __builtin_amdgcn_sched_barrier(0);
    mfma_row(2, fa1, fb1);
    put_w(cur ^ 1, 5, tp, lk);
    fetch_w(sS, 6, tp, lk);
    __builtin_amdgcn_sched_barrier(0);
    mfma_row(3, fa1, fb1);
    __builtin_amdgcn_sched_barrier(0);
    // sub-step 2
    read_frags(cur, 3, fa1, fb1);
    mfma_row(0, fa0, fb0);
    put_w(cur ^ 1, 6, tp, lk);
    fetch_w(sS, 7, tp, lk);
    __builtin_amdgcn_sched_barrier(0);
    mfma_row(1, fa0, fb0);
    put_w(cur ^ 1, 7, tp, lk);
    __builtin_amdgcn_sched_barrier(0);
    mfma_row(2, fa0, fb0);
    load_w(sS, knext);  // the weight registers of set sS are free after word 7
    __builtin_amdgcn_sched_barrier(0);
    mfma_row(3, fa0, fb0);
    const NibPlanes tn = planes(sc);  // step kb + 2's planes, while this step's are still in use
    __syncthreads();
    // sub-step 3
    read_frags(cur ^ 1, 0, fa0, fb0);
    mfma_row(0, fa1, fb1);
    tp = tn;
    store_a(cur, 0);
    store_a(cur, 1);
    fetch_w(sT, 0, tp, lk);
    __builtin_amdgcn_sched_barrier(0);
    mfma_row(1, fa1, fb1);
    put_w(cur, 0, tp, lk);
    fetch_w(sT, 1, tp, lk);
    store_a(cur, 2);
    store_a(cur, 3);
    __builtin_amdgcn_sched_barrier(0);
    mfma_row(2, fa1, fb1);
    put_w(cur, 1, tp, lk);
    fetch_w(sT, 2, tp, lk);
    store_a(cur, 4);
    store_a(cur, 5);
    __builtin_amdgcn_sched_barrier(0);
    mfma_row(3, fa1, fb1);
    store_a(cur, 6);
    store_a(cur, 7);
    __builtin_amdgcn_sched_barrier(0);
  };
  const int64_t kmain = ksteps - ksteps % ST;
  for (int64_t kb0 = 0; kb0 < kmain; kb0 += ST) {
    iteration(std::integral_constant<int, 0>{}, kb0);
    iteration(std::integral_constant<int, 1>{}, kb0 + 1);
  }
  if (kmain < ksteps) iteration(std::integral_constant<int, 0>{}, kmain);

  // Epilogue. Tile row of accumulator register i of MFMA tile ms; the lane's column is
  // nbase[ns] + (lane & 31). The lane index is formed again here (v_mbcnt): values kept from
  // before the loop would be spilled across it, and a scratch reload in the epilogue waits for
  // every store issued before it.
  const int lane_e = static_cast<int>(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)));
  auto row_of = [&](int ms, int i) { return wave_m * 128 + ms * 32 + 8 * (i >> 2) + 4 * (lane_e >> 5) + (i & 3); };
  if constexpr (F16C) {
    static_for<MS>([&](auto ms) {
      static_for<16>([&](auto i) {
        const int d = -(row_shift_s[row_of(ms, i)] + wsh);
        static_for<NS>([&](auto ns) { acc[ms][ns][int(i)] = __builtin_amdgcn_ldexpf(acc[ms][ns][int(i)], d); });
      });
    });
  }
  const bool has_bias = p.w.bias != nullptr;
  const uint16_t* bias = static_cast<const uint16_t*>(p.w.bias);
  if (pair && p.epi == E4B_EPI_SWIGLU && !has_bias && !p.out_f32) {  // gate_up: silu(g) * u -> dt
    uint16_t* const out = static_cast<uint16_t*>(p.out);
    const int64_t cbase = col0 + wave_n * (WCOL / 2) + (lane_e & 31);
    static_for<MS>([&](auto ms) {
      static_for<16>([&](auto i) {
        const int rr = row0 + row_of(ms, i);
        uint16_t* const orow = out + int64_t(rr) * p.n_out + cbase;
        static_for<NS / 2>([&](auto ns) {
          const float v = silu_f32(acc[ms][ns][int(i)]) * acc[ms][ns + NS / 2][int(i)];
          if (rr < row_end && cbase + ns * 32 < p.n_out) orow[ns * 32] = from_f<DT>(v);
        });
      });
    });
    return;
  }
  if (!pair && p.epi == E4B_EPI_NONE && !has_bias && p.out_f32) {  // down: fp32 rows
    float* const out = static_cast<float*>(p.out);
    const int64_t cbase = col0 + wave_n * WCOL + (lane_e & 31);
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
          static_for<NS / 2>([&](auto ns) {
            const int64_t jj = col0 + wave_n * (WCOL / 2) + ns * 32 + (lane_e & 31);
            if (jj < p.n_out) {
              const float bg = has_bias ? to_f<DT>(bias[int64_t(e) * n + jj]) : 0.0f;
              const float bu = has_bias ? to_f<DT>(bias[int64_t(e) * n + n / 2 + jj]) : 0.0f;
              store_elem<DT>(p, orow + jj,
                             gated(p.epi, acc[ms][ns][int(i)], acc[ms][ns + NS / 2][int(i)], p.alpha, p.limit, bg, bu));
            }
          });
        } else {
          static_for<NS>([&](auto ns) {
            const int64_t nn = col0 + wave_n * WCOL + ns * 32 + (lane_e & 31);
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

template <int DT, int FMT, bool F16C = false, bool LORA = false>
__global__ void __launch_bounds__(kWideThreads) gemm_wide_kernel(GemmArgs p) {
  static_assert(!F16C || (DT == E4B_BF16 && FMT != E4B_FMT_MXFP4), "fp16 mode: bf16 activations, NF4 weights");
  static_assert(!LORA || F16C, "the LoRA epilogue runs in the fp16 mode");
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
  const int tile = item.tile, n_tile = item.n_tile;
  if constexpr (F16C) {
    // the table of code pairs: pass j fills entries 16 j .. 16 j + 15, all copies; entry
    // 16 j + t / 16 of copy t % 16 (high nibble j, low nibble t / 16)
    static_assert(kWideThreads == 16 * kPairCopies, "table fill");
    const float lo = p.w.code[threadIdx.x / kPairCopies];
#pragma unroll
    for (int j = 0; j < 16; ++j) ptab[j * kWideThreads + threadIdx.x] = cvt_pair<E4B_FP16>(p.w.code[j], lo);
  }
  const int rows = p.rt.offsets[item.e + 1] - item.row0;  // the tile's rows, capped at BM below
  if (rows <= BM / 2) wide_tile<DT, FMT, F16C, true, LORA>(p, tile, n_tile, As, Ws, code2_s, row_shift_s, ptab);
  else wide_tile<DT, FMT, F16C, false, LORA>(p, tile, n_tile, As, Ws, code2_s, row_shift_s, ptab);
}

}  // namespace e4b
