// Decode path (tokens * top_k <= 64): the whole MoE layer in two launches, no routing round trip.
//
//   decode_up_kernel    block (column tile, a): gate_up GEMV of the a-th routed expert (ascending
//                       id) for a tile of output columns, fused epilogue, writes h[flat, :]
//                       (flat = token * k + slot). One token.
//   decode_up_items_kernel  the same GEMV for 2..8 tokens whose activations fit in LDS: one
//                       block per CU stages every token once, and its waves take (routed
//                       expert, column group) items in turn.
//   decode_down_kernel  block = kDownCols output columns: the down GEMV of every routed row for
//                       those columns, then the deterministic k-slot combine of the columns in
//                       slot order -- the combine never leaves the block. A G-lane group takes
//                       one routed expert at a time (a "job") for all the block's columns, so a
//                       routed row's activation chunk is loaded once per job.
//
// Critical path of either kernel: one global round trip for the ids (issued together with the
// code table and, for down, the router weights the combine uses), a wave-local routing step,
// then every weight / scale / activation load of the block is issued -- interleaved by chunk,
// so the dot products can start on the first chunk while later ones are in flight. The LDS
// decode table is written around that issue (before it in the up kernel, after it in the down
// kernel, whichever measured faster), and one __syncthreads separates the table build from
// its use. Each wave computes the routing itself (one id per lane, a per-wave LDS bitmap of
// routed experts, one LDS atomic per lane for the row masks), so no block barrier waits on it.
//
// Weight decode. e2m1 bytes are converted in registers: one v_cvt_scalef32_pk_{bf16,f16}_fp4
// (scale 1) turns a byte into its two codes as an activation-dtype pair, exact in either type.
// NF4 goes through a 64 KB LDS table that holds, for every byte value b, the two codes the byte
// encodes, one 256-byte row per byte value, in one of two forms:
//   single  one 4-byte entry (two 16-bit codes), 32 copies in the first half of the row, lane
//           l reads copy l % 32: NF4 codes in fp16 (up kernels).
//   split   NF4 codes as activation-dtype pairs hi = dt(code), lo = dt(code - hi), so hi + lo
//           carries the fp32 code to ~16 significant bits (8-byte entries, 32 copies, lane l
//           reads copy l % 32): the down kernel, whose activations are read straight from
//           global memory in the activation dtype.
// A byte's table address is one v_perm_b32 (byte -> bits 8..15, lane copy offset -> bits
// 0..7); an element pair then costs one ds_read_b32 and one v_dot2 (single) or one ds_read_b64
// and two v_dot2 (split) against the packed activation pair. The block scale multiplies the
// fp32 sum once per 32 values.
//
// fp16 NF4 codes (up kernel). An fp16 code is within 2^-11 relative of the fp32 code and an
// fp16 x fp16 product is exact in fp32, so the only new error is that rounding of the code --
// 8x below a bf16 code's and far below the rounding of h itself. bf16 activations are restaged
// through LDS as fp16 scaled by a power of two per 32-value chunk (the chunk maximum lands in
// [2^14, 2^15)): bf16's 8 significant bits fit fp16's 11, so every element at least 2^-28 of
// its chunk's maximum converts exactly, and the chunk's dot product is scaled back once. Against
// the split bf16 table this removes one of the two v_dot2 per byte and halves the table read.
//
// Chunk c (16 packed bytes = 32 values) of a row goes to lane gl = c % G of the row's group,
// as its (c / G)-th chunk. When the row's chunk count is not a multiple of G the spare slots
// load chunk 0 and their products are dropped by a select, so no load is behind a branch.
//
// LoRA variants (template LR > 0, ranks up to LR): every routed row f carries t[f, :] = x_f .
// A[e]^T from a small preceding launch; a weight row's fp32 sum gains lscale * t[f, :] . B[e,
// row, :] before the epilogue (up) or the combine (down). The G lanes of the row's group split
// the rank, so the delta costs one fused multiply-add per rank slot and rides the existing
// group reduction; B is loaded with the weights, t with the row's activations.
#pragma once

#include "common.h"
#include "dequant.h"

namespace e4b {

constexpr int kDecThreads = 256;
constexpr int kDecWaves = kDecThreads / kWave;
constexpr int kDecMaxRows = kWave;   // tokens * top_k: one routed row per lane
constexpr int kDecMaxExperts = 256;
constexpr int kDecExpWords = kDecMaxExperts / 64;
constexpr int kLutRowBytes = 256;  // one table row per byte value: 256 rows, 64 KB

// Table geometry: split entries carry (hi, lo) pairs, single entries the codes alone. 32 copies
// either way (LDS serves a wave's reads in half-waves, so lane l reading copy l % 32 is
// conflict-free); single entries fill the first half of each 256-byte row, so a byte's address
// stays one v_perm_b32 (byte -> bits 8..15) and the table build stores half as much.
template <bool SPLIT>
struct LutGeom {
  static constexpr int kEntryBytes = SPLIT ? 8 : 4;
  static constexpr int kCopies = 32;
  static constexpr int kFillBytes = kCopies * kEntryBytes;
  static_assert(kFillBytes <= kLutRowBytes, "copies fit a row");
  // byte offset of lane's copy within a row
  static E4B_DEV uint32_t lane_off(int lane) { return static_cast<uint32_t>(lane % kCopies) * kEntryBytes; }
};
constexpr int kDownCols = 4;         // output columns per decode_down block
// decode_up_kernel: chunks per lane issued before the table barrier, the rest at the chunk loop's
// steps. Only NF4 defers, and at most two chunks: its steps are long (table lookups), so a
// deferred chunk is issued two steps before its use (OLMoE / Qwen3 double-quant bs=1 per layer,
// four chunks per lane: 15.33 / 14.85 us with all four up front, 15.04 / 13.84 with two). e2m1
// steps are short, and deferring four of six chunks there took gpt-oss bs=1 from 20.3 to 28.2 us.
template <int FMT, int CPL>
constexpr int up_issue_chunks() {
  return FMT == E4B_FMT_MXFP4 || CPL <= 2 ? CPL : CPL <= 4 ? 2 : CPL - 2;
}
constexpr int kDecMaxK = 4096;       // longest row the decode kernels take

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
  // LoRA delta (the LORA kernel variants): lt [T*k, lr] fp32 holds t = x . A[e]^T of every flat
  // row; lb is B [E, w.n, lr] in lbdt; weight row `row` of flat row f gains
  // lscale * sum_q lt[f, q] * B[e, row, q] in fp32 before its epilogue / combine.
  const float* lt;
  const void* lb;
  int lbdt, lr;
  float lscale;
};

// Every kernel argument a decode kernel reads, requested in one batch at its entry: left to
// itself the compiler loads each just before its first use, so the pointers first read after
// the routing (weights, scales, outputs) cost a scalar-cache round trip of their own. (Not in
// the LoRA variants, whose scalar registers are already short.)
template <bool LORA>
E4B_DEV void preload_args(const DecodeArgs& p) {
  if constexpr (LORA) return;
  asm volatile("; decode args %0 %1 %2 %3 %4 %5" ::"s"(p.x), "s"(p.topk), "s"(p.topk_w), "s"(p.out), "s"(p.n_out),
               "s"(p.w.packed));
  asm volatile("; decode weights %0 %1 %2 %3 %4 %5" ::"s"(p.w.absmax), "s"(p.w.absmax2), "s"(p.w.offset),
               "s"(p.w.code), "s"(p.w.code2), "s"(p.w.bias));
  asm volatile("; decode sizes %0 %1 %2 %3 %4 %5 %6 %7" ::"s"(p.tokens), "s"(p.k), "s"(p.E), "s"(p.w.n), "s"(p.w.k),
               "s"(p.epi), "s"(p.odt), "s"(p.wdt));
}

// LoRA inside the decode GEMVs: lane gl of a G-lane column group takes ranks q = gl + G * i
// (i < lora_slots<G, LR>()), so its partial delta rides the group's existing reduction. B entries
// are loaded as raw bits with the weights and converted when used. Every slot is loaded (a slot
// past the rank re-reads rank 0 and is zeroed by a select) and the adapter dtype is applied by
// selects: branches here, even uniform ones, measured ~100 more VGPRs in the up kernel and
// spills in the items kernel.
constexpr int kDecLoraMaxRank = 64;

// Rank slots per lane for LoRA variants built for ranks up to LR (LR = 0: no LoRA, one unused slot).
template <int G, int LR>
constexpr int lora_slots() {
  return LR > 0 ? (LR + G - 1) / G : 1;
}

// Raw bits of B[e, row, gl + G * i] for the lane's slots (0 past the rank).
template <int G, int LR>
E4B_DEV void load_lora_b(const DecodeArgs& p, int e, int64_t row, int gl, uint32_t (&b)[lora_slots<G, LR>()]) {
  const int64_t base = (int64_t(e) * p.w.n + row) * p.lr;
  // two 16-bit loads per entry (the second re-reads the first for 16-bit adapters), no branch
  const char* bp = static_cast<const char*>(p.lb);
  const int es = p.lbdt == E4B_FP32 ? 4 : 2;
#pragma unroll
  for (int i = 0; i < lora_slots<G, LR>(); ++i) {
    const int q = gl + G * i;
    const int64_t o = (base + (q < p.lr ? q : 0)) * es;
    const uint32_t lo = *reinterpret_cast<const uint16_t*>(bp + o);
    const uint32_t hi = *reinterpret_cast<const uint16_t*>(bp + o + es - 2);
    b[i] = q < p.lr ? (es == 4 ? lo | (hi << 16) : lo) : 0u;
  }
}

// t[f, gl + G * i] for the lane's slots (0 past the rank).
template <int G, int LR>
E4B_DEV void load_lora_t(const DecodeArgs& p, int f, int gl, float (&t)[lora_slots<G, LR>()]) {
#pragma unroll
  for (int i = 0; i < lora_slots<G, LR>(); ++i) {
    const int q = gl + G * i;
    const float v = p.lt[int64_t(f) * p.lr + (q < p.lr ? q : 0)];
    t[i] = q < p.lr ? v : 0.0f;
  }
}

E4B_DEV float lora_b_value(uint32_t bits, int bdt) {
  const uint16_t h = static_cast<uint16_t>(bits);
  const float f16 = to_f<E4B_FP16>(h), bf16 = to_f<E4B_BF16>(h), f32 = __uint_as_float(bits);
  return bdt == E4B_FP32 ? f32 : (bdt == E4B_BF16 ? bf16 : f16);
}

// The lane's share of lscale * t . B[e, row, :] (summed over the group by its reduction).
template <int G, int LR>
E4B_DEV float lora_partial(const DecodeArgs& p, const float (&t)[lora_slots<G, LR>()],
                           const uint32_t (&b)[lora_slots<G, LR>()]) {
  float d = 0.0f;
#pragma unroll
  for (int i = 0; i < lora_slots<G, LR>(); ++i)
    d = __builtin_fmaf(t[i], lora_b_value(b[i], p.lbdt), d);
  return p.lscale * d;
}

// The first round trip of both kernels loads raw values without branching on them (lanes
// beyond M read row 0) and decodes them only after every load of the round trip is issued: a
// value used inside the branch that loads it is waited for on its own, one round trip each.

// Raw router-weight bits of flat row `lane`; row_weight converts them to fp32.
E4B_DEV uint32_t load_row_weight_bits(const DecodeArgs& p, int M) {
  const int lane = threadIdx.x & (kWave - 1);
  const int f = lane < M ? lane : 0;
  if (p.wdt == E4B_FP32) return static_cast<const uint32_t*>(p.topk_w)[f];
  return static_cast<const uint16_t*>(p.topk_w)[f];
}

E4B_DEV float row_weight(const DecodeArgs& p, uint32_t bits) {
  if (p.wdt == E4B_FP32) return __uint_as_float(bits);
  const uint16_t b = static_cast<uint16_t>(bits);
  return p.wdt == E4B_BF16 ? to_f<E4B_BF16>(b) : to_f<E4B_FP16>(b);
}

// Per-wave routing state in LDS: the bitmap of routed experts, their ascending list and, for
// each listed expert, the mask of flat rows routed to it.
struct WaveRoute {
  unsigned long long bm[kDecExpWords];
  int act[kDecMaxRows];
  unsigned long long rows[kDecMaxRows];
};

// Raw id of flat row `lane`; row_id validates it.
E4B_DEV int64_t load_row_id_raw(const DecodeArgs& p, int M) {
  const int lane = threadIdx.x & (kWave - 1);
  return p.topk[lane < M ? lane : 0];
}

// The id of flat row `lane` (-1: beyond M or outside [0, E)).
E4B_DEV int row_id(const DecodeArgs& p, int M, int64_t v) {
  const int lane = threadIdx.x & (kWave - 1);
  return (lane < M && v >= 0 && v < p.E) ? static_cast<int>(v) : -1;
}

// Wave-local routing: fills r (this wave's copy) and returns the number of routed experts.
// Lane f holds flat row f's expert id; its position in the ascending list is the number of
// routed experts below it, and it ORs its own bit into that expert's row mask.
E4B_DEV int wave_route(int id, WaveRoute& r) {
  const int lane = threadIdx.x & (kWave - 1);
  if (lane < kDecExpWords) r.bm[lane] = 0ull;
  r.rows[lane] = 0ull;
  __builtin_amdgcn_wave_barrier();
  if (id >= 0) atomicOr(&r.bm[id >> 6], 1ull << (id & 63));
  __builtin_amdgcn_wave_barrier();
  const unsigned long long below = (lane == 0) ? 0ull : ((~0ull) >> (kWave - lane));
  const int idw = id >> 6;
  const unsigned long long id_below = (1ull << (id & 63)) - 1ull;
  int n = 0, pos = 0;
#pragma unroll
  for (int w = 0; w < kDecExpWords; ++w) {
    const unsigned long long m = r.bm[w];
    if ((m >> lane) & 1ull) r.act[n + __popcll(m & below)] = w * 64 + lane;
    if (idw == w) pos = n + __popcll(m & id_below);
    n += __popcll(m);
  }
  if (id >= 0) atomicOr(&r.rows[pos], 1ull << lane);
  __builtin_amdgcn_wave_barrier();
  return n;
}

// Table entry for byte b: the (first, second) element codes as 16-bit pairs in dtype DT, hi
// parts in x and lo parts in y (y is zero, and unused, for single entries).
template <int DT, bool SPLIT>
E4B_DEV uint2 pair_entry(float first, float second) {
  const uint16_t h1 = from_f<DT>(first), h2 = from_f<DT>(second);
  if constexpr (!SPLIT) return make_uint2(pack2(h1, h2), 0u);
  const uint16_t l1 = from_f<DT>(first - to_f<DT>(h1)), l2 = from_f<DT>(second - to_f<DT>(h2));
  return make_uint2(pack2(h1, h2), pack2(l1, l2));
}

// The two codes byte threadIdx.x encodes, read straight from the code table (first element:
// high nibble for NF4, low nibble for e2m1).
template <int FMT>
E4B_DEV void load_pair_codes(const e4b_qweight& w, float& first, float& second) {
  const uint32_t b = threadIdx.x & 0xffu;
  if constexpr (FMT == E4B_FMT_MXFP4) {
    first = kFp4E2M1[b & 0xfu];
    second = kFp4E2M1[b >> 4];
  } else {
    first = w.code[b >> 4];
    second = w.code[b & 0xfu];
  }
}

// Thread t fills row t (byte t's entry in every copy) with 16-byte stores, rotating the stores
// with t so the lanes of a wave spread them over the banks. Needs 256 threads.
template <bool SPLIT>
E4B_DEV void store_pair_entry(uint4* lut, uint2 e) {
  const uint32_t b = threadIdx.x;
  const uint4 v = SPLIT ? make_uint4(e.x, e.y, e.x, e.y) : make_uint4(e.x, e.x, e.x, e.x);
  constexpr uint32_t kStores = LutGeom<SPLIT>::kFillBytes / 16;
  uint4* row = lut + b * (kLutRowBytes / 16);
#pragma unroll
  for (uint32_t c = 0; c < kStores; ++c) row[(c + b) & (kStores - 1)] = v;
}

// Raw per-chunk scale data (loaded before the table is built), resolved after the barrier.
struct RawScale {
  float a;      // NF4: absmax; NF4_DQ: absmax2; MXFP4: unused
  uint32_t q;   // NF4_DQ: u8 code; MXFP4: e8m0
};

// Scale of chunk c of weight row `row` of expert e.
template <int FMT>
E4B_DEV RawScale load_scale(const e4b_qweight& w, int e, int64_t row, int c) {
  RawScale s{0.0f, 0u};
  if constexpr (FMT == E4B_FMT_MXFP4) {
    s.q = static_cast<const uint8_t*>(w.absmax)[(int64_t(e) * w.n + row) * (w.k / 32) + c];
  } else if constexpr (FMT == E4B_FMT_NF4) {
    s.a = static_cast<const float*>(w.absmax)[(int64_t(e) * w.n + row) * (w.k / 64) + c / 2];
  } else {
    const int64_t nb = w.n * (w.k / 64);
    const int64_t blk = row * (w.k / 64) + c / 2;
    s.q = static_cast<const uint8_t*>(w.absmax)[e * nb + blk];
    s.a = w.absmax2[e * ((nb + 255) / 256) + blk / 256];
  }
  return s;
}

// Double quant, per weight row: the absmax2 entries of the row's first and last blocks. A row
// holds at most kDecMaxK / 64 = 64 blocks and an absmax2 entry covers 256, so these are the
// only two the row uses; its chunks pick theirs with pick_absmax2 instead of one load each.
struct RowAbsmax2 {
  float a0, a1;
  int64_t g0;  // absmax2 group of the row's first block
};

template <int FMT>
E4B_DEV RowAbsmax2 load_row_absmax2(const e4b_qweight& w, int e, int64_t row) {
  if constexpr (FMT != E4B_FMT_NF4_DQ) {
    return RowAbsmax2{0.0f, 0.0f, 0};
  } else {
    const int64_t bpr = w.k / 64, nb = w.n * bpr, base = int64_t(e) * ((nb + 255) / 256);
    const int64_t g0 = (row * bpr) >> 8, g1 = (row * bpr + bpr - 1) >> 8;
    return RowAbsmax2{w.absmax2[base + g0], w.absmax2[base + g1], g0};
  }
}

// Scale data of chunk c of weight row `row` without the absmax2 entry (taken from the row's
// RowAbsmax2 after the loads have landed).
template <int FMT>
E4B_DEV RawScale load_scale_block(const e4b_qweight& w, int e, int64_t row, int c) {
  if constexpr (FMT != E4B_FMT_NF4_DQ) {
    return load_scale<FMT>(w, e, row, c);
  } else {
    RawScale s{0.0f, 0u};
    s.q = static_cast<const uint8_t*>(w.absmax)[int64_t(e) * w.n * (w.k / 64) + row * (w.k / 64) + c / 2];
    return s;
  }
}

template <int FMT>
E4B_DEV RawScale pick_absmax2(RawScale s, const RowAbsmax2& ra2, const e4b_qweight& w, int64_t row, int c) {
  if constexpr (FMT == E4B_FMT_NF4_DQ) s.a = ((row * (w.k / 64) + c / 2) >> 8) == ra2.g0 ? ra2.a0 : ra2.a1;
  return s;
}

template <int FMT>
E4B_DEV float resolve_scale(const RawScale& s, const float* code2_s, float offset) {
  if constexpr (FMT == E4B_FMT_MXFP4) return e8m0_to_f32(s.q);
  else if constexpr (FMT == E4B_FMT_NF4) return s.a;
  else return __fadd_rn(mul_f32(code2_s[s.q], s.a), offset);
}

// sum over one 16-byte chunk (32 values) of code * x, unscaled, fp32; table entries and x pairs
// in dtype DT.
template <int DT, bool SPLIT>
E4B_DEV float chunk_dot(const uint4& q, const uint4 (&xq)[4], const char* lut_bytes, uint32_t lane_off) {
  const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
  float acc = 0.0f;
#pragma unroll
  for (int wi = 0; wi < 4; ++wi) {
    const uint32_t xs[4] = {xq[wi].x, xq[wi].y, xq[wi].z, xq[wi].w};
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      // address = (byte b of the word) << 8 | lane_off
      const uint32_t addr = __builtin_amdgcn_perm(lane_off, qw[wi], 0x0c0c0004u | (static_cast<uint32_t>(b) << 8));
      if constexpr (SPLIT) {
        const uint2 e = *reinterpret_cast<const uint2*>(lut_bytes + addr);
        acc = dot2<DT>(e.x, xs[b], acc);
        acc = dot2<DT>(e.y, xs[b], acc);
      } else {
        acc = dot2<DT>(*reinterpret_cast<const uint32_t*>(lut_bytes + addr), xs[b], acc);
      }
    }
  }
  return acc;
}

// e2m1 byte SEL of w -> its two codes as a DT pair, the first element (low nibble) in the low
// half: one v_cvt_scalef32_pk_{bf16,f16}_fp4 with scale 1, exact (every e2m1 value is exact in
// either type), so it equals the table entry of that byte.
template <int DT, int SEL>
E4B_DEV uint32_t fp4_pair(uint32_t w) {
  if constexpr (DT == E4B_BF16) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, SEL));
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, SEL));
  }
}

// chunk_dot for e2m1 weights, codes converted in registers: the same v_dot2 sequence on the
// same operands as the table path, without the table reads.
template <int DT>
E4B_DEV float chunk_dot_fp4(const uint4& q, const uint4 (&xq)[4]) {
  const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
  float acc = 0.0f;
#pragma unroll
  for (int wi = 0; wi < 4; ++wi) {
    acc = dot2<DT>(fp4_pair<DT, 0>(qw[wi]), xq[wi].x, acc);
    acc = dot2<DT>(fp4_pair<DT, 1>(qw[wi]), xq[wi].y, acc);
    acc = dot2<DT>(fp4_pair<DT, 2>(qw[wi]), xq[wi].z, acc);
    acc = dot2<DT>(fp4_pair<DT, 3>(qw[wi]), xq[wi].w, acc);
  }
  return acc;
}

// One 32-value chunk of a weight row against activations: e2m1 converted in registers, NF4
// looked up in the LDS table (the decode kernels build no table for e2m1).
template <int DT, int FMT, bool SPLIT>
E4B_DEV float weight_dot(const uint4& q, const uint4 (&xq)[4], const char* lut_bytes, uint32_t lane_off) {
  if constexpr (FMT == E4B_FMT_MXFP4) return chunk_dot_fp4<DT>(q, xq);
  else return chunk_dot<DT, SPLIT>(q, xq, lut_bytes, lane_off);
}

// The 16 single-table entries of one chunk's bytes (byte b of word wi -> t[4 * wi + b]).
E4B_DEV void lut_lookup(const uint4& q, const char* lut_bytes, uint32_t lane_off, uint32_t (&t)[16]) {
  const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int wi = 0; wi < 4; ++wi)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t addr = __builtin_amdgcn_perm(lane_off, qw[wi], 0x0c0c0004u | (static_cast<uint32_t>(b) << 8));
      t[4 * wi + b] = *reinterpret_cast<const uint32_t*>(lut_bytes + addr);
    }
}

// chunk_dot over entries already read: the same v_dot2 sequence on the same operands.
template <int DT>
E4B_DEV float lut_dot(const uint32_t (&t)[16], const uint4 (&xq)[4]) {
  float acc = 0.0f;
#pragma unroll
  for (int wi = 0; wi < 4; ++wi) {
    acc = dot2<DT>(t[4 * wi + 0], xq[wi].x, acc);
    acc = dot2<DT>(t[4 * wi + 1], xq[wi].y, acc);
    acc = dot2<DT>(t[4 * wi + 2], xq[wi].z, acc);
    acc = dot2<DT>(t[4 * wi + 3], xq[wi].w, acc);
  }
  return acc;
}

// The split-table counterparts: (hi, lo) entries of one chunk's bytes, and their dot products
// in chunk_dot<DT, true>'s order.
E4B_DEV void lut_lookup_split(const uint4& q, const char* lut_bytes, uint32_t lane_off, uint2 (&t)[16]) {
  const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int wi = 0; wi < 4; ++wi)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t addr = __builtin_amdgcn_perm(lane_off, qw[wi], 0x0c0c0004u | (static_cast<uint32_t>(b) << 8));
      t[4 * wi + b] = *reinterpret_cast<const uint2*>(lut_bytes + addr);
    }
}

template <int DT>
E4B_DEV float lut_dot_split(const uint2 (&t)[16], const uint4 (&xq)[4]) {
  float acc = 0.0f;
#pragma unroll
  for (int wi = 0; wi < 4; ++wi) {
    const uint32_t xs[4] = {xq[wi].x, xq[wi].y, xq[wi].z, xq[wi].w};
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      acc = dot2<DT>(t[4 * wi + b].x, xs[b], acc);
      acc = dot2<DT>(t[4 * wi + b].y, xs[b], acc);
    }
  }
  return acc;
}

// A lane's CPL chunks of one weight row (qa), and of its gate partner (qb) when PAIR, against
// the activation chunks xread(i, xv) fills (returning the chunk's restaging shift):
// fin_a(i, dot, shift) / fin_b(i, dot, shift) take each chunk's unscaled dot product in chunk
// order. With AHEAD, single-table NF4 reads chunk i + 1's entries before the dot products of
// chunk i, so the table round trip of one chunk overlaps the arithmetic of the previous
// (OLMoE bs=1 gate_up: 8.03 -> 7.45 us per launch; it holds 32 more registers); e2m1 converts
// in registers.
// pre(i) runs at the top of chunk i's step (the up kernel issues later chunks' loads there).
template <int DT, int FMT, int CPL, bool PAIR, bool AHEAD, class XR, class FA, class FB, class PRE>
E4B_DEV void pair_chunk_dots(const uint4 (&qa)[CPL], const uint4 (&qb)[CPL], const char* lut_bytes,
                             uint32_t lane_off, XR&& xread, FA&& fin_a, FB&& fin_b, PRE&& pre) {
  if constexpr (FMT == E4B_FMT_MXFP4 || !AHEAD) {
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      pre(i);
      uint4 xv[4];
      const int sh = xread(i, xv);
      fin_a(i, weight_dot<DT, FMT, false>(qa[i], xv, lut_bytes, lane_off), sh);
      __builtin_amdgcn_sched_barrier(0);  // keep each chunk's table reads together
      if constexpr (PAIR) {
        fin_b(i, weight_dot<DT, FMT, false>(qb[i], xv, lut_bytes, lane_off), sh);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  } else {
    uint32_t ta[16], tb[16];
    lut_lookup(qa[0], lut_bytes, lane_off, ta);
    if constexpr (PAIR) lut_lookup(qb[0], lut_bytes, lane_off, tb);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      constexpr int kLast = CPL - 1;
      pre(i);
      uint4 xv[4];
      const int sh = xread(i, xv);
      const float da = lut_dot<DT>(ta, xv);
      if (i < kLast) lut_lookup(qa[i < kLast ? i + 1 : i], lut_bytes, lane_off, ta);
      __builtin_amdgcn_sched_barrier(0);
      fin_a(i, da, sh);
      if constexpr (PAIR) {
        const float db = lut_dot<DT>(tb, xv);
        if (i < kLast) lut_lookup(qb[i < kLast ? i + 1 : i], lut_bytes, lane_off, tb);
        __builtin_amdgcn_sched_barrier(0);
        fin_b(i, db, sh);
      }
    }
  }
}

// bf16 -> scaled fp16 restaging of activations (up kernel, NF4 weights): bf16_exp_max gives a
// 16-byte piece's largest exponent field.
// Maximum over the aligned quad of lanes (the four pieces of one 32-value chunk).
E4B_DEV uint32_t quad_max(uint32_t v) {
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0xb1, 0xf, 0xf, false)));
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x4e, 0xf, 0xf, false)));
  return v;
}

// Shift that puts a chunk whose largest biased exponent is e into [2^14, 2^15).
E4B_DEV int chunk_shift(uint32_t exp_bits) { return exp_shift(static_cast<int>(exp_bits >> 7)); }

E4B_DEV uint4 piece_to_f16(const uint4& v, int d) {
  return make_uint4(bf16x2_to_f16x2(v.x, d), bf16x2_to_f16x2(v.y, d), bf16x2_to_f16x2(v.z, d),
                    bf16x2_to_f16x2(v.w, d));
}

// v + the value of the lane selected by a DPP pattern within each 16-lane row.
template <int CTRL>
E4B_DEV float dpp_add(float v) {
  const int o = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false);
  return v + __int_as_float(o);
}

// Sum over aligned groups of G lanes (G a power of two, 2..64); every lane gets its group's sum.
// Within a 16-lane row the steps are DPP moves (xor 1 and xor 2 by quad_perm, then the
// half-row and row mirrors, which pair each lane with one holding the complementary partial
// sum); wider groups finish with cross-row swaps.
template <int G>
E4B_DEV float group_reduce(float v) {
  v = dpp_add<0xb1>(v);                          // quad_perm [1,0,3,2]
  if constexpr (G >= 4) v = dpp_add<0x4e>(v);    // quad_perm [2,3,0,1]
  if constexpr (G >= 8) v = dpp_add<0x141>(v);   // row_half_mirror
  if constexpr (G >= 16) v = dpp_add<0x140>(v);  // row_mirror
  if constexpr (G >= 32) v += __shfl_xor(v, 16);
  if constexpr (G >= 64) v += __shfl_xor(v, 32);
  return v;
}

// The i-th chunk slot of lane gl: its chunk index, and whether it is a real chunk.
template <int G, bool FULL>
E4B_DEV int slot_chunk(int gl, int i, int nchunk, bool& valid) {
  const int c = gl + i * G;
  valid = FULL || c < nchunk;
  return valid ? c : 0;
}

E4B_DEV void load_chunk_x(const uint16_t* xr, int c, uint4 (&xv)[4]) {
  const uint4* xp = reinterpret_cast<const uint4*>(xr + 32 * c);
#pragma unroll
  for (int q = 0; q < 4; ++q) xv[q] = xp[q];
}

E4B_DEV uint4 load_chunk_w(const e4b_qweight& w, int e, int64_t row, int c) {
  return *reinterpret_cast<const uint4*>(w.packed + (int64_t(e) * w.n + row) * (w.k / 2) + 16 * c);
}

// gate_up GEMV + fused epilogue for the a-th routed expert (blockIdx.y), G lanes per column.
template <int DT, int FMT, int G, int CPL, bool FULL, bool PAIR, int LR>
__global__ void __launch_bounds__(kDecThreads) decode_up_kernel(DecodeArgs p) {
  constexpr bool LORA = LR > 0;
  // NF4 codes as fp16 single entries; e2m1 codes in the activation dtype
  constexpr int CDT = FMT == E4B_FMT_MXFP4 ? DT : E4B_FP16;
  constexpr bool kConv = CDT != DT;  // bf16 activations restaged as scaled fp16
  __shared__ __align__(16) uint4 lut[FMT == E4B_FMT_MXFP4 ? 1 : 256 * kLutRowBytes / 16];  // none for e2m1
  __shared__ __align__(16) uint4 xs[kDecMaxK / 8 + 1];  // the activation row being multiplied + a spare slot
  __shared__ int xsh[kConv ? kDecMaxK / 32 + 1 : 1];     // per chunk: the inverse of its restaging shift
  __shared__ WaveRoute route[kDecWaves];
  __shared__ float code2_s[(FMT == E4B_FMT_NF4_DQ) ? 256 : 1];
  preload_args<LORA>(p);
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  const int M = p.tokens * p.k;
  const e4b_qweight& w = p.w;

  // round trip 1: ids, the code pair of this thread's table entry, code2
  const int64_t id_raw = load_row_id_raw(p, M);
  float cf, cs;
  load_pair_codes<FMT>(w, cf, cs);
  const float c2 = (FMT == E4B_FMT_NF4_DQ) ? w.code2[threadIdx.x] : 0.0f;

  WaveRoute& r = route[wid];
  const int nact = wave_route(row_id(p, M, id_raw), r);
  const int a = blockIdx.y;
  if (a >= nact) return;  // uniform over the block: every wave computed the same routing
  const int e = r.act[a];
  unsigned long long rows = r.rows[a];

  const int gl = lane % G;
  const int nchunk = static_cast<int>(w.k / 32);
  constexpr bool pair = PAIR;  // gated epilogue: gate row j and up row j + n/2
  const int64_t n = w.n, k = w.k;
  const int64_t j = (int64_t(blockIdx.x) * kDecWaves + wid) * (kWave / G) + lane / G;
  const bool live = j < p.n_out;  // whole G-lane groups share it
  const int64_t row_a = live ? j : 0, row_b = pair ? row_a + n / 2 : row_a;
  int f = __ffsll(static_cast<long long>(rows)) - 1;
  const int nx4 = nchunk * 4;  // 16-byte pieces of an activation row
  // The activation row of the expert's current routed row goes through LDS: thread t loads
  // 16-byte pieces t and t + 256 (clamped, no branch) and stores the real ones. Loaded before
  // the weights, so waiting for them leaves the weight loads in flight. (Two named registers,
  // not an array: an array indexed in an unrolled loop can end up in scratch memory.)
  static_assert(kDecMaxK / 8 == 2 * kDecThreads, "two 16-byte pieces per thread");
  const int t0 = static_cast<int>(threadIdx.x), t1 = t0 + kDecThreads;
  uint4 xp0, xp1;
  auto load_x = [&](int row) {
    const uint4* x4 = reinterpret_cast<const uint4*>(p.x + int64_t(row / p.k) * k);
    xp0 = x4[t0 < nx4 ? t0 : 0];
    xp1 = x4[t1 < nx4 ? t1 : 0];
  };
  auto store_x = [&]() {  // pieces beyond the row go to the spare slot: no branch to sink the loads into
    const int i0 = t0 < nx4 ? t0 : kDecMaxK / 8, i1 = t1 < nx4 ? t1 : kDecMaxK / 8;
    if constexpr (kConv) {
      // the four lanes of a quad hold the four pieces of a chunk (thread t: pieces t, t + 256)
      const int d0 = chunk_shift(quad_max(bf16_exp_max(xp0)));
      const int d1 = chunk_shift(quad_max(bf16_exp_max(xp1)));
      xs[i0] = piece_to_f16(xp0, d0);
      xs[i1] = piece_to_f16(xp1, d1);
      xsh[i0 / 4] = -d0;
      xsh[i1 / 4] = -d1;
    } else {
      xs[i0] = xp0;
      xs[i1] = xp1;
    }
  };

  // the decode table first: its stores then overlap the ids' wait, not the weight issue
  if constexpr (FMT != E4B_FMT_MXFP4) store_pair_entry<false>(lut, pair_entry<CDT, false>(cf, cs));

  // round trip 2: the activation row, then the weights and scales of the first kIssue chunks,
  // biases; the remaining chunks are issued at the top of the chunk loop's steps, so a wave
  // does not sit in the load issue while the data of its first chunks is already there
  load_x(f);
  uint4 qa[CPL], qb[CPL];
  RawScale ra[CPL], rb[CPL];
  bool valid[CPL];
  int cidx[CPL];
  auto issue_chunk = [&](int i) {
    const int c = slot_chunk<G, FULL>(gl, i, nchunk, valid[i]);
    cidx[i] = c;
    qa[i] = load_chunk_w(w, e, row_a, c);
    if constexpr (pair) qb[i] = load_chunk_w(w, e, row_b, c);
    ra[i] = load_scale_block<FMT>(w, e, row_a, c);
    if constexpr (pair) rb[i] = load_scale_block<FMT>(w, e, row_b, c);
  };
  // chunk i + 1's table entries are read in step i: it must be issued by then
  constexpr int kIssue = up_issue_chunks<FMT, CPL>();
  static_assert(kIssue >= 2 || kIssue == CPL, "chunk 1 is issued before the loop");
#pragma unroll
  for (int i = 0; i < kIssue; ++i) issue_chunk(i);
  const RowAbsmax2 r2a = load_row_absmax2<FMT>(w, e, row_a);
  const RowAbsmax2 r2b = pair ? load_row_absmax2<FMT>(w, e, row_b) : r2a;
  // biases as raw bits, loaded without a branch (a spare load of x[0] when there is none) and
  // converted after the loop, so nothing here waits on the loads in flight
  const bool has_bias = w.bias != nullptr;
  const uint16_t* bias = has_bias ? static_cast<const uint16_t*>(w.bias) + int64_t(e) * n : p.x;
  const uint32_t bg_bits = bias[has_bias ? row_a : 0];
  const uint32_t bu_bits = bias[has_bias ? row_b : 0];
  const float off = (FMT == E4B_FMT_NF4_DQ) ? w.offset[e] : 0.0f;
  // LoRA: the column's B entries (once per block) and the row's t entries, after the weights
  uint32_t lba[lora_slots<G, LR>()], lbb[lora_slots<G, LR>()];
  float ltv[lora_slots<G, LR>()];
  if constexpr (LORA) {
    load_lora_b<G, LR>(p, e, row_a, gl, lba);
    if constexpr (pair) load_lora_b<G, LR>(p, e, row_b, gl, lbb);
    load_lora_t<G, LR>(p, f, gl, ltv);
  }

  // the activation row while the weights are in flight; the chunk loop then waits for each
  // chunk's weights only
  if constexpr (FMT == E4B_FMT_NF4_DQ) code2_s[threadIdx.x] = c2;
  store_x();
  __syncthreads();

  uint32_t lane_off = LutGeom<false>::lane_off(lane);
  const char* lut_bytes = reinterpret_cast<const char*>(lut);
  // chunk scales, resolved at their first use (the first row's pass)
  float sa[CPL], sb[CPL];
  // One routed row: the first row's pass (FIRST) issues the deferred chunks and resolves the
  // scales; later rows of the same expert reuse both.
  auto row_pass = [&](auto first_tag) {
    constexpr bool kFirst = decltype(first_tag)::value;
    // the table addresses depend only on the weights, which do not change from row to row;
    // recomputing them per row keeps 128 addresses from being hoisted and held in registers
    asm volatile("" : "+v"(lane_off));
    float acc_a = 0.0f, acc_b = 0.0f;
    pair_chunk_dots<CDT, FMT, CPL, pair, true>(
        qa, qb, lut_bytes, lane_off,
        [&](int i, uint4 (&xv)[4]) {
#pragma unroll
          for (int q = 0; q < 4; ++q) xv[q] = xs[cidx[i] * 4 + q];
          return kConv ? xsh[cidx[i]] : 0;
        },
        [&](int i, float d, int sh) {
          if constexpr (kFirst)
            sa[i] = valid[i] ? resolve_scale<FMT>(pick_absmax2<FMT>(ra[i], r2a, w, row_a, cidx[i]), code2_s, off)
                             : 0.0f;
          if constexpr (kConv) d = __builtin_amdgcn_ldexpf(d, sh);
          acc_a += valid[i] ? d * sa[i] : 0.0f;
        },
        [&](int i, float d, int sh) {
          if constexpr (kFirst)
            sb[i] = (pair && valid[i])
                        ? resolve_scale<FMT>(pick_absmax2<FMT>(rb[i], r2b, w, row_b, cidx[i]), code2_s, off)
                        : 0.0f;
          if constexpr (kConv) d = __builtin_amdgcn_ldexpf(d, sh);
          acc_b += valid[i] ? d * sb[i] : 0.0f;
        },
        [&](int i) {
          if constexpr (kFirst) {
            if (i + kIssue < CPL) issue_chunk(i + kIssue < CPL ? i + kIssue : CPL - 1);
          }
        });
    if constexpr (LORA) {
      acc_a += lora_partial<G, LR>(p, ltv, lba);
      if constexpr (pair) acc_b += lora_partial<G, LR>(p, ltv, lbb);
    }
    acc_a = group_reduce<G>(acc_a);
    if constexpr (pair) acc_b = group_reduce<G>(acc_b);
    if (live && gl == 0) {
      // the empty asm pins the bias conversion here: hoisted above the table barrier it would
      // wait for every load in flight
      uint32_t gb = bg_bits, ub = bu_bits;
      asm volatile("" : "+v"(gb), "+v"(ub));
      const float bg = has_bias ? to_f<DT>(static_cast<uint16_t>(gb)) : 0.0f;
      const float bu = has_bias ? to_f<DT>(static_cast<uint16_t>(ub)) : 0.0f;
      const float v = pair ? gated(p.epi, acc_a, acc_b, p.alpha, p.limit, bg, bu) : single(p.epi, acc_a, bg);
      static_cast<uint16_t*>(p.out)[int64_t(f) * p.n_out + j] = from_f<DT>(v);
    }
  };
  // next routed row of this expert (the same for the whole block): restage its activations
  auto next_row = [&]() {
    f = __ffsll(static_cast<long long>(rows)) - 1;
    load_x(f);
    if constexpr (LORA) load_lora_t<G, LR>(p, f, gl, ltv);
    __syncthreads();  // every wave is done with the current row
    store_x();
    __syncthreads();
  };
  if constexpr (FMT != E4B_FMT_MXFP4) {
    row_pass(std::true_type{});
    for (rows &= rows - 1; rows; rows &= rows - 1) {
      next_row();
      row_pass(std::false_type{});
    }
  } else {
    // e2m1 defers nothing: scales resolved up front and one loop body (a peeled first row
    // measured 217 -> 255 VGPRs at six chunks per lane)
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      sa[i] = valid[i] ? resolve_scale<FMT>(ra[i], code2_s, off) : 0.0f;
      sb[i] = (pair && valid[i]) ? resolve_scale<FMT>(rb[i], code2_s, off) : 0.0f;
    }
    for (;;) {
      row_pass(std::false_type{});
      rows &= rows - 1;
      if (!rows) break;
      next_row();
    }
  }
}

// gate_up for 2..8 tokens. Every token's activations fit in LDS at once, so the layer's work is
// split into items -- one routed expert x kWave / G output columns -- that each wave takes in
// turn with no barrier after the setup: one block per CU builds the decode table, routes, and
// stages all activation rows once, then each wave streams its items' weights, loading the next
// item while it computes the current one. (decode_up_kernel runs one block per (column tile,
// routed expert) and restages the activations per routed row behind two barriers: at 8 tokens
// on 64 experts that is ~2600 blocks, each paying the id round trip and the table build.)
constexpr int kItemThreads = 512;
constexpr int kItemWaves = kItemThreads / kWave;
constexpr int kItemMaxX = 16384;  // tokens * k1 activation elements staged (32 KB)

template <int DT, int FMT, int G, int CPL, bool FULL, bool PAIR, int LR>
__global__ void __launch_bounds__(kItemThreads) decode_up_items_kernel(DecodeArgs p) {
  constexpr bool LORA = LR > 0;
  preload_args<LORA>(p);
  constexpr int CDT = FMT == E4B_FMT_MXFP4 ? DT : E4B_FP16;
  constexpr bool kConv = CDT != DT;
  constexpr int kXU = kItemMaxX / 8 / kItemThreads;  // 16-byte activation pieces per thread
  __shared__ __align__(16) uint4 lut[FMT == E4B_FMT_MXFP4 ? 1 : 256 * kLutRowBytes / 16];  // none for e2m1
  __shared__ __align__(16) uint4 xs[kItemMaxX / 8 + 1];  // every token's activations + a spare slot
  __shared__ int xsh[kConv ? kItemMaxX / 32 + 1 : 1];     // per chunk: the inverse restaging shift
  __shared__ WaveRoute route[kItemWaves];
  __shared__ float code2_s[(FMT == E4B_FMT_NF4_DQ) ? 256 : 1];
  __shared__ float lts[LR > 0 ? kDecMaxRows * LR : 1];  // LoRA: t of every flat row
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & (kWave - 1);
  const int wid = tid / kWave;
  const int M = p.tokens * p.k;
  const e4b_qweight& w = p.w;
  const int64_t n = w.n, k = w.k;
  const int nx = static_cast<int>(p.tokens * k / 8);  // <= kItemMaxX / 8: checked by the launcher

  // round trip 1: ids, every activation piece (clamped, no branch), the code pair, code2
  const int64_t id_raw = load_row_id_raw(p, M);
  // (four named registers, not an array: an array here ends up in LDS or scratch memory)
  static_assert(kXU == 4, "four 16-byte activation pieces per thread");
  const uint4* x4 = reinterpret_cast<const uint4*>(p.x);
  auto piece = [&](int u) { return tid + u * kItemThreads; };
  const uint4 xp0 = x4[piece(0) < nx ? piece(0) : 0], xp1 = x4[piece(1) < nx ? piece(1) : 0];
  const uint4 xp2 = x4[piece(2) < nx ? piece(2) : 0], xp3 = x4[piece(3) < nx ? piece(3) : 0];
  float cf, cs;
  load_pair_codes<FMT>(w, cf, cs);
  const float c2 = (FMT == E4B_FMT_NF4_DQ) ? w.code2[tid & 255] : 0.0f;
  // LoRA: the t entries of every flat row (M * lr <= 64 * LR), staged beside the activations
  constexpr int kTU = LORA ? kDecMaxRows * LR / kItemThreads : 1;
  const int nt = M * p.lr;
  float tv[kTU];
  if constexpr (LORA) {
#pragma unroll
    for (int u = 0; u < kTU; ++u) {
      const int i = tid + u * kItemThreads;
      tv[u] = p.lt[i < nt ? i : 0];
    }
  }

  WaveRoute& r = route[wid];
  const int nact = wave_route(row_id(p, M, id_raw), r);
  if constexpr (LORA) {
#pragma unroll
    for (int u = 0; u < kTU; ++u) {
      const int i = tid + u * kItemThreads;
      if (i < nt) lts[i] = tv[u];
    }
  }
  if (tid < 256) {
    if constexpr (FMT != E4B_FMT_MXFP4) store_pair_entry<false>(lut, pair_entry<CDT, false>(cf, cs));
    if constexpr (FMT == E4B_FMT_NF4_DQ) code2_s[tid] = c2;
  }
  // Piece (token t, chunk c, quarter q) goes to xs[t * xrow + q * nchunk + c]: the G lanes of a
  // group then read 16 consecutive bytes each for the same quarter (conflict-free), where the
  // row-major order puts them 64 bytes apart. The four pieces of a chunk sit in an aligned lane
  // quad (kItemThreads is a multiple of 4, rows are whole chunks); pieces beyond the
  // activations go to the spare slot.
  const int xrow = static_cast<int>(k / 8), nchunk = static_cast<int>(k / 32);
  auto stage = [&](int u, const uint4& v) {
    const int pc = piece(u);
    const int t = pc / xrow, rp = pc - t * xrow;
    const bool real = pc < nx;
    const int idx = real ? t * xrow + (rp & 3) * nchunk + (rp >> 2) : kItemMaxX / 8;
    if constexpr (kConv) {
      const int d = chunk_shift(quad_max(bf16_exp_max(v)));
      xs[idx] = piece_to_f16(v, d);
      xsh[real ? pc / 4 : kItemMaxX / 32] = -d;
    } else {
      xs[idx] = v;
    }
  };
  stage(0, xp0);
  stage(1, xp1);
  stage(2, xp2);
  stage(3, xp3);
  __syncthreads();

  constexpr bool pair = PAIR;  // gated epilogue: gate row j and up row j + n/2
  constexpr int kCols = kWave / G;
  // item it: routed expert it / ncg, column group it % ncg (32-bit: at most 64 x n_out / kCols)
  const int n_out = static_cast<int>(p.n_out);
  const int ncg = (n_out + kCols - 1) / kCols;
  const int nitems = nact * ncg;
  const int stride = static_cast<int>(gridDim.x) * kItemWaves;
  const int gl = lane % G;
  uint32_t lane_off = LutGeom<false>::lane_off(lane);
  const char* lut_bytes = reinterpret_cast<const char*>(lut);
  const bool has_bias = w.bias != nullptr;
  bool valid[CPL];
  int cidx[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) cidx[i] = slot_chunk<G, FULL>(gl, i, nchunk, valid[i]);

  // one item's loads: weights and scales chunk by chunk, then the bias bits and the offset
  struct Buf {
    uint4 qa[CPL], qb[CPL];
    RawScale ra[CPL], rb[CPL];
    uint32_t bg, bu;
    float off;
    uint32_t lba[lora_slots<G, LR>()], lbb[lora_slots<G, LR>()];  // LoRA B entries of the two rows
  };
  auto load = [&](int it, Buf& b) {
    const int a = it / ncg;
    const int e = r.act[a];
    const int j = (it - a * ncg) * kCols + lane / G;
    const int64_t row_a = j < n_out ? j : 0, row_b = pair ? row_a + n / 2 : row_a;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      b.qa[i] = load_chunk_w(w, e, row_a, cidx[i]);
      if constexpr (pair) b.qb[i] = load_chunk_w(w, e, row_b, cidx[i]);
      b.ra[i] = load_scale<FMT>(w, e, row_a, cidx[i]);
      if constexpr (pair) b.rb[i] = load_scale<FMT>(w, e, row_b, cidx[i]);
    }
    const uint16_t* bias = has_bias ? static_cast<const uint16_t*>(w.bias) + int64_t(e) * n : p.x;
    b.bg = bias[has_bias ? row_a : 0];
    b.bu = bias[has_bias ? row_b : 0];
    b.off = (FMT == E4B_FMT_NF4_DQ) ? w.offset[e] : 0.0f;
    if constexpr (LORA) {
      load_lora_b<G, LR>(p, e, row_a, gl, b.lba);
      if constexpr (pair) load_lora_b<G, LR>(p, e, row_b, gl, b.lbb);
    }
  };
  auto compute = [&](int it, const Buf& b) {
    const int a = it / ncg;
    const int j = (it - a * ncg) * kCols + lane / G;
    const bool live = j < n_out;
    unsigned long long rows = r.rows[a];
    float sa[CPL], sb[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      sa[i] = valid[i] ? resolve_scale<FMT>(b.ra[i], code2_s, b.off) : 0.0f;
      sb[i] = (pair && valid[i]) ? resolve_scale<FMT>(b.rb[i], code2_s, b.off) : 0.0f;
    }
    const float bg = has_bias ? to_f<DT>(static_cast<uint16_t>(b.bg)) : 0.0f;
    const float bu = has_bias ? to_f<DT>(static_cast<uint16_t>(b.bu)) : 0.0f;
    while (rows) {
      const int f = __ffsll(static_cast<long long>(rows)) - 1;
      rows &= rows - 1;
      const int tok = f / p.k;
      asm volatile("" : "+v"(lane_off));  // table addresses recomputed per row, not held
      float acc_a = 0.0f, acc_b = 0.0f;
      // (no look-ahead past four chunks per lane, nor beside more than two LoRA rank slots per
      // lane: with two weight buffers it spills)
      pair_chunk_dots<CDT, FMT, CPL, pair, (CPL <= 4 && !(LORA && lora_slots<G, LR>() > 2))>(
          b.qa, b.qb, lut_bytes, lane_off,
          [&](int i, uint4 (&xv)[4]) {
#pragma unroll
            for (int q = 0; q < 4; ++q) xv[q] = xs[tok * xrow + q * nchunk + cidx[i]];
            return kConv ? xsh[tok * nchunk + cidx[i]] : 0;
          },
          [&](int i, float d, int sh) {
            if constexpr (kConv) d = __builtin_amdgcn_ldexpf(d, sh);
            acc_a += valid[i] ? d * sa[i] : 0.0f;
          },
          [&](int i, float d, int sh) {
            if constexpr (kConv) d = __builtin_amdgcn_ldexpf(d, sh);
            acc_b += valid[i] ? d * sb[i] : 0.0f;
          },
          [](int) {});
      if constexpr (LORA) {
        float ltv[lora_slots<G, LR>()];
#pragma unroll
        for (int i = 0; i < lora_slots<G, LR>(); ++i) {
          const int q = gl + G * i;
          const float v = lts[f * p.lr + (q < p.lr ? q : 0)];  // no branch around the read
          ltv[i] = q < p.lr ? v : 0.0f;
        }
        acc_a += lora_partial<G, LR>(p, ltv, b.lba);
        if constexpr (pair) acc_b += lora_partial<G, LR>(p, ltv, b.lbb);
      }
      acc_a = group_reduce<G>(acc_a);
      if constexpr (pair) acc_b = group_reduce<G>(acc_b);
      if (live && gl == 0) {
        const float v = pair ? gated(p.epi, acc_a, acc_b, p.alpha, p.limit, bg, bu) : single(p.epi, acc_a, bg);
        static_cast<uint16_t*>(p.out)[int64_t(f) * n_out + j] = from_f<DT>(v);
      }
    }
  };

  // Two buffers in turn (named, not an indexed pair, so nothing goes to scratch memory). Every
  // load is unconditional -- past the last item a wave reloads the item it is about to compute,
  // which the cache holds -- so the compiler's wait before each compute counts exactly the
  // loads issued after that item's.
  int it = static_cast<int>(blockIdx.x) * kItemWaves + wid;
  if (it >= nitems) return;  // no barrier follows
  Buf b0, b1;
  load(it, b0);
  for (;;) {
    const int i1 = it + stride;
    load(i1 < nitems ? i1 : it, b1);
    compute(it, b0);
    if (i1 >= nitems) break;
    const int i2 = i1 + stride;
    load(i2 < nitems ? i2 : i1, b0);
    compute(i1, b1);
    if (i2 >= nitems) break;
    it = i2;
  }
}

// down GEMV over every routed row for kDownCols output columns, then the k-slot combine.
// Jobs (one routed expert, all kDownCols columns) go to G-lane groups, JOBS per group in flight.
template <int DT, int FMT, int G, int CPL, int JOBS, bool FULL, int LR>
__global__ void __launch_bounds__(kDecThreads) decode_down_kernel(DecodeArgs p) {
  constexpr bool LORA = LR > 0;
  preload_args<LORA>(p);
  __shared__ __align__(16) uint4 lut[FMT == E4B_FMT_MXFP4 ? 1 : 256 * kLutRowBytes / 16];  // none for e2m1
  __shared__ WaveRoute route[kDecWaves];
  __shared__ float res[kDecMaxRows * kDownCols];
  __shared__ float wts[kDecMaxRows];
  __shared__ float code2_s[(FMT == E4B_FMT_NF4_DQ) ? 256 : 1];
  constexpr int C = kDownCols;
  constexpr int kGroups = kDecThreads / G;
  constexpr bool kSplit = FMT != E4B_FMT_MXFP4;  // NF4: (hi, lo) entries in the activation dtype
  // one chunk per lane and column (the split-table path): scales resolved column by column at
  // their first use, so column 0's products wait for column 0's loads only
  constexpr bool kLazy = kSplit && CPL == 1;
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  const int M = p.tokens * p.k;
  const e4b_qweight& w = p.w;

  // round trip 1: ids and router weights (for the combine), code pair, code2
  const int64_t id_raw = load_row_id_raw(p, M);
  const uint32_t wt_bits = load_row_weight_bits(p, M);
  float cf, cs;
  load_pair_codes<FMT>(w, cf, cs);
  const float c2 = (FMT == E4B_FMT_NF4_DQ) ? w.code2[threadIdx.x] : 0.0f;

  WaveRoute& r = route[wid];
  const int id = row_id(p, M, id_raw);
  const int nact = wave_route(id, r);
  const unsigned long long routed_rows = __ballot(id >= 0);  // the same in every wave

  const int gl = lane % G;
  const int group = threadIdx.x / G;
  const int nchunk = static_cast<int>(w.k / 32);
  const int64_t n = w.n, k = w.k;
  const int64_t col0 = int64_t(blockIdx.x) * C;
  const bool has_bias = w.bias != nullptr;
  const uint16_t* bias = static_cast<const uint16_t*>(w.bias);
  uint32_t lane_off = LutGeom<kSplit>::lane_off(lane);
  const char* lut_bytes = reinterpret_cast<const char*>(lut);
  int64_t cols[C];
#pragma unroll
  for (int cl = 0; cl < C; ++cl) cols[cl] = (col0 + cl < n) ? col0 + cl : col0;  // spare columns repeat col0

  bool table_ready = false;
  for (int base = group * JOBS; base < nact || !table_ready; base += kGroups * JOBS) {
    // issue every load of this pass: the first routed row's activation chunks, then each
    // column's weight chunk and scale, chunk by chunk
    uint4 q[JOBS][CPL][C], xv[JOBS][CPL][4];
    RawScale rs[JOBS][CPL][C];
    float joff[JOBS];      // double quant: the expert's absmax offset
    uint16_t bb[JOBS][C];  // raw bias bits, converted when the job runs
    uint32_t lbw[JOBS][C][lora_slots<G, LR>()];  // LoRA: B entries of the job's columns
    float ltv[JOBS][lora_slots<G, LR>()];        // LoRA: t entries of the job's current row
    bool valid[CPL];
    int je[JOBS], jf[JOBS];
    unsigned long long jrows[JOBS];
#pragma unroll
    for (int t = 0; t < JOBS; ++t) {
      const int job = base + t;
      const bool ok = job < nact;
      je[t] = ok ? r.act[job] : -1;
      jrows[t] = ok ? r.rows[job] : 0ull;
      jf[t] = ok ? __ffsll(static_cast<long long>(jrows[t])) - 1 : 0;
      // NF4 (split table): a group without a job loads the first routed expert's chunks (which
      // its group loads anyway), so no branch sits around the loads whose count each wait below
      // depends on; the offset and the bias bits go first (the row pass converts them before its
      // first table lookup, which, loads being counted in issue order, then waits for them and
      // column 0's loads only; issued last, they made it wait for every column's weights and
      // scales). e2m1 keeps the branch and the bias last: the same order measured slower there
      // (gpt-oss bs=1 21.6 -> 22.1 us).
      const int e = ok ? je[t] : ((kSplit && nact > 0) ? r.act[0] : 0);
      // a spare load of x[0] when there is no bias: no branch on the loaded value
      const uint16_t* bp = has_bias ? bias + int64_t(e) * n : p.x;
      if constexpr (kSplit) {
        joff[t] = (FMT == E4B_FMT_NF4_DQ) ? w.offset[e] : 0.0f;
#pragma unroll
        for (int cl = 0; cl < C; ++cl) bb[t][cl] = bp[has_bias ? cols[cl] : 0];
      }
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = slot_chunk<G, FULL>(gl, i, nchunk, valid[i]);
        if (kSplit || ok) {
          load_chunk_x(p.x + int64_t(jf[t]) * k, c, xv[t][i]);
#pragma unroll
          for (int cl = 0; cl < C; ++cl) {
            q[t][i][cl] = load_chunk_w(w, e, cols[cl], c);
            rs[t][i][cl] = load_scale<FMT>(w, e, cols[cl], c);
            // NF4: each column's weights and scale issued together (left to itself the
            // scheduler groups the weight loads ahead of the scale loads, and column 0's scale
            // then arrives behind every column's weights)
            if constexpr (kSplit) __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
      if constexpr (!kSplit) {
        joff[t] = 0.0f;
#pragma unroll
        for (int cl = 0; cl < C; ++cl) bb[t][cl] = bp[has_bias ? cols[cl] : 0];
      }
      if constexpr (LORA) {
        if (ok) {
#pragma unroll
          for (int cl = 0; cl < C; ++cl) load_lora_b<G, LR>(p, e, cols[cl], gl, lbw[t][cl]);
          load_lora_t<G, LR>(p, jf[t], gl, ltv[t]);
        }
      }
    }
    if (!table_ready) {
      if constexpr (FMT != E4B_FMT_MXFP4) store_pair_entry<kSplit>(lut, pair_entry<DT, kSplit>(cf, cs));
      if constexpr (FMT == E4B_FMT_NF4_DQ) code2_s[threadIdx.x] = c2;
      if (wid == 0) wts[lane] = row_weight(p, wt_bits);  // read by the combine
      __syncthreads();
      table_ready = true;
    }
#pragma unroll
    for (int t = 0; t < JOBS; ++t) {
      if (je[t] < 0) continue;  // whole group skips together
      const float off = joff[t];
      float sc[CPL][C], b[C];
      auto resolve = [&](int i, int cl) {
        sc[i][cl] = valid[i] ? resolve_scale<FMT>(rs[t][i][cl], code2_s, off) : 0.0f;
      };
      if constexpr (!kLazy) {
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
#pragma unroll
          for (int cl = 0; cl < C; ++cl) resolve(i, cl);
        }
      }
#pragma unroll
      for (int cl = 0; cl < C; ++cl) b[cl] = has_bias ? to_f<DT>(bb[t][cl]) : 0.0f;
      unsigned long long rows = jrows[t];
      int f = jf[t];
      // One routed row of the job. The first row's pass (FIRST) resolves the scales column by
      // column; later rows reuse them.
      auto row_pass = [&](auto first_tag) {
        constexpr bool kFirst = decltype(first_tag)::value;
        asm volatile("" : "+v"(lane_off));  // no hoisting of the per-row table addresses
        float acc[C];
#pragma unroll
        for (int cl = 0; cl < C; ++cl) acc[cl] = 0.0f;
        if constexpr (kSplit && CPL == 1) {
          // (chunk, column) pairs in order, the next pair's table entries read before the
          // current pair's dot products (CPL == 1: beyond it the extra 32 registers spill)
          uint2 te[16];
          lut_lookup_split(q[t][0][0], lut_bytes, lane_off, te);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int cl = 0; cl < C; ++cl) {
            if constexpr (kFirst && kLazy) resolve(0, cl);
            const float d = lut_dot_split<DT>(te, xv[t][0]) * sc[0][cl];
            if (cl + 1 < C) lut_lookup_split(q[t][0][cl + 1 < C ? cl + 1 : cl], lut_bytes, lane_off, te);
            __builtin_amdgcn_sched_barrier(0);
            acc[cl] += valid[0] ? d : 0.0f;
          }
        } else {
#pragma unroll
          for (int i = 0; i < CPL; ++i) {
#pragma unroll
            for (int cl = 0; cl < C; ++cl) {
              const float d = weight_dot<DT, FMT, kSplit>(q[t][i][cl], xv[t][i], lut_bytes, lane_off) * sc[i][cl];
              acc[cl] += valid[i] ? d : 0.0f;
              __builtin_amdgcn_sched_barrier(0);  // keep each chunk's 16 table reads together
            }
          }
        }
        if constexpr (LORA) {
#pragma unroll
          for (int cl = 0; cl < C; ++cl) acc[cl] += lora_partial<G, LR>(p, ltv[t], lbw[t][cl]);
        }
#pragma unroll
        for (int cl = 0; cl < C; ++cl) {
          const float v = group_reduce<G>(acc[cl]);
          if (gl == 0) res[f * C + cl] = v + b[cl];
        }
      };
      // the next routed row of the job: its activations (and LoRA t entries)
      auto next_row = [&]() {
        f = __ffsll(static_cast<long long>(rows)) - 1;
        if constexpr (LORA) load_lora_t<G, LR>(p, f, gl, ltv[t]);
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
          bool v;
          load_chunk_x(p.x + int64_t(f) * k, slot_chunk<G, FULL>(gl, i, nchunk, v), xv[t][i]);
        }
      };
      if constexpr (kLazy) {
        row_pass(std::true_type{});
        for (rows &= rows - 1; rows; rows &= rows - 1) {
          next_row();
          row_pass(std::false_type{});
        }
      } else {
        // one loop body: a peeled first row measured 168 -> 256 VGPRs (one wave per SIMD) at
        // three chunks per lane
        for (;;) {
          row_pass(std::false_type{});
          rows &= rows - 1;
          if (!rows) break;
          next_row();
        }
      }
    }
  }
  __syncthreads();

  // combine: out[t, col] = sum_s res[t*k+s][col] * w[t, s], slots in order, fp32
  for (int i = threadIdx.x; i < p.tokens * C; i += blockDim.x) {
    const int t = i / C;
    const int cl = i % C;
    const int64_t col = col0 + cl;
    if (col >= n) continue;
    // slots in groups of 8: every LDS read of a group is issued before the in-order sum, so the
    // group costs one LDS round trip, not eight
    float acc = 0.0f;
    for (int s0 = 0; s0 < p.k; s0 += 8) {
      float pr[8];
      bool ok[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int s = s0 + j < p.k ? s0 + j : p.k - 1;
        const int f = t * p.k + s;
        ok[j] = s0 + j < p.k && ((routed_rows >> f) & 1ull);
        pr[j] = mul_f32(res[f * C + cl], wts[f]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) acc = ok[j] ? __fadd_rn(acc, pr[j]) : acc;
    }
    const int64_t o = int64_t(t) * n + col;
    if (p.odt == E4B_FP32) static_cast<float*>(p.out)[o] = acc;
    else if (p.odt == E4B_BF16) static_cast<uint16_t*>(p.out)[o] = from_f<E4B_BF16>(acc);
    else static_cast<uint16_t*>(p.out)[o] = from_f<E4B_FP16>(acc);
  }
}

}  // namespace e4b
