// Single-token decode in ONE launch: routing, gate_up + epilogue, down and the slot-ordered
// combine of a whole MoE layer.
//
// Two launches per layer (decode_up_kernel, decode_down_kernel) pay the launch and ramp cost
// twice and serialise the two projections' weight streams. Here every block of a co-resident
// grid (gridDim.x <= the blocks that fit at once) does one slice of each projection:
//   1. one round trip: the token's expert ids and router weights, its activation row, the code
//      table pair of this thread, and the block's own launch counter;
//   2. wave-local routing (as in the two-launch kernels) and the NF4 decode table in LDS; the
//      block's gate_up weight loads, the staging of the activation row, then its first down
//      weight loads, so the down projection's bytes stream while gate_up computes;
//   3. gate_up for (routed expert, column) pairs -- the token's routed slots all multiply the
//      same activation row, so an expert's h row is computed once, for its routed position --
//      with the epilogue fused, each h value written through to the device coherence point
//      (sc1 store) into an exchange buffer that holds zeros until then (a computed +0 is stored
//      as -0, so a zero always means "not written yet");
//   4. down: a 32-lane group loads the h chunks of its routed expert with coherent (sc1) loads,
//      repeating them until no value is zero (a bounded wait: past `timeout` real-time ticks it
//      raises the error flag and goes on), then finishes the down projection of the block's
//      output columns over every routed expert, and the combine, in LDS.
// The data moves only through sc1 accesses: no cache-wide writeback or invalidate, no counter a
// consumer must wait for before it may read. Each stream slot owns two exchange buffers; launch
// n on the slot uses buffer n % 2 and zeroes buffer (n + 1) % 2 for the next launch (the
// previous launch, which read that buffer, has ended: launches on a slot run in stream order).
// n comes from the slot's launch counters: every launch adds exactly kSyncPerLaunch to each of
// its kSyncCounters counters (block b adds its share to counter b % kSyncCounters after reading
// it), and a block's own counter cannot yet hold that block's increment when it reads it, so
// n = floor(counter / kSyncPerLaunch). A launch that gave up waiting still adds its share and
// zeroes the next buffer, so later launches are unaffected.
//
// NF4 codes come from the fp16 single-entry table of decode_up_kernel in both projections; bf16
// activations and h are restaged as fp16 scaled by a power of two per 32-value chunk (exact, see
// decode.h), so the only rounding beyond the two-launch path's is that of the fp16 codes.
//
// Measured on MI355X (OLMoE geometry, one token, 16 layers back to back): about 18 us per layer
// against 14.7 us for the two launches. Per-block timestamps show why: both projections' weights
// (28 MB) share one HBM window, so gate_up ends later than it does alone, and the h hand-off
// across the device (write-through store, visibility, re-read by 512 blocks) takes longer than a
// kernel boundary. A variant that waited on per-slot counters instead of polling h measured the
// same. e4b_moe_forward therefore runs this kernel only when asked (E4B_PATH_DECODE_FUSED).
#pragma once

#include "decode.h"

namespace e4b {

constexpr int kSyncSlots = 64;
constexpr int kSyncCounters = 16;
constexpr int kSyncStride = 32;          // unsigned per counter: one 128-byte line each
constexpr unsigned kSyncPerLaunch = 32;  // increments each counter receives per launch
constexpr int kFusedMaxGrid = 512;       // kSyncPerLaunch * kSyncCounters: at least one unit per block
constexpr int kFusedMaxCpld = 3;         // down chunks per lane (k2 <= 3072)
constexpr int kFusedMaxH = 16384;        // h values per exchange buffer: routed experts * k2

struct FusedArgs {
  const uint16_t* x;     // hidden [1, w1.k]
  const int64_t* topk;   // [1, k]
  const void* topk_w;    // [1, k]
  int wdt;               // router weight dtype
  int k, E;
  e4b_qweight w1, w2;
  int epi;
  float alpha, limit;
  uint16_t* hx;          // this slot's two exchange buffers [2][kFusedMaxH], zero until written
  int64_t n_out;         // h columns = w2.k (routed experts * n_out <= kFusedMaxH)
  void* out;             // [1, w2.n] in odt
  int odt;
  unsigned* ctr;         // this slot's kSyncCounters launch counters, kSyncStride apart
  unsigned* errors;      // raised by a wait that timed out
  unsigned add;          // increment per block: kSyncPerLaunch * kSyncCounters / gridDim.x
  unsigned long long timeout;  // wait bound in s_memrealtime ticks (100 MHz)
};

E4B_DEV __amdgpu_buffer_rsrc_t buffer_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, 0x00020000);
}
constexpr int kSc1 = 16;  // cache-policy bits of a buffer access: sc1, coherent at device scope
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// Non-zero when one of the eight 16-bit values of a 16-byte piece is zero.
E4B_DEV uint32_t piece_has_zero(const uint4& v) {
  auto z = [](uint32_t w) { return (w - 0x00010001u) & ~w & 0x80008000u; };
  return z(v.x) | z(v.y) | z(v.z) | z(v.w);
}

template <int DT, int FMT, int G, int CPL, int CPLD>
__global__ void __launch_bounds__(kDecThreads) decode_fused_kernel(FusedArgs p) {
  constexpr int CDT = FMT == E4B_FMT_MXFP4 ? DT : E4B_FP16;  // NF4 codes as fp16 table entries
  constexpr bool kConv = CDT != DT;                          // bf16 activations restaged as fp16
  constexpr int GD = 32;                                     // lanes per down job
  constexpr int C = kDownCols;                               // down columns per block and pass
  constexpr int kUpGroups = kDecThreads / G;
  constexpr int kDnGroups = kDecThreads / GD;
  __shared__ __align__(16) uint4 lut[FMT == E4B_FMT_MXFP4 ? 1 : 256 * kLutRowBytes / 16];
  __shared__ __align__(16) uint4 xs[kDecMaxK / 8 + 1];
  __shared__ int xsh[kConv ? kDecMaxK / 32 + 1 : 1];
  __shared__ WaveRoute route[kDecWaves];
  __shared__ float code2_s[(FMT == E4B_FMT_NF4_DQ) ? 256 : 1];
  __shared__ float res[kDecMaxRows * C];
  __shared__ float wts[kDecMaxRows];
  __shared__ unsigned s_parity;
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & (kWave - 1);
  const int wid = tid / kWave;
  const int M = p.k;  // one token: k routed slots
  const int P = static_cast<int>(gridDim.x), b = static_cast<int>(blockIdx.x);
  const e4b_qweight& w1 = p.w1;
  const e4b_qweight& w2 = p.w2;
  unsigned* const my_ctr = p.ctr + (b % kSyncCounters) * kSyncStride;

  // ---- round trip 1: ids and router weights, this thread's code pair, code2, the token row,
  // the block's own counter (all loads unconditional, converted only after the issue)
  const int64_t id_raw = p.topk[lane < M ? lane : 0];
  const uint32_t wt_bits = p.wdt == E4B_FP32 ? static_cast<const uint32_t*>(p.topk_w)[lane < M ? lane : 0]
                                             : static_cast<const uint16_t*>(p.topk_w)[lane < M ? lane : 0];
  float cf, cs;
  load_pair_codes<FMT>(w1, cf, cs);
  const float c2 = (FMT == E4B_FMT_NF4_DQ) ? w1.code2[tid] : 0.0f;
  const int nx4 = static_cast<int>(w1.k / 8);
  static_assert(kDecMaxK / 8 == 2 * kDecThreads, "two 16-byte pieces per thread");
  const int t0 = tid, t1 = tid + kDecThreads;
  const uint4* x4 = reinterpret_cast<const uint4*>(p.x);
  const uint4 xp0 = x4[t0 < nx4 ? t0 : 0], xp1 = x4[t1 < nx4 ? t1 : 0];
  const unsigned cnt0 = __hip_atomic_load(my_ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  WaveRoute& r = route[wid];
  const int id = (lane < M && id_raw >= 0 && id_raw < p.E) ? static_cast<int>(id_raw) : -1;
  const int nact = wave_route(id, r);
  const unsigned long long routed_rows = __ballot(id >= 0);
  // the decode table first: its stores overlap the first round trip's wait
  if constexpr (FMT != E4B_FMT_MXFP4) store_pair_entry<false>(lut, pair_entry<CDT, false>(cf, cs));

  // ---- gate_up work: (routed expert, column) pairs, one per G-lane group and pass
  const int grp = tid / G, gl = tid % G;
  const int nchunk = static_cast<int>(w1.k / 32);
  const int64_t n1 = w1.n;
  const int64_t npairs = int64_t(nact) * p.n_out;
  const int64_t pstride = int64_t(P) * kUpGroups;
  bool valid[CPL];
  int cidx[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) cidx[i] = slot_chunk<G, false>(gl, i, nchunk, valid[i]);
  struct UpBuf {
    uint4 qa[CPL], qb[CPL];
    RawScale ra[CPL], rb[CPL];
    uint32_t bg, bu;
    float off;
  };
  const bool has_bias1 = w1.bias != nullptr;
  // expert of routed position a; expert 0 (in range) past the last one
  auto expert_at = [&](int a) { return a < nact ? r.act[a] : 0; };
  auto up_load = [&](int64_t pidx, UpBuf& u) {
    const int64_t q = pidx < npairs ? pidx : 0;  // spare loads past the last pair: no branch
    const int a = static_cast<int>(q / p.n_out);
    const int64_t j = q - int64_t(a) * p.n_out;
    const int e = expert_at(a);
    const int64_t row_a = j, row_b = j + n1 / 2;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      u.qa[i] = load_chunk_w(w1, e, row_a, cidx[i]);
      u.qb[i] = load_chunk_w(w1, e, row_b, cidx[i]);
      u.ra[i] = load_scale<FMT>(w1, e, row_a, cidx[i]);
      u.rb[i] = load_scale<FMT>(w1, e, row_b, cidx[i]);
    }
    // without a bias: spare loads of x[0] and x[1] -- distinct addresses, so the compiler cannot
    // merge them into one load and a register copy, which would wait for every load in flight
    const uint16_t* bias = has_bias1 ? static_cast<const uint16_t*>(w1.bias) + int64_t(e) * n1 : p.x;
    u.bg = bias[has_bias1 ? row_a : 0];
    u.bu = bias[has_bias1 ? row_b : 1];
    u.off = (FMT == E4B_FMT_NF4_DQ) ? w1.offset[e] : 0.0f;
  };

  // ---- down work: column tile col0 (C columns), routed expert `job` per 32-lane group
  const int grpd = tid / GD, gld = tid % GD;
  const int nchunk2 = static_cast<int>(w2.k / 32);
  const int64_t n2 = w2.n;
  bool validd[CPLD];
  int cidxd[CPLD];
#pragma unroll
  for (int i = 0; i < CPLD; ++i) cidxd[i] = slot_chunk<GD, false>(gld, i, nchunk2, validd[i]);
  struct DnBuf {
    uint4 q[CPLD][C];
    RawScale rs[CPLD][C];
    uint16_t bb[C];
    float off;
  };
  const bool has_bias2 = w2.bias != nullptr;
  auto dn_load = [&](int job, int64_t col0, DnBuf& d) {
    const int e = expert_at(job);
#pragma unroll
    for (int i = 0; i < CPLD; ++i)
#pragma unroll
      for (int cl = 0; cl < C; ++cl) {
        const int64_t col = col0 + cl < n2 ? col0 + cl : 0;
        d.q[i][cl] = load_chunk_w(w2, e, col, cidxd[i]);
        d.rs[i][cl] = load_scale<FMT>(w2, e, col, cidxd[i]);
      }
    const uint16_t* bias = has_bias2 ? static_cast<const uint16_t*>(w2.bias) + int64_t(e) * n2 : p.x;
#pragma unroll
    for (int cl = 0; cl < C; ++cl) d.bb[cl] = bias[has_bias2 && col0 + cl < n2 ? col0 + cl : cl];  // x[cl]: as above
    d.off = (FMT == E4B_FMT_NF4_DQ) ? w2.offset[e] : 0.0f;
  };

  // ---- round trip 2: the first gate_up pair's loads
  const int64_t pidx0 = int64_t(b) * kUpGroups + grp;
  UpBuf u;
  up_load(pidx0, u);

  // staging while the weights are in flight: the token row (as fp16 per 32-value chunk for
  // NF4 with bf16 activations; the four lanes of a quad hold the four pieces of a chunk), code2,
  // the router weights, the launch's buffer parity
  {
    const int i0 = t0 < nx4 ? t0 : kDecMaxK / 8, i1 = t1 < nx4 ? t1 : kDecMaxK / 8;
    if constexpr (kConv) {
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
  }
  if constexpr (FMT == E4B_FMT_NF4_DQ) code2_s[tid] = c2;
  if (wid == 0) {
    const uint16_t wb = static_cast<uint16_t>(wt_bits);
    wts[lane] = p.wdt == E4B_FP32 ? __uint_as_float(wt_bits)
                                  : (p.wdt == E4B_BF16 ? to_f<E4B_BF16>(wb) : to_f<E4B_FP16>(wb));
  }
  if (tid == 0) {
    s_parity = (cnt0 / kSyncPerLaunch) & 1u;
    // this block's share of the launch count, after its own read of the counter (same address,
    // program order)
    __hip_atomic_fetch_add(my_ctr, p.add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();

  // the first down tile's loads (a prefetch: they stream while gate_up computes)
  DnBuf d;
  const int64_t col_first = int64_t(b) * C;
  dn_load(grpd, col_first, d);

  const unsigned parity = s_parity;
  const uint32_t hbytes = kFusedMaxH * 2;
  const __amdgpu_buffer_rsrc_t hrs = buffer_rsrc(p.hx, 2 * hbytes);
  const uint32_t hcur = parity * hbytes;          // byte offset of this launch's buffer
  const uint32_t hnext = (parity ^ 1u) * hbytes;  // and of the next launch's

  // ---- gate_up: the block's pairs; h stored write-through (sc1) at its routed position
  uint32_t lane_off = LutGeom<false>::lane_off(lane);
  const char* lut_bytes = reinterpret_cast<const char*>(lut);
  auto up_compute = [&](int64_t pidx, const UpBuf& ub) {
    const bool live = pidx < npairs;  // the same for a whole group
    float sa[CPL], sb[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      sa[i] = valid[i] ? resolve_scale<FMT>(ub.ra[i], code2_s, ub.off) : 0.0f;
      sb[i] = valid[i] ? resolve_scale<FMT>(ub.rb[i], code2_s, ub.off) : 0.0f;
    }
    asm volatile("" : "+v"(lane_off));  // table addresses recomputed per pair, not held
    float acc_a = 0.0f, acc_b = 0.0f;
    pair_chunk_dots<CDT, FMT, CPL, true, true>(
        ub.qa, ub.qb, lut_bytes, lane_off,
        [&](int i, uint4 (&xv)[4]) {
#pragma unroll
          for (int qq = 0; qq < 4; ++qq) xv[qq] = xs[cidx[i] * 4 + qq];
          return kConv ? xsh[cidx[i]] : 0;
        },
        [&](int i, float dd, int sh) {
          if constexpr (kConv) dd = __builtin_amdgcn_ldexpf(dd, sh);
          acc_a += valid[i] ? dd * sa[i] : 0.0f;
        },
        [&](int i, float dd, int sh) {
          if constexpr (kConv) dd = __builtin_amdgcn_ldexpf(dd, sh);
          acc_b += valid[i] ? dd * sb[i] : 0.0f;
        },
        [](int) {});
    acc_a = group_reduce<G>(acc_a);
    acc_b = group_reduce<G>(acc_b);
    if (live && gl == 0) {
      uint32_t gb = ub.bg, xb = ub.bu;
      asm volatile("" : "+v"(gb), "+v"(xb));  // bias conversion kept here, after the loads' wait
      const float bg = has_bias1 ? to_f<DT>(static_cast<uint16_t>(gb)) : 0.0f;
      const float bu = has_bias1 ? to_f<DT>(static_cast<uint16_t>(xb)) : 0.0f;
      const float v = gated(p.epi, acc_a, acc_b, p.alpha, p.limit, bg, bu);
      const uint16_t hv = from_f<DT>(v);
      // pidx = a * n_out + j is the h index itself
      __builtin_amdgcn_raw_buffer_store_b16(hv ? hv : uint16_t(0x8000), hrs, static_cast<int>(hcur + 2 * pidx), 0,
                                            kSc1);
    }
  };
  up_compute(pidx0, u);
  for (int64_t pidx = pidx0 + pstride; pidx < npairs; pidx += pstride) {  // more pairs than groups
    up_load(pidx, u);
    up_compute(pidx, u);
  }

  // ---- zero the next launch's buffer (every launch zeroes all of it)
  for (int i = b * kDecThreads + tid; i < kFusedMaxH / 8; i += P * kDecThreads)
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, hrs, static_cast<int>(hnext + 16 * i), 0, kSc1);

  // ---- down + combine over the block's column tiles (the first tile's weights are in flight)
  for (int64_t col0 = col_first; col0 < n2; col0 += int64_t(P) * C) {
    for (int job0 = 0; job0 < nact; job0 += kDnGroups) {
      const int job = job0 + grpd;
      if (col0 != col_first || job0 != 0) dn_load(job, col0, d);
      // h chunks of routed position `job`, read until complete (the whole wave waits together)
      const int jh = job < nact ? job : 0;
      uint4 hv[CPLD][4];
      auto load_h = [&]() {
#pragma unroll
        for (int i = 0; i < CPLD; ++i)
#pragma unroll
          for (int qq = 0; qq < 4; ++qq)
            hv[i][qq] = __builtin_bit_cast(
                uint4, __builtin_amdgcn_raw_buffer_load_b128(
                           hrs, static_cast<int>(hcur + (int64_t(jh) * p.n_out + 32 * cidxd[i]) * 2 + 16 * qq), 0,
                           kSc1));
      };
      auto missing = [&]() {
        uint32_t z = 0;
#pragma unroll
        for (int i = 0; i < CPLD; ++i)
#pragma unroll
          for (int qq = 0; qq < 4; ++qq) z |= piece_has_zero(hv[i][qq]);
        return z != 0 && job < nact;
      };
      load_h();
      if (__any(missing())) {
        const unsigned long long t_start = __builtin_amdgcn_s_memrealtime();
        for (;;) {
          __builtin_amdgcn_s_sleep(1);
          load_h();
          if (!__any(missing())) break;
          if (__builtin_amdgcn_s_memrealtime() - t_start > p.timeout) {
            if (lane == 0) __hip_atomic_fetch_or(p.errors, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
          }
        }
      }
      if (job < nact) {  // whole 32-lane groups
        const unsigned long long rows = r.rows[job];
        float acc[C];
#pragma unroll
        for (int cl = 0; cl < C; ++cl) acc[cl] = 0.0f;
#pragma unroll
        for (int i = 0; i < CPLD; ++i) {
          int sh = 0;
          if constexpr (kConv) {  // the lane holds the whole 32-value chunk
            const uint32_t em = max(max(bf16_exp_max(hv[i][0]), bf16_exp_max(hv[i][1])),
                                    max(bf16_exp_max(hv[i][2]), bf16_exp_max(hv[i][3])));
            const int dd = chunk_shift(em);
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) hv[i][qq] = piece_to_f16(hv[i][qq], dd);
            sh = -dd;
          }
#pragma unroll
          for (int cl = 0; cl < C; ++cl) {
            float dot = weight_dot<CDT, FMT, false>(d.q[i][cl], hv[i], lut_bytes, lane_off);
            if constexpr (kConv) dot = __builtin_amdgcn_ldexpf(dot, sh);
            const float sc = resolve_scale<FMT>(d.rs[i][cl], code2_s, d.off);
            acc[cl] += validd[i] ? dot * sc : 0.0f;
            __builtin_amdgcn_sched_barrier(0);  // keep each chunk's table reads together
          }
        }
#pragma unroll
        for (int cl = 0; cl < C; ++cl) {
          const float v = group_reduce<GD>(acc[cl]) + (has_bias2 ? to_f<DT>(d.bb[cl]) : 0.0f);
          if (gld == 0)
            for (unsigned long long rr = rows; rr; rr &= rr - 1)
              res[(__ffsll(static_cast<long long>(rr)) - 1) * C + cl] = v;
        }
      }
    }
    __syncthreads();
    // combine: out[col] = sum over slots s in order of res[s][col] * w[s], fp32, slots in groups
    // of 8 (each group's LDS reads issued before its in-order sum)
    if (tid < C && col0 + tid < n2) {
      const int cl = tid;
      float acc = 0.0f;
      for (int s0 = 0; s0 < M; s0 += 8) {
        float pr[8];
        bool ok[8];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
          const int s = s0 + jj < M ? s0 + jj : M - 1;
          ok[jj] = s0 + jj < M && ((routed_rows >> s) & 1ull);
          pr[jj] = mul_f32(res[s * C + cl], wts[s]);
        }
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) acc = ok[jj] ? __fadd_rn(acc, pr[jj]) : acc;
      }
      const int64_t o = col0 + cl;
      if (p.odt == E4B_FP32) static_cast<float*>(p.out)[o] = acc;
      else if (p.odt == E4B_BF16) static_cast<uint16_t*>(p.out)[o] = from_f<E4B_BF16>(acc);
      else static_cast<uint16_t*>(p.out)[o] = from_f<E4B_FP16>(acc);
    }
    __syncthreads();  // res is rewritten by the next tile
  }
}

}  // namespace e4b
