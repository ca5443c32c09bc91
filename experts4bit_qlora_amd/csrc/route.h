// Token -> expert routing permutation and the deterministic combine.
//
// route_kernel restates engines/fast.py:125-133 on the device: the expert-sorted order is
// exactly numpy/torch's STABLE argsort of top_k_index.reshape(-1) (equal ids keep their flat
// order), the per-expert counts are bincount(minlength=E), and the active experts ascend.
// It is a stable counting sort in one workgroup of 8 waves:
//   1. each wave histograms a contiguous, chunk-aligned segment into its own LDS row;
//   2. an exclusive scan over (expert, wave) turns the rows into write cursors;
//   3. each wave re-walks its segment 64 ids at a time, in order; equal ids inside a chunk
//      are ranked by lane (ballot + popcount over the lanes below), so the output order is
//      segment order, then chunk order, then lane order == flat order.
// It also emits the tile list (expert, first row) the grouped MFMA GEMM schedules from, so
// no count ever travels to the host (the reference's .tolist() sync, fast.py:132-133).
//
// Beyond kRouteSingleMaxRows ids one workgroup is too narrow, and the same counting sort runs
// in four launches over 256-id chunks (four waves of 64 ids each):
//   route_count_kernel    per-chunk histograms (one LDS add per distinct expert per 64 ids);
//   route_colscan_kernel  one workgroup per expert: each chunk's rows of the expert in earlier
//                         chunks (chunk order = flat order), and the expert's total;
//   route_tables_kernel   one workgroup: offsets, tiles, active list, meta from the totals;
//   route_place_kernel    each chunk re-walks its ids in order from offset + earlier chunks.
// (One workgroup doing the column sums and the rewrite took 18.5 us at 32,768 ids over 128
// experts; the columns are independent.)
//
// For prefill the table step (route_kernel's, or route_tables_kernel's) also re-tiles the routed
// rows into two lists (emit_split_tiles): big tiles, plus a small tile for an expert whose last
// big tile would hold only a few rows.
#pragma once

#include <rocprim/warp/warp_scan.hpp>

#include "common.h"
#include "scale.h"

namespace e4b {

constexpr int kRouteThreads = 512;
constexpr int kRouteWaves = kRouteThreads / kWave;
constexpr int kRouteMaxExperts = 1024;
constexpr int kRouteSingleMaxRows = 4096;  // above: the four-launch chunked route
constexpr int kRouteChunk = 4 * kWave;     // ids per chunk (one workgroup) in the chunked route

// Exclusive scan of one int per thread across the 512-thread block (order = thread order).
E4B_DEV int block_exclusive_scan(int v, int* total, int* wsum) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  // the wave's inclusive scan in registers (rocPRIM's cross-lane scan: DPP row shifts and
  // broadcasts on gfx950, no LDS round trip per step)
  int x;
  {
    using wave_scan = rocprim::warp_scan<int, kWave>;
    typename wave_scan::storage_type st;
    wave_scan().inclusive_scan(v, x, st);
  }
  if (lane == kWave - 1) wsum[wid] = x;
  __syncthreads();
  int base = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kRouteWaves; ++i) {
    const int s = wsum[i];
    base += (i < wid) ? s : 0;
    tot += s;
  }
  __syncthreads();
  *total = tot;
  return base + x - v;
}

// Stable rank of each lane's id among the wave's 64 ids: the number of lanes below holding the
// same id (e < 0 for none; its rank is not used). The ids go through this wave's 16-byte
// aligned 64-int LDS row s, written and read by the wave alone in program order, and each lane
// compares its id with all 64, four per 16-byte read: ~200 VALU operations per chunk, where a
// loop over the distinct ids (ballot, broadcast, cursor read per id) pays an LDS round trip per
// distinct id.
E4B_DEV int wave_rank(int e, int* s) {
  const int lane = threadIdx.x & (kWave - 1);
  s[lane] = e;
  __builtin_amdgcn_wave_barrier();
  const int4* s4 = reinterpret_cast<const int4*>(s);
  // (the lane index is opaque to the compiler, so its 64 comparisons are not hoisted out of a
  // caller's loop and held as 64 scalar masks)
  int ln = lane;
  asm volatile("" : "+v"(ln));
  int r = 0;
#pragma unroll
  for (int j = 0; j < kWave / 4; ++j) {
    const int4 v = s4[j];
    r += (v.x == e && 4 * j + 0 < ln) ? 1 : 0;
    r += (v.y == e && 4 * j + 1 < ln) ? 1 : 0;
    r += (v.z == e && 4 * j + 2 < ln) ? 1 : 0;
    r += (v.w == e && 4 * j + 3 < ln) ? 1 : 0;
  }
  __builtin_amdgcn_wave_barrier();
  return r;
}

// Two tile lists from the routed offsets, for grouped GEMMs run at two tile heights. A tile
// costs about the same whatever its height until its MFMA work catches up with its weight
// decoding (the whole expert matrix per tile), so every expert keeps big tiles
// (`big.tile_m` rows, the last one partial) unless its last big tile would hold at most
// `small.tile_m` rows: those rows go to one small tile instead. The big list holds every
// expert's full tiles first, then the partial ones, so a grid that takes the list in order runs
// the long tiles first and the short ones last. One 512-thread block; thread t owns experts 2t
// and 2t + 1 (counts ca, cb from offsets oa, ob); active / dropped go to both lists' meta.
struct SplitTiles {
  e4b_routing big, small;
  int on;  // 0: no split lists
};

E4B_DEV void emit_split_tiles(int ca, int cb, int oa, int ob, int active, int dropped, const e4b_routing& big,
                              const e4b_routing& small, int* wsum) {
  const int tid = threadIdx.x;
  const int ea = 2 * tid, eb = 2 * tid + 1;
  const int bt = big.tile_m, st = small.tile_m;
  // remainder past the full big tiles: one partial big tile, or one small tile when it fits
  const int ra = ca % bt, rb = cb % bt;
  const int nsa = (ra > 0 && ra <= st) ? 1 : 0, nsb = (rb > 0 && rb <= st) ? 1 : 0;
  const int nfa = ca / bt, nfb = cb / bt;                        // full big tiles
  const int npa = ra > st ? 1 : 0, npb = rb > st ? 1 : 0;        // partial big tiles
  int nfull, npart, nsmall;
  const int f0 = block_exclusive_scan(nfa + nfb, &nfull, wsum);
  const int p0 = block_exclusive_scan(npa + npb, &npart, wsum);
  const int s0 = block_exclusive_scan(nsa + nsb, &nsmall, wsum);
  auto put_big = [&](int t, int e, int row) {
    if (t < big.max_tiles) {
      big.tiles[2 * t] = e;
      big.tiles[2 * t + 1] = row;
    }
  };
  for (int j = 0; j < nfa + nfb; ++j) {
    const bool in_a = j < nfa;
    put_big(f0 + j, in_a ? ea : eb, in_a ? oa + j * bt : ob + (j - nfa) * bt);
  }
  for (int j = 0; j < npa + npb; ++j) {
    const bool in_a = j < npa;
    put_big(nfull + p0 + j, in_a ? ea : eb, in_a ? oa + nfa * bt : ob + nfb * bt);
  }
  for (int j = 0; j < nsa + nsb; ++j) {
    const int t = s0 + j;
    const bool in_a = j < nsa;
    if (t < small.max_tiles) {
      small.tiles[2 * t] = in_a ? ea : eb;
      small.tiles[2 * t + 1] = in_a ? oa + nfa * bt : ob + nfb * bt;  // at most one small tile per expert
    }
  }
  if (tid == 0) {
    big.meta[0] = min(nfull + npart, big.max_tiles);
    small.meta[0] = min(nsmall, small.max_tiles);
    big.meta[1] = small.meta[1] = active;
    big.meta[2] = small.meta[2] = dropped;
    big.meta[3] = bt;
    small.meta[3] = st;
  }
}

// Offsets, tile list, active list and meta from per-expert totals. Thread t of the 512-thread
// block owns experts 2t and 2t+1 with totals ta and tb; offa / offb receive their first sorted
// rows. `dropped` must be the same value in every thread.
E4B_DEV void emit_expert_tables(int ta, int tb, int E, int dropped, const e4b_routing& rt, int* wsum, int& offa,
                                int& offb, const SplitTiles* sp = nullptr) {
  const int tid = threadIdx.x;
  const int ea = 2 * tid, eb = 2 * tid + 1;
  int total;
  offa = block_exclusive_scan(ta + tb, &total, wsum);
  offb = offa + ta;
  if (ea < E) rt.offsets[ea] = offa;
  if (eb < E) rt.offsets[eb] = offb;
  if (tid == 0) rt.offsets[E] = total;

  const int tm = rt.tile_m;
  const int na = (ta + tm - 1) / tm, nb = (tb + tm - 1) / tm;
  int num_tiles;
  const int tbase = block_exclusive_scan(na + nb, &num_tiles, wsum);
  for (int j = 0; j < na; ++j) {
    const int t = tbase + j;
    if (t < rt.max_tiles) {
      rt.tiles[2 * t] = ea;
      rt.tiles[2 * t + 1] = offa + j * tm;
    }
  }
  for (int j = 0; j < nb; ++j) {
    const int t = tbase + na + j;
    if (t < rt.max_tiles) {
      rt.tiles[2 * t] = eb;
      rt.tiles[2 * t + 1] = offb + j * tm;
    }
  }
  int num_active;
  const int abase = block_exclusive_scan((ta > 0) + (tb > 0), &num_active, wsum);
  if (ta > 0) rt.active[abase] = ea;
  if (tb > 0) rt.active[abase + (ta > 0)] = eb;
  if (tid == 0) {
    rt.meta[0] = min(num_tiles, rt.max_tiles);
    rt.meta[1] = num_active;
    rt.meta[2] = dropped;
    rt.meta[3] = tm;
  }
  // the prefill's two tile lists from the same counts and offsets: no launch of their own
  if (sp && sp->on) emit_split_tiles(ta, tb, offa, offb, num_active, dropped, sp->big, sp->small, wsum);
}

// The whole permutation in one kRouteThreads-thread workgroup (M <= kRouteSingleMaxRows).
E4B_DEV void route_single(const int64_t* __restrict__ idx, int64_t M, int E, const e4b_routing& rt,
                          const SplitTiles* sp = nullptr) {
  __shared__ int cnt[kRouteWaves * kRouteMaxExperts];
  __shared__ int wsum[kRouteWaves];
  __shared__ int dropped;
  __shared__ __align__(16) int rank_s[kRouteWaves][kWave];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wid = tid / kWave;

  for (int i = tid; i < kRouteWaves * E; i += kRouteThreads) cnt[i] = 0;
  if (tid == 0) dropped = 0;
  __syncthreads();

  const int64_t nchunks = (M + kWave - 1) / kWave;
  const int64_t chunks_per_wave = (nchunks + kRouteWaves - 1) / kRouteWaves;
  const int64_t seg0 = min(M, wid * chunks_per_wave * kWave);
  const int64_t seg1 = min(M, (wid + 1) * chunks_per_wave * kWave);
  int* mycnt = cnt + wid * E;

  // The wave's ids, loaded once with every load in flight (the histogram and the placement each
  // walked them with one dependent load per 64-id chunk): chunk j of the wave holds ids seg0 +
  // 64 j + lane, kept as experts (-1: past the segment, -2: dropped).
  constexpr int kPer = kRouteSingleMaxRows / kRouteThreads;  // chunks per wave at most
  static_assert(kPer * kRouteThreads == kRouteSingleMaxRows, "whole chunks per wave");
  int ev[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) ev[j] = -1;
  if (seg1 > seg0) {  // uniform; no load at all when the wave has no ids (M may be 0, idx NULL)
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int64_t i = seg0 + int64_t(j) * kWave + lane;
      const int64_t v = idx[i < seg1 ? i : seg1 - 1];
      ev[j] = i >= seg1 ? -1 : (v >= 0 && v < E) ? static_cast<int>(v) : -2;
    }
  }

  // 1. per-wave histogram
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    if (ev[j] >= 0) atomicAdd(&mycnt[ev[j]], 1);
    else if (ev[j] == -2) atomicAdd(&dropped, 1);
  }
  __syncthreads();

  // 2. offsets, cursors, tiles, active list. Thread t owns experts 2t and 2t+1.
  const int ea = 2 * tid, eb = 2 * tid + 1;
  int ta = 0, tb = 0;
  if (ea < E)
    for (int w = 0; w < kRouteWaves; ++w) ta += cnt[w * E + ea];
  if (eb < E)
    for (int w = 0; w < kRouteWaves; ++w) tb += cnt[w * E + eb];
  const int ndropped = dropped;
  int offa, offb;
  emit_expert_tables(ta, tb, E, ndropped, rt, wsum, offa, offb, sp);
  if (ea < E) {
    int run = offa;
    for (int w = 0; w < kRouteWaves; ++w) {
      const int c = cnt[w * E + ea];
      cnt[w * E + ea] = run;
      run += c;
    }
  }
  if (eb < E) {
    int run = offb;
    for (int w = 0; w < kRouteWaves; ++w) {
      const int c = cnt[w * E + eb];
      cnt[w * E + eb] = run;
      run += c;
    }
  }
  __syncthreads();

  // 3. stable placement, one 64-id chunk at a time per wave, chunks in order: an id's position
  // is its expert's cursor plus its rank among the chunk's equal ids; then each id bumps its
  // expert's cursor (the wave's cursor reads precede its adds in LDS order).
  int* rs = rank_s[wid];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int64_t base = seg0 + int64_t(j) * kWave;
    if (base >= seg1) break;  // uniform over the wave
    const int64_t i = base + lane;
    const int e = ev[j] >= 0 ? ev[j] : -1;
    if (ev[j] == -2) rt.inv[i] = -1;
    const int rank = wave_rank(e, rs);
    if (e >= 0) {
      const int pos = mycnt[e] + rank;
      rt.sorted_flat[pos] = static_cast<int>(i);
      rt.inv[i] = pos;
    }
    __builtin_amdgcn_wave_barrier();
    if (e >= 0) atomicAdd(&mycnt[e], 1);
    __builtin_amdgcn_wave_barrier();
  }
}

__global__ void __launch_bounds__(kRouteThreads) route_kernel(const int64_t* __restrict__ idx, int64_t M,
                                                              int E, e4b_routing rt, SplitTiles sp) {
  route_single(idx, M, E, rt, &sp);
}

// route_kernel and, in the same launch, row_exp_row over the T rows of x: block 0 routes, block
// b > 0 takes rows kRouteWaves (b - 1) .. + kRouteWaves - 1, one wave each. The fused forward's
// token rows (exponents and scaled fp16 copies) then cost no launch of their own.
template <int RP>
__global__ void __launch_bounds__(kRouteThreads) route_rowexp_kernel(const int64_t* __restrict__ idx, int64_t M,
                                                                     int E, e4b_routing rt, SplitTiles sp,
                                                                     const uint16_t* x, int64_t T, int64_t k,
                                                                     int32_t* row_exp, uint16_t* x16) {
  if (blockIdx.x == 0) {
    route_single(idx, M, E, rt, &sp);
    return;
  }
  const int64_t row = int64_t(blockIdx.x - 1) * kRouteWaves + threadIdx.x / kWave;
  if (row < T) row_exp_row<RP>(x, row, k, row_exp, x16);
}

// ---- chunked route (M > kRouteSingleMaxRows); counts is [nchunks, E + 1] int32, column E the
// chunk's dropped ids. A chunk of kRouteChunk ids is one workgroup of 4 waves, 64 ids each.

constexpr int kChunkWaves = kRouteChunk / kWave;

E4B_DEV int chunk_id(const int64_t* idx, int64_t i, int64_t M, int E, bool& dropped) {
  dropped = false;
  if (i >= M) return -1;
  const int64_t v = idx[i];
  if (v >= 0 && v < E) return static_cast<int>(v);
  dropped = true;
  return -1;
}

// Per-wave histogram of the wave's 64 ids into its LDS row c (E entries, one LDS add per id),
// returning the number of dropped ids.
E4B_DEV int wave_histogram(int e, bool drop, int* c, int E) {
  const int lane = threadIdx.x & (kWave - 1);
  for (int x = lane; x < E; x += kWave) c[x] = 0;
  __builtin_amdgcn_wave_barrier();
  if (e >= 0) atomicAdd(&c[e], 1);
  __builtin_amdgcn_wave_barrier();
  return __popcll(__ballot(drop));
}

// The counts of chunk `chunk` (one kRouteChunk-thread workgroup).
E4B_DEV void route_count_chunk(const int64_t* __restrict__ idx, int64_t M, int E, int32_t* __restrict__ counts,
                               int64_t chunk) {
  __shared__ int c[kChunkWaves][kRouteMaxExperts];
  __shared__ int nd[kChunkWaves];
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  bool drop;
  const int e = chunk_id(idx, chunk * kRouteChunk + threadIdx.x, M, E, drop);
  const int d = wave_histogram(e, drop, c[wid], E);
  if (lane == 0) nd[wid] = d;
  __syncthreads();
  int32_t* row = counts + chunk * (E + 1);
  for (int x = threadIdx.x; x < E; x += kRouteChunk) {
    int t = 0;
#pragma unroll
    for (int w = 0; w < kChunkWaves; ++w) t += c[w][x];
    row[x] = t;
  }
  if (threadIdx.x == 0) {
    int t = 0;
#pragma unroll
    for (int w = 0; w < kChunkWaves; ++w) t += nd[w];
    row[E] = t;
  }
}

__global__ void __launch_bounds__(kRouteChunk) route_count_kernel(const int64_t* __restrict__ idx, int64_t M, int E,
                                                                  int32_t* __restrict__ counts) {
  route_count_chunk(idx, M, E, counts, blockIdx.x);
}

// route_count_kernel's nchunks blocks and, after them, row_exp_row over the T rows of x
// (kChunkWaves rows per block, one wave each) in one launch.
template <int RP>
__global__ void __launch_bounds__(kRouteChunk) route_count_rowexp_kernel(const int64_t* __restrict__ idx, int64_t M,
                                                                         int E, int32_t* __restrict__ counts,
                                                                         int64_t nchunks, const uint16_t* x, int64_t T,
                                                                         int64_t k, int32_t* row_exp, uint16_t* x16) {
  if (blockIdx.x < nchunks) {
    route_count_chunk(idx, M, E, counts, blockIdx.x);
    return;
  }
  const int64_t row = (int64_t(blockIdx.x) - nchunks) * kChunkWaves + threadIdx.x / kWave;
  if (row < T) row_exp_row<RP>(x, row, k, row_exp, x16);
}

// Column scan, one workgroup per column x of the [nchunks, E + 1] count matrix (x < E: expert x,
// x == E: the dropped ids): each chunk's count becomes the number of rows of that column in
// earlier chunks (its offset within the expert's sorted rows), and the column's total goes to
// totals[x] (rt.offsets, rewritten as sorted offsets by route_tables_kernel).
__global__ void __launch_bounds__(kRouteThreads) route_colscan_kernel(int64_t nchunks, int E,
                                                                      int32_t* __restrict__ counts,
                                                                      int32_t* __restrict__ totals) {
  __shared__ int wsum[kRouteWaves];
  const int x = blockIdx.x;
  const int64_t pitch = E + 1;
  int carry = 0;
  for (int64_t b0 = 0; b0 < nchunks; b0 += kRouteThreads) {
    const int64_t b = b0 + threadIdx.x;
    const int v = b < nchunks ? counts[b * pitch + x] : 0;
    int tot;
    const int ex = block_exclusive_scan(v, &tot, wsum);
    if (b < nchunks) counts[b * pitch + x] = carry + ex;
    carry += tot;
  }
  if (threadIdx.x == 0) totals[x] = carry;
}

// One workgroup: the expert totals route_colscan_kernel left in rt.offsets[0 .. E) (and the
// dropped count in rt.offsets[E]) become the sorted offsets, tiles, active list and meta, and
// with sp.on the prefill's two tile lists.
__global__ void __launch_bounds__(kRouteThreads) route_tables_kernel(int E, e4b_routing rt, SplitTiles sp) {
  __shared__ int wsum[kRouteWaves];
  const int tid = threadIdx.x;
  const int ta = (2 * tid < E) ? rt.offsets[2 * tid] : 0;
  const int tb = (2 * tid + 1 < E) ? rt.offsets[2 * tid + 1] : 0;
  const int dropped = rt.offsets[E];
  // every total is read before the first scan's barrier, so before any offset is written
  int offa, offb;
  emit_expert_tables(ta, tb, E, dropped, rt, wsum, offa, offb, &sp);
}

__global__ void __launch_bounds__(kRouteChunk) route_place_kernel(const int64_t* __restrict__ idx, int64_t M, int E,
                                                                  const int32_t* __restrict__ counts, e4b_routing rt) {
  __shared__ int c[kChunkWaves][kRouteMaxExperts];
  __shared__ __align__(16) int rank_s[kChunkWaves][kWave];
  const int wid = threadIdx.x / kWave;
  const int64_t i = int64_t(blockIdx.x) * kRouteChunk + threadIdx.x;
  bool drop;
  const int e = chunk_id(idx, i, M, E, drop);
  wave_histogram(e, drop, c[wid], E);
  __syncthreads();
  // cursors: the expert's first sorted row, plus its rows in earlier chunks, plus the ids of the
  // same expert in earlier waves
  const int32_t* row = counts + int64_t(blockIdx.x) * (E + 1);
  for (int x = threadIdx.x; x < E; x += kRouteChunk) {
    int run = rt.offsets[x] + row[x];
#pragma unroll
    for (int w = 0; w < kChunkWaves; ++w) {
      const int cw = c[w][x];
      c[w][x] = run;
      run += cw;
    }
  }
  __syncthreads();
  if (drop) rt.inv[i] = -1;
  const int rank = wave_rank(e, rank_s[wid]);
  if (e >= 0) {
    const int pos = c[wid][e] + rank;
    rt.sorted_flat[pos] = static_cast<int>(i);
    rt.inv[i] = pos;
  }
}

// out[t, :] = out_t( sum_s float(down[inv[t*k+s], :]) * w[t, s] ), s ascending, fp32 adds of
// rounded fp32 products -- engines/fast.py:158 and 276-278 (buf[order] = down.float() * w;
// buf.view(T, k, H).sum(1).to(dtype)). Dropped slots (inv < 0) contribute nothing.
template <int WDT>
E4B_DEV float load_weight(const void* w, int64_t i) {
  if constexpr (WDT == E4B_FP32) {
    return static_cast<const float*>(w)[i];
  } else {
    return to_f<WDT>(static_cast<const uint16_t*>(w)[i]);
  }
}

// Routing of host-described row groups whose expert ids are on the device (the grouped call of
// engines/pipelined.py:502-508: fixed group sizes, device ids, no host read-back). Group g holds
// input rows [off[g], off[g + 1]) for expert ids[g]; the rows of an expert's groups go to its
// segment in group order (sorted_flat: sorted row -> input row, inv: input row -> sorted row, -1
// for a group whose id is outside [0, E)). The offsets come as a kernel argument, so no host
// data travels through memory. One 512-thread block; groups <= kGroupsMax.
constexpr int kGroupsMax = 512;
struct GroupOffsets {
  int32_t off[kGroupsMax + 1];
};

__global__ void __launch_bounds__(kRouteThreads) route_groups_kernel(GroupOffsets go, int G,
                                                                     const int64_t* __restrict__ ids, int E,
                                                                     e4b_routing rt) {
  __shared__ int goff[kGroupsMax + 1];
  __shared__ int gid[kGroupsMax];
  __shared__ int gpos[kGroupsMax];
  __shared__ int cnt[kRouteMaxExperts];
  __shared__ int start[kRouteMaxExperts];
  __shared__ int wsum[kRouteWaves];
  __shared__ int dropped;
  const int tid = threadIdx.x;
  for (int i = tid; i < E; i += kRouteThreads) cnt[i] = 0;
  for (int i = tid; i <= G; i += kRouteThreads) goff[i] = go.off[i];
  if (tid == 0) dropped = 0;
  int e = -1;
  if (tid < G) {
    const int64_t v = ids[tid];
    e = (v >= 0 && v < E) ? static_cast<int>(v) : -1;
    gid[tid] = e;
  }
  __syncthreads();
  if (tid < G) {
    const int sz = goff[tid + 1] - goff[tid];
    if (e >= 0) atomicAdd(&cnt[e], sz);
    else atomicAdd(&dropped, sz);
  }
  __syncthreads();
  const int ea = 2 * tid, eb = 2 * tid + 1;
  int offa, offb;
  emit_expert_tables(ea < E ? cnt[ea] : 0, eb < E ? cnt[eb] : 0, E, dropped, rt, wsum, offa, offb);
  if (ea < E) start[ea] = offa;
  if (eb < E) start[eb] = offb;
  __syncthreads();
  // a group's first sorted row: its expert's first row plus the rows of earlier groups of it
  if (tid < G && e >= 0) {
    int before = 0;
    for (int g = 0; g < tid; ++g) before += (gid[g] == e) ? goff[g + 1] - goff[g] : 0;
    gpos[tid] = start[e] + before;
  }
  __syncthreads();
  for (int g = 0; g < G; ++g) {
    const int r0 = goff[g], n = goff[g + 1] - r0, eg = gid[g];
    for (int i = tid; i < n; i += kRouteThreads) {
      if (eg >= 0) {
        rt.sorted_flat[gpos[g] + i] = r0 + i;
        rt.inv[r0 + i] = gpos[g] + i;
      } else {
        rt.inv[r0 + i] = -1;
      }
    }
  }
}

template <int ODT>
E4B_DEV void store_out(void* out, int64_t i, float v) {
  if constexpr (ODT == E4B_FP32) {
    static_cast<float*>(out)[i] = v;
  } else {
    static_cast<uint16_t*>(out)[i] = from_f<ODT>(v);
  }
}

template <int DDT>
E4B_DEV float load_down(const void* d, int64_t i) {
  if constexpr (DDT == E4B_FP32) {
    return static_cast<const float*>(d)[i];
  } else {
    return to_f<DDT>(static_cast<const uint16_t*>(d)[i]);
  }
}

// fp16 down rows with their operand scales left on (GemmArgs::out_f16_shift): the sorted row r
// of slot (t, s) holds its values times 2^(exp_shift(rexp[r]) + wshift[e] - shift), e =
// idx[t k + s]; the combine folds the inverse power of two into the slot's router weight (exact:
// (v 2^d) w and v (w 2^d) round alike while w 2^d stays a normal fp32).
struct CombineScale {
  const int32_t* rexp;    // h row exponents by sorted row (row_exp_kernel)
  const int64_t* idx;     // top_k_index [T, k]
  const int32_t* wshift;  // the down weights' expert shifts
  int shift;
};

template <int DDT, int WDT, int ODT, bool SC = false>
__global__ void __launch_bounds__(256) combine_kernel(const void* __restrict__ down,
                                                      const int32_t* __restrict__ inv,
                                                      const void* __restrict__ wts, int64_t T, int k,
                                                      int64_t H, void* __restrict__ out, CombineScale cs) {
  static_assert(!SC || DDT == E4B_FP16, "scaled down rows are fp16");
  const bool vec = (H % 8) == 0;
  const int64_t per_tok = vec ? H / 8 : H;
  const int64_t total = T * per_tok;
  for (int64_t g = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; g < total;
       g += int64_t(gridDim.x) * blockDim.x) {
    const int64_t t = g / per_tok;
    const int64_t c = g % per_tok;
    if (vec) {
      float acc[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
      // slots eight at a time: every load of the eight is issued before the in-order sum (a
      // dropped slot reads row 0 and is left out by a select, not a branch around its loads)
      constexpr int kS = 8;
      for (int s0 = 0; s0 < k; s0 += kS) {
        int rr[kS];
        bool ok[kS];
        float w[kS], dv[kS][8];
        int64_t ei[kS];        // SC: the slot's expert
        int rx[kS], wx[kS];    // SC: its row exponent and expert shift
#pragma unroll
        for (int u = 0; u < kS; ++u) {
          const int s = s0 + u < k ? s0 + u : k - 1;
          rr[u] = inv[t * k + s];
          w[u] = load_weight<WDT>(wts, t * k + s);
          if constexpr (SC) ei[u] = cs.idx[t * k + s];
          ok[u] = s0 + u < k && rr[u] >= 0;
        }
        // the scale loads go out beside the row loads; they are used only in the sum
#pragma unroll
        for (int u = 0; u < kS; ++u) {
          const int64_t r = rr[u] >= 0 ? rr[u] : 0;
          if constexpr (SC) {
            rx[u] = cs.rexp[r];
            wx[u] = cs.wshift[ok[u] ? ei[u] : 0];
          }
          if constexpr (DDT == E4B_FP32) {
            const float4* dp = reinterpret_cast<const float4*>(static_cast<const float*>(down) + r * H + 8 * c);
            const float4 d0 = dp[0], d1 = dp[1];
            dv[u][0] = d0.x; dv[u][1] = d0.y; dv[u][2] = d0.z; dv[u][3] = d0.w;
            dv[u][4] = d1.x; dv[u][5] = d1.y; dv[u][6] = d1.z; dv[u][7] = d1.w;
          } else {
            const uint4 d = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(down) + r * H + 8 * c);
            const uint32_t q[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              dv[u][2 * j] = lo_f<DDT>(q[j]);
              dv[u][2 * j + 1] = hi_f<DDT>(q[j]);
            }
          }
        }
#pragma unroll
        for (int u = 0; u < kS; ++u) {
          if constexpr (SC) w[u] = __builtin_amdgcn_ldexpf(w[u], cs.shift - exp_shift(rx[u]) - wx[u]);
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[j] = ok[u] ? __fadd_rn(acc[j], mul_f32(dv[u][j], w[u])) : acc[j];
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) store_out<ODT>(out, t * H + 8 * c + j, acc[j]);
    } else {
      float acc = 0.0f;
      for (int s = 0; s < k; ++s) {
        const int r = inv[t * k + s];
        if (r < 0) continue;
        float w = load_weight<WDT>(wts, t * k + s);
        if constexpr (SC) w = __builtin_amdgcn_ldexpf(w, cs.shift - exp_shift(cs.rexp[r]) - cs.wshift[cs.idx[t * k + s]]);
        acc = __fadd_rn(acc, mul_f32(load_down<DDT>(down, int64_t(r) * H + c), w));
      }
      store_out<ODT>(out, t * H + c, acc);
    }
  }
}

}  // namespace e4b
