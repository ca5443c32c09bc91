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
#pragma once

#include "common.h"

namespace e4b {

constexpr int kRouteThreads = 512;
constexpr int kRouteWaves = kRouteThreads / kWave;
constexpr int kRouteMaxExperts = 1024;

// Exclusive scan of one int per thread across the 512-thread block (order = thread order).
E4B_DEV int block_exclusive_scan(int v, int* total, int* wsum) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  int x = v;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
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

__global__ void __launch_bounds__(kRouteThreads) route_kernel(const int64_t* __restrict__ idx, int64_t M,
                                                              int E, e4b_routing rt) {
  __shared__ int cnt[kRouteWaves * kRouteMaxExperts];
  __shared__ int wsum[kRouteWaves];
  __shared__ int dropped;
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

  // 1. per-wave histogram
  for (int64_t i = seg0 + lane; i < seg1; i += kWave) {
    const int64_t v = idx[i];
    if (v >= 0 && v < E) {
      atomicAdd(&mycnt[v], 1);
    } else {
      atomicAdd(&dropped, 1);
    }
  }
  __syncthreads();

  // 2. offsets, cursors, tiles, active list. Thread t owns experts 2t and 2t+1.
  const int ea = 2 * tid, eb = 2 * tid + 1;
  int ta = 0, tb = 0;
  if (ea < E)
    for (int w = 0; w < kRouteWaves; ++w) ta += cnt[w * E + ea];
  if (eb < E)
    for (int w = 0; w < kRouteWaves; ++w) tb += cnt[w * E + eb];
  int total;
  const int offa = block_exclusive_scan(ta + tb, &total, wsum);
  const int offb = offa + ta;
  if (ea < E) {
    rt.offsets[ea] = offa;
    int run = offa;
    for (int w = 0; w < kRouteWaves; ++w) {
      const int c = cnt[w * E + ea];
      cnt[w * E + ea] = run;
      run += c;
    }
  }
  if (eb < E) {
    rt.offsets[eb] = offb;
    int run = offb;
    for (int w = 0; w < kRouteWaves; ++w) {
      const int c = cnt[w * E + eb];
      cnt[w * E + eb] = run;
      run += c;
    }
  }
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
  __syncthreads();
  if (tid == 0) {
    rt.meta[0] = min(num_tiles, rt.max_tiles);
    rt.meta[1] = num_active;
    rt.meta[2] = dropped;
    rt.meta[3] = tm;
  }

  // 3. stable placement, one 64-id chunk at a time per wave, chunks in order.
  const unsigned long long below = (lane == 0) ? 0ull : ((~0ull) >> (kWave - lane));
  for (int64_t base = seg0; base < seg1; base += kWave) {
    const int64_t i = base + lane;
    int e = -1;
    if (i < seg1) {
      const int64_t v = idx[i];
      if (v >= 0 && v < E) {
        e = static_cast<int>(v);
      } else {
        rt.inv[i] = -1;
      }
    }
    unsigned long long pending = __ballot(e >= 0);
    while (pending) {
      const int leader = __ffsll(static_cast<long long>(pending)) - 1;
      const int e0 = __shfl(e, leader);
      const unsigned long long m = __ballot(e == e0);
      const int c0 = mycnt[e0];
      if (e == e0) {
        const int pos = c0 + __popcll(m & below);
        rt.sorted_flat[pos] = static_cast<int>(i);
        rt.inv[i] = pos;
      }
      if (lane == leader) mycnt[e0] = c0 + __popcll(m);
      pending &= ~m;
    }
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

template <int DDT, int WDT, int ODT>
__global__ void __launch_bounds__(256) combine_kernel(const void* __restrict__ down,
                                                      const int32_t* __restrict__ inv,
                                                      const void* __restrict__ wts, int64_t T, int k,
                                                      int64_t H, void* __restrict__ out) {
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
      for (int s = 0; s < k; ++s) {
        const int r = inv[t * k + s];
        if (r < 0) continue;
        const float w = load_weight<WDT>(wts, t * k + s);
        float dv[8];
        if constexpr (DDT == E4B_FP32) {
          const float4* dp = reinterpret_cast<const float4*>(static_cast<const float*>(down) + int64_t(r) * H + 8 * c);
          const float4 d0 = dp[0], d1 = dp[1];
          dv[0] = d0.x; dv[1] = d0.y; dv[2] = d0.z; dv[3] = d0.w;
          dv[4] = d1.x; dv[5] = d1.y; dv[6] = d1.z; dv[7] = d1.w;
        } else {
          const uint4 d = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(down) + int64_t(r) * H + 8 * c);
          const uint32_t q[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            dv[2 * j] = lo_f<DDT>(q[j]);
            dv[2 * j + 1] = hi_f<DDT>(q[j]);
          }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = __fadd_rn(acc[j], mul_f32(dv[j], w));
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) store_out<ODT>(out, t * H + 8 * c + j, acc[j]);
    } else {
      float acc = 0.0f;
      for (int s = 0; s < k; ++s) {
        const int r = inv[t * k + s];
        if (r < 0) continue;
        const float w = load_weight<WDT>(wts, t * k + s);
        acc = __fadd_rn(acc, mul_f32(load_down<DDT>(down, int64_t(r) * H + c), w));
      }
      store_out<ODT>(out, t * H + c, acc);
    }
  }
}

}  // namespace e4b
