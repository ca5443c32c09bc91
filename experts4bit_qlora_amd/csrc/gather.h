// Address-table row gather: the copy kernel of a routed-expert residency engine
// (engines/pipelined.py:117-151). Slot s of a slot store receives n_bytes read at the absolute
// address src[s] -- device memory, or pinned host memory mapped into the device's address
// space, so one launch serves resident (hot) and streamed (cold) rows alike -- unless the slot
// already holds the wanted row: ident[s] == have[s] skips the slot. The decision is on the
// device, so a decode step enqueues the same launches whatever the routing.
#pragma once

#include "common.h"

namespace e4b {

constexpr int kGatherThreads = 256;
constexpr int64_t kGatherChunk = 64 * 1024;  // bytes per block (blockIdx.x), slot = blockIdx.y

__global__ void __launch_bounds__(kGatherThreads) gather_rows_kernel(
    uint8_t* __restrict__ dst, int64_t row_bytes, int64_t dst_off, const int64_t* __restrict__ src,
    const int64_t* __restrict__ ident, const int64_t* __restrict__ have, int64_t n_bytes,
    unsigned long long* __restrict__ copied) {
  const int64_t s = blockIdx.y;
  if (ident[s] == have[s]) return;  // the whole block: the slot already holds this row
  const int64_t b0 = int64_t(blockIdx.x) * kGatherChunk;
  const int64_t b1 = min(n_bytes, b0 + kGatherChunk);
  const uint8_t* from = reinterpret_cast<const uint8_t*>(src[s]);
  uint8_t* to = dst + s * row_bytes + dst_off;
  const uintptr_t align = reinterpret_cast<uintptr_t>(from) | reinterpret_cast<uintptr_t>(to);
  if ((align & 15) == 0 && (b0 & 15) == 0 && (b1 & 15) == 0) {  // the same for every lane
    for (int64_t i = b0 + 16 * int64_t(threadIdx.x); i < b1; i += 16 * kGatherThreads)
      *reinterpret_cast<uint4*>(to + i) = *reinterpret_cast<const uint4*>(from + i);
  } else if ((align & 7) == 0 && (b0 & 7) == 0 && (b1 & 7) == 0) {
    for (int64_t i = b0 + 8 * int64_t(threadIdx.x); i < b1; i += 8 * kGatherThreads)
      *reinterpret_cast<uint64_t*>(to + i) = *reinterpret_cast<const uint64_t*>(from + i);
  } else {
    for (int64_t i = b0 + threadIdx.x; i < b1; i += kGatherThreads) to[i] = from[i];
  }
  if (copied != nullptr && blockIdx.x == 0 && threadIdx.x == 0) atomicAdd(copied, static_cast<unsigned long long>(n_bytes));
}

}  // namespace e4b
