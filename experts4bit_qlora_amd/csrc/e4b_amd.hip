// C-ABI entry points of libe4b_amd.so (declared in include/e4b_amd.h).
//
// Host code only validates, picks a kernel instantiation and launches on the caller's stream.
// No device memory is allocated here and no call synchronises the device.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

#include <mutex>
#include <utility>

#include "common.h"
#include "decode.h"
#include "decode_launch.h"
#include "dequant.h"
#include "gather.h"
#include "gemm.h"
#include "gemm_launch.h"
#include "gemv.h"
#include "lora.h"
#include "lora_mfma.h"
#include "route.h"
#include "scale.h"
#include "train.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(E4B_ELAUNCH, "%s: %s", what, hipGetErrorString(err));
  return E4B_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr int kMaxDevices = 64;
// Second streams of prefill forwards on each device, each with its own fork / join events
// (created on first use outside graph capture, default priority, kept for the process). The
// 32-row tile launches run on one beside the big-tile launches: the wide kernel holds one
// workgroup per CU and its last round leaves CUs idle, which the 32-row tiles fill.
//
// A call checks a stream out of its device's pool for the whole of its enqueue (fork record,
// wait, launches, join record, wait) and returns it afterwards, so the events a call waits on
// are its own records whatever other host threads do. A stream that another thread's graph
// capture has joined stays part of that capture until the capture ends, so it is only taken by
// calls of the same capture (same capture id) or once the capture is over. With every stream of
// the pool busy or captured (and no new one allowed: the pool is full, or this call is being
// captured) the call runs both tile heights on its own stream.
struct SideStream {
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
  bool busy = false;
};
constexpr int kSidePool = 8;
struct SidePool {
  SideStream slot[kSidePool];
  int used = 0;
  bool failed = false;  // creation failed once: one stream on this device from then on
};
std::mutex g_side_mu;
SidePool g_side[kMaxDevices];

// capture status and id of `s` (status None with id 0 when the query fails)
std::pair<hipStreamCaptureStatus, unsigned long long> capture_of(hipStream_t s) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  unsigned long long id = 0;
  if (hipStreamGetCaptureInfo(s, &cs, &id) != hipSuccess) {
    (void)hipGetLastError();
    return {hipStreamCaptureStatusInvalidated, 0};
  }
  return {cs, id};
}

class SideLease {
 public:
  // enabled = false: no stream is leased (the call runs on its own stream)
  SideLease(hipStream_t stream, bool enabled) {
    if (!enabled) return;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
      (void)hipGetLastError();
      return;
    }
    const auto mine = capture_of(stream);
    if (mine.first == hipStreamCaptureStatusInvalidated) return;
    std::lock_guard<std::mutex> lk(g_side_mu);
    SidePool& p = g_side[dev];
    if (p.failed) return;
    for (int i = 0; i < p.used; ++i) {
      SideStream& ss = p.slot[i];
      if (ss.busy) continue;
      const auto c = capture_of(ss.s);
      const bool free_eager = c.first == hipStreamCaptureStatusNone;
      const bool same_capture = mine.first == hipStreamCaptureStatusActive &&
                                c.first == hipStreamCaptureStatusActive && c.second == mine.second;
      if (free_eager || same_capture) {
        ss.busy = true;
        ss_ = &ss;
        return;
      }
    }
    // a new stream: never under capture (no stream or event creation there)
    if (p.used == kSidePool || mine.first != hipStreamCaptureStatusNone) return;
    SideStream& ss = p.slot[p.used];
    const bool ok = hipStreamCreateWithFlags(&ss.s, hipStreamNonBlocking) == hipSuccess &&
                    hipEventCreateWithFlags(&ss.fork, hipEventDisableTiming) == hipSuccess &&
                    hipEventCreateWithFlags(&ss.join, hipEventDisableTiming) == hipSuccess;
    if (!ok) {
      (void)hipGetLastError();
      p.failed = true;
      return;
    }
    ++p.used;
    ss.busy = true;
    ss_ = &ss;
  }
  ~SideLease() {
    if (!ss_) return;
    std::lock_guard<std::mutex> lk(g_side_mu);
    ss_->busy = false;
  }
  SideLease(const SideLease&) = delete;
  SideLease& operator=(const SideLease&) = delete;
  const SideStream* get() const { return ss_; }

 private:
  SideStream* ss_ = nullptr;
};

// Measurement hook (e4b_set_probe): the watched launch site and the caller's event pair, read
// by every split forward (the atomic keeps the unwatched case to one load).
std::atomic<int> g_probe_site{E4B_PROBE_OFF};
std::mutex g_probe_mu;
hipEvent_t g_probe_ev[2] = {nullptr, nullptr};

struct ProbeEvents {
  hipEvent_t before = nullptr, after = nullptr;
};
ProbeEvents probe_for(int site) {
  if (g_probe_site.load(std::memory_order_relaxed) != site) return {};
  std::lock_guard<std::mutex> lk(g_probe_mu);
  if (g_probe_site.load(std::memory_order_relaxed) != site) return {};
  return {g_probe_ev[0], g_probe_ev[1]};
}

// launch(r, s) between the probe's event records when `site` is watched
template <class F>
int probed(int site, const e4b_routing* r, hipStream_t s, F&& launch) {
  const ProbeEvents pe = probe_for(site);
  if (pe.before && hipEventRecord(pe.before, s) != hipSuccess) return check_launch("probe event");
  const int rc = launch(r, s);
  if (pe.after && hipEventRecord(pe.after, s) != hipSuccess) return check_launch("probe event");
  return rc;
}

// launch(rbig, stream) and launch(rsmall, the side stream), the side stream forked from `stream`
// after everything enqueued so far and joined back into it (both on `stream` without a side
// stream): the two tile heights write disjoint rows. site_big / site_big + 1: the probe sites of
// the two launches.
template <class F>
int run_tile_heights(const SideStream* side, hipStream_t stream, const e4b_routing* rbig, const e4b_routing* rsmall,
                     int site_big, F&& launch) {
  // while a probe is set both heights run on the caller's stream: the probed launch then runs
  // alone, so its time does not depend on whether the two streams share a hardware queue
  if (side && g_probe_site.load(std::memory_order_relaxed) == E4B_PROBE_OFF) {
    if (hipEventRecord(side->fork, stream) != hipSuccess || hipStreamWaitEvent(side->s, side->fork, 0) != hipSuccess)
      return check_launch("side stream fork");
    int r = probed(site_big, rbig, stream, launch);
    if (!r) r = probed(site_big + 1, rsmall, side->s, launch);
    // joined whatever happened, so the caller's stream never runs ahead of the side stream
    const bool joined = hipEventRecord(side->join, side->s) == hipSuccess &&
                        hipStreamWaitEvent(stream, side->join, 0) == hipSuccess;
    if (r) return r;
    return joined ? 0 : check_launch("side stream join");
  }
  int r = probed(site_big, rbig, stream, launch);
  return r ? r : probed(site_big + 1, rsmall, stream, launch);
}

bool act_dtype_ok(int dt) { return dt == E4B_BF16 || dt == E4B_FP16; }
bool any_dtype_ok(int dt) { return dt == E4B_BF16 || dt == E4B_FP16 || dt == E4B_FP32; }

int check_weight(const e4b_qweight* w) {
  if (!w) return fail(E4B_EINVAL, "weight descriptor is NULL");
  if (w->num_experts <= 0 || w->n <= 0 || w->k <= 0)
    return fail(E4B_EINVAL, "weight dims must be positive (E=%d n=%lld k=%lld)", w->num_experts,
                (long long)w->n, (long long)w->k);
  if (w->k % 64) return fail(E4B_EUNSUPPORTED, "k=%lld is not a multiple of 64", (long long)w->k);
  if (!w->packed || !w->absmax) return fail(E4B_EINVAL, "packed/absmax pointer is NULL");
  if (!aligned16(w->packed)) return fail(E4B_EINVAL, "packed weights must be 16-byte aligned");
  switch (w->format) {
    case E4B_FMT_NF4:
      if (!w->code) return fail(E4B_EINVAL, "NF4 needs the 16-entry code table");
      break;
    case E4B_FMT_NF4_DQ:
      if (!w->code || !w->code2 || !w->absmax2 || !w->offset)
        return fail(E4B_EINVAL, "double-quant NF4 needs code, code2, absmax2 and offset");
      break;
    case E4B_FMT_MXFP4:
      break;
    default:
      return fail(E4B_EINVAL, "unknown weight format %d", w->format);
  }
  return E4B_OK;
}

int check_routing(const e4b_routing* rt, int64_t M) {
  if (!rt) return fail(E4B_EINVAL, "routing descriptor is NULL");
  if (!rt->sorted_flat || !rt->inv || !rt->offsets || !rt->active || !rt->tiles || !rt->meta)
    return fail(E4B_EINVAL, "routing buffers must all be non-NULL");
  if (rt->tile_m <= 0) return fail(E4B_EINVAL, "tile_m must be positive");
  if (M > 0 && rt->max_tiles <= 0) return fail(E4B_EINVAL, "max_tiles must be positive");
  return E4B_OK;
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

template <int FMT>
int launch_dequant_fmt(const e4b_qweight& w, int eb, int ec, int od, void* out, hipStream_t s) {
  const int64_t words = int64_t(ec) * w.n * w.k / 8;
  const int grid = static_cast<int>(std::min<int64_t>(cdiv(words, 256), 16384));
  switch (od) {
    case E4B_FP32:
      hipLaunchKernelGGL((e4b::dequant_kernel<FMT, E4B_FP32>), dim3(grid), dim3(256), 0, s, w, eb, words, out);
      break;
    case E4B_BF16:
      hipLaunchKernelGGL((e4b::dequant_kernel<FMT, E4B_BF16>), dim3(grid), dim3(256), 0, s, w, eb, words, out);
      break;
    default:
      hipLaunchKernelGGL((e4b::dequant_kernel<FMT, E4B_FP16>), dim3(grid), dim3(256), 0, s, w, eb, words, out);
      break;
  }
  return check_launch("dequant_kernel");
}

// GEMV lanes per weight row: about four 16-byte chunks per lane.
int gemv_group(int64_t k) {
  const int64_t chunks = k / 32;
  int g = 2;
  while (g < 64 && chunks / (2 * g) >= 4) g *= 2;
  return g;
}

template <int DT, int FMT, int G>
void launch_gemv_g(const e4b::GemmArgs& a, int64_t max_active, hipStream_t s) {
  constexpr int slots = e4b::kWave / G;
  const int64_t cols_per_block = (e4b::kGemvThreads / e4b::kWave) * slots;
  dim3 grid(static_cast<unsigned>(cdiv(a.n_out, cols_per_block)), static_cast<unsigned>(max_active));
  hipLaunchKernelGGL((e4b::gemv_kernel<DT, FMT, G>), grid, dim3(e4b::kGemvThreads), 0, s, a);
}

template <int DT, int FMT>
void launch_gemv_fmt(const e4b::GemmArgs& a, int64_t max_active, hipStream_t s) {
  switch (gemv_group(a.w.k)) {
    case 2: launch_gemv_g<DT, FMT, 2>(a, max_active, s); break;
    case 4: launch_gemv_g<DT, FMT, 4>(a, max_active, s); break;
    case 8: launch_gemv_g<DT, FMT, 8>(a, max_active, s); break;
    case 16: launch_gemv_g<DT, FMT, 16>(a, max_active, s); break;
    case 32: launch_gemv_g<DT, FMT, 32>(a, max_active, s); break;
    default: launch_gemv_g<DT, FMT, 64>(a, max_active, s); break;
  }
}

template <int DT>
int launch_gemm_dt(const e4b::GemmArgs& a, bool gemv, int64_t max_active, hipStream_t s) {
  switch (a.w.format) {
    case E4B_FMT_NF4:
      gemv ? launch_gemv_fmt<DT, E4B_FMT_NF4>(a, max_active, s) : e4b::launch_mfma_gemm<DT, E4B_FMT_NF4>(a, s);
      break;
    case E4B_FMT_NF4_DQ:
      gemv ? launch_gemv_fmt<DT, E4B_FMT_NF4_DQ>(a, max_active, s) : e4b::launch_mfma_gemm<DT, E4B_FMT_NF4_DQ>(a, s);
      break;
    default:
      gemv ? launch_gemv_fmt<DT, E4B_FMT_MXFP4>(a, max_active, s) : e4b::launch_mfma_gemm<DT, E4B_FMT_MXFP4>(a, s);
      break;
  }
  return check_launch(gemv ? "gemv_kernel" : "gemm_mfma_kernel");
}

template <int DDT, int WDT, bool SC>
void launch_combine_w(const void* down, const int32_t* inv, const void* w, int64_t T, int k, int64_t H,
                      void* out, int od, const e4b::CombineScale& cs, hipStream_t s) {
  const int64_t work = T * ((H % 8) == 0 ? H / 8 : H);
  const int grid = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(cdiv(work, 256), 16384)));
  switch (od) {
    case E4B_FP32:
      hipLaunchKernelGGL((e4b::combine_kernel<DDT, WDT, E4B_FP32, SC>), dim3(grid), dim3(256), 0, s, down, inv, w, T, k,
                         H, out, cs);
      break;
    case E4B_BF16:
      hipLaunchKernelGGL((e4b::combine_kernel<DDT, WDT, E4B_BF16, SC>), dim3(grid), dim3(256), 0, s, down, inv, w, T, k,
                         H, out, cs);
      break;
    default:
      hipLaunchKernelGGL((e4b::combine_kernel<DDT, WDT, E4B_FP16, SC>), dim3(grid), dim3(256), 0, s, down, inv, w, T, k,
                         H, out, cs);
      break;
  }
}

template <int DDT, bool SC = false>
void launch_combine_dt(const void* down, const int32_t* inv, const void* w, int wd, int64_t T, int k, int64_t H,
                       void* out, int od, hipStream_t s, const e4b::CombineScale& cs = {}) {
  switch (wd) {
    case E4B_FP32: launch_combine_w<DDT, E4B_FP32, SC>(down, inv, w, T, k, H, out, od, cs, s); break;
    case E4B_BF16: launch_combine_w<DDT, E4B_BF16, SC>(down, inv, w, T, k, H, out, od, cs, s); break;
    default: launch_combine_w<DDT, E4B_FP16, SC>(down, inv, w, T, k, H, out, od, cs, s); break;
  }
}

// Decode path: shapes come from decode_launch.h; the launchers live in decode_inst.hip.
template <bool UP>
void launch_decode(const e4b::DecodeArgs& a, int act_dtype, int64_t max_active, int64_t M, hipStream_t s) {
  const e4b::DecShape d = UP ? e4b::decode_up_shape(a.w.k) : e4b::decode_down_shape(a.w.k, M);
#define E4B_DEC(DT, FMT)                                         \
  if (act_dtype == DT && a.w.format == FMT) {                    \
    if (UP) e4b::launch_decode_up<DT, FMT>(a, d, max_active, s); \
    else e4b::launch_decode_down<DT, FMT>(a, d, s);              \
    return;                                                      \
  }
  E4B_DEC(E4B_BF16, E4B_FMT_NF4) E4B_DEC(E4B_BF16, E4B_FMT_NF4_DQ) E4B_DEC(E4B_BF16, E4B_FMT_MXFP4)
  E4B_DEC(E4B_FP16, E4B_FMT_NF4) E4B_DEC(E4B_FP16, E4B_FMT_NF4_DQ) E4B_DEC(E4B_FP16, E4B_FMT_MXFP4)
#undef E4B_DEC
}

bool decode_supported(int64_t M, int E, const e4b_qweight* w, bool up) {
  const e4b::DecShape d = up ? e4b::decode_up_shape(w->k) : e4b::decode_down_shape(w->k, M);
  return M <= e4b::kDecMaxRows && E <= e4b::kDecMaxExperts && d.G > 0;
}

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

int64_t max_tiles_for(int64_t M, int E, int tile_m) { return cdiv(M, tile_m) + std::min<int64_t>(E, M); }

// MFMA tile rows for a forward of M routed rows over E experts: 128-row tiles once experts
// average 64 rows or more, else 32-row tiles (less padding when experts get few rows each).
int mfma_tile_for(int64_t M, int E) {
  const int64_t groups = std::min<int64_t>(E, M);
  return M >= 64 * groups ? e4b::kTileM : e4b::kTileMSmall;
}

// Prefill re-tiling (emit_split_tiles, in the routing's table step): 256-row tiles in the fp16 matrix-core mode (the wide
// kernel), 128-row tiles otherwise, except that an expert whose last tile would hold at most 32
// rows runs those rows in one 32-row tile. The workspace holds the longer (128-row) tile list.
int64_t max_big_tiles(int64_t M, int E) { return max_tiles_for(M, E, e4b::kTileM); }
int64_t max_small_tiles(int64_t M, int E) { return std::max<int64_t>(1, std::min<int64_t>(E, M)); }

bool is_gated_epi(int epi) {
  return epi == E4B_EPI_SWIGLU || epi == E4B_EPI_CLAMP_SWIGLU || epi == E4B_EPI_GPTOSS;
}

// The fused forward's token rows in the fp16 matrix-core mode (row_exp_row over x), computed in
// the routing's first launch by route_impl.
struct RowExpArgs {
  const uint16_t* x;  // [tokens, k] bf16
  int64_t k;
  int32_t* row_exp;   // [tokens]
  uint16_t* x16;      // [tokens, k] scaled fp16
};
int route_impl(const int64_t* top_k_index, int64_t tokens, int32_t top_k, int32_t num_experts, const e4b_routing* rt,
               const RowExpArgs* rx, hipStream_t stream, const e4b::SplitTiles& sp = {});

}  // namespace

extern "C" {

const char* e4b_version(void) { return "e4b_amd 0.1.0 (gfx950)"; }

const char* e4b_last_error(void) { return g_last_error.c_str(); }

int32_t e4b_mfma_tile_m(void) { return e4b::kTileM; }

int e4b_dequant(const e4b_qweight* w, int32_t expert_begin, int32_t expert_count, int32_t out_dtype, void* out,
                hipStream_t stream) {
  int rc = check_weight(w);
  if (rc) return rc;
  if (!out) return fail(E4B_EINVAL, "out is NULL");
  if (!any_dtype_ok(out_dtype)) return fail(E4B_EINVAL, "bad out_dtype %d", out_dtype);
  if (expert_begin < 0 || expert_count < 0 || expert_begin + expert_count > w->num_experts)
    return fail(E4B_EINVAL, "expert range [%d, %d) outside [0, %d)", expert_begin, expert_begin + expert_count,
                w->num_experts);
  if (!aligned16(out)) return fail(E4B_EINVAL, "out must be 16-byte aligned");
  if (expert_count == 0) return E4B_OK;
  switch (w->format) {
    case E4B_FMT_NF4: return launch_dequant_fmt<E4B_FMT_NF4>(*w, expert_begin, expert_count, out_dtype, out, stream);
    case E4B_FMT_NF4_DQ:
      return launch_dequant_fmt<E4B_FMT_NF4_DQ>(*w, expert_begin, expert_count, out_dtype, out, stream);
    default: return launch_dequant_fmt<E4B_FMT_MXFP4>(*w, expert_begin, expert_count, out_dtype, out, stream);
  }
}

int e4b_route(const int64_t* top_k_index, int64_t tokens, int32_t top_k, int32_t num_experts, const e4b_routing* rt,
              hipStream_t stream) {
  return route_impl(top_k_index, tokens, top_k, num_experts, rt, nullptr, stream);
}

}  // extern "C"

namespace {

// e4b_route, and with rx the fused forward's token rows (row_exp_row over x [tokens, k]) in the
// routing's first launch; with sp.on the prefill's two tile lists (sp.big, sp.small) from the
// routing's table step.
int route_impl(const int64_t* top_k_index, int64_t tokens, int32_t top_k, int32_t num_experts, const e4b_routing* rt,
               const RowExpArgs* rx, hipStream_t stream, const e4b::SplitTiles& sp) {
  if (tokens < 0 || top_k <= 0) return fail(E4B_EINVAL, "tokens must be >= 0 and top_k > 0");
  const int64_t M = tokens * top_k;
  if (M > 0x7fffffffLL) return fail(E4B_EUNSUPPORTED, "tokens*top_k=%lld exceeds int32", (long long)M);
  if (num_experts <= 0 || num_experts > e4b::kRouteMaxExperts)
    return fail(E4B_EUNSUPPORTED, "num_experts=%d outside [1, %d]", num_experts, e4b::kRouteMaxExperts);
  int rc = check_routing(rt, M);
  if (rc) return rc;
  if (M > 0 && !top_k_index) return fail(E4B_EINVAL, "top_k_index is NULL");
  if (M > 0 && rt->max_tiles < max_tiles_for(M, num_experts, rt->tile_m))
    return fail(E4B_ESPACE, "max_tiles=%d < %lld needed", rt->max_tiles,
                (long long)max_tiles_for(M, num_experts, rt->tile_m));
  const int rp = rx ? e4b::row_exp_pieces(rx->k) : 0;
  if (M <= e4b::kRouteSingleMaxRows) {
    if (!rx) {
      hipLaunchKernelGGL(e4b::route_kernel, dim3(1), dim3(e4b::kRouteThreads), 0, stream, top_k_index, M, num_experts,
                         *rt, sp);
      return check_launch("route_kernel");
    }
    const dim3 grid(static_cast<unsigned>(1 + cdiv(tokens, e4b::kRouteWaves)));
#define E4B_RRX(RP)                                                                                                  \
  hipLaunchKernelGGL(e4b::route_rowexp_kernel<RP>, grid, dim3(e4b::kRouteThreads), 0, stream, top_k_index, M,        \
                     num_experts, *rt, sp, rx->x, tokens, rx->k, rx->row_exp, rx->x16)
    if (rp == 1) E4B_RRX(1); else if (rp == 2) E4B_RRX(2); else if (rp == 4) E4B_RRX(4); else E4B_RRX(8);
#undef E4B_RRX
    return check_launch("route_rowexp_kernel");
  }
  if (!rt->scratch) return fail(E4B_EINVAL, "routing scratch is NULL (needed above %d rows)", e4b::kRouteSingleMaxRows);
  const int64_t nchunks = cdiv(M, e4b::kRouteChunk);
  if (!rx) {
    hipLaunchKernelGGL(e4b::route_count_kernel, dim3(static_cast<unsigned>(nchunks)), dim3(e4b::kRouteChunk), 0,
                       stream, top_k_index, M, num_experts, rt->scratch);
  } else {
    const dim3 grid(static_cast<unsigned>(nchunks + cdiv(tokens, e4b::kChunkWaves)));
#define E4B_RCX(RP)                                                                                                  \
  hipLaunchKernelGGL(e4b::route_count_rowexp_kernel<RP>, grid, dim3(e4b::kRouteChunk), 0, stream, top_k_index, M,    \
                     num_experts, rt->scratch, nchunks, rx->x, tokens, rx->k, rx->row_exp, rx->x16)
    if (rp == 1) E4B_RCX(1); else if (rp == 2) E4B_RCX(2); else if (rp == 4) E4B_RCX(4); else E4B_RCX(8);
#undef E4B_RCX
  }
  hipLaunchKernelGGL(e4b::route_colscan_kernel, dim3(static_cast<unsigned>(num_experts + 1)),
                     dim3(e4b::kRouteThreads), 0, stream, nchunks, num_experts, rt->scratch, rt->offsets);
  hipLaunchKernelGGL(e4b::route_tables_kernel, dim3(1), dim3(e4b::kRouteThreads), 0, stream, num_experts, *rt, sp);
  hipLaunchKernelGGL(e4b::route_place_kernel, dim3(static_cast<unsigned>(nchunks)), dim3(e4b::kRouteChunk), 0, stream,
                     top_k_index, M, num_experts, rt->scratch, *rt);
  return check_launch("route_count/colscan/tables/place kernels");
}

}  // namespace

extern "C" {

int e4b_route_groups(const int64_t* sizes, int32_t groups, const int64_t* expert_ids, int32_t num_experts,
                     const e4b_routing* rt, hipStream_t stream) {
  if (groups < 0 || groups > e4b::kGroupsMax)
    return fail(E4B_EUNSUPPORTED, "groups=%d outside [0, %d]", groups, e4b::kGroupsMax);
  if (num_experts <= 0 || num_experts > e4b::kRouteMaxExperts)
    return fail(E4B_EUNSUPPORTED, "num_experts=%d outside [1, %d]", num_experts, e4b::kRouteMaxExperts);
  if (groups > 0 && (!sizes || !expert_ids)) return fail(E4B_EINVAL, "NULL pointer");
  e4b::GroupOffsets go{};
  int64_t M = 0;
  for (int g = 0; g < groups; ++g) {
    if (sizes[g] < 0) return fail(E4B_EINVAL, "group %d has a negative size", g);
    go.off[g] = static_cast<int32_t>(M);
    M += sizes[g];
    if (M > 0x7fffffffLL) return fail(E4B_EUNSUPPORTED, "groups hold more than 2^31 - 1 rows");
  }
  go.off[groups] = static_cast<int32_t>(M);
  int rc = check_routing(rt, M);
  if (rc) return rc;
  // every expert's rows are whole tiles but its last: at most ceil(M / tile_m) + min(E, groups)
  const int64_t need = cdiv(M, rt->tile_m) + std::min<int64_t>(num_experts, groups);
  if (M > 0 && rt->max_tiles < need)
    return fail(E4B_ESPACE, "max_tiles=%d < %lld needed", rt->max_tiles, (long long)need);
  hipLaunchKernelGGL(e4b::route_groups_kernel, dim3(1), dim3(e4b::kRouteThreads), 0, stream, go, groups, expert_ids,
                     num_experts, *rt);
  return check_launch("route_groups_kernel");
}

int e4b_gather_rows(void* dst, int64_t row_bytes, int64_t dst_off, const int64_t* src_addr, const int64_t* ident,
                    const int64_t* have, int32_t slots, int64_t n_bytes, unsigned long long* bytes_copied,
                    hipStream_t stream) {
  if (slots < 0 || n_bytes < 0 || row_bytes < 0 || dst_off < 0) return fail(E4B_EINVAL, "negative sizes");
  if (slots == 0 || n_bytes == 0) return E4B_OK;
  if (!dst || !src_addr || !ident || !have) return fail(E4B_EINVAL, "NULL pointer");
  if (dst_off + n_bytes > row_bytes)
    return fail(E4B_EINVAL, "segment [%lld, %lld) runs past the %lld-byte slot row", (long long)dst_off,
                (long long)(dst_off + n_bytes), (long long)row_bytes);
  if (slots > 65535) return fail(E4B_EUNSUPPORTED, "slots=%d > 65535", slots);
  const dim3 grid(static_cast<unsigned>(cdiv(n_bytes, e4b::kGatherChunk)), static_cast<unsigned>(slots));
  hipLaunchKernelGGL(e4b::gather_rows_kernel, grid, dim3(e4b::kGatherThreads), 0, stream, static_cast<uint8_t*>(dst),
                     row_bytes, dst_off, src_addr, ident, have, n_bytes, bytes_copied);
  return check_launch("gather_rows_kernel");
}

int64_t e4b_route_scratch_ints(int64_t M, int32_t num_experts) {
  if (M <= e4b::kRouteSingleMaxRows || num_experts <= 0) return 0;
  return cdiv(M, e4b::kRouteChunk) * (int64_t(num_experts) + 1);
}

// e4b_grouped_gemm, plus the fp16 matrix-core mode of the fused forward: a_exp (the A rows'
// largest exponents, the rows stored as scaled fp16 by row_exp_kernel) selects it on the MFMA
// path.
// The LoRA delta a grouped GEMM adds in its epilogue: lscale * t[m, :] . B[e, row, :] (t fp32 [M, rank]
// of the routed rows, B [E, n, rank] in dtype).
struct LoraEpi {
  const float* t;
  const void* b;
  int dtype, rank;
  float scaling;
};

static int grouped_gemm_impl(const void* a, int32_t act_dtype, int32_t gather_k, const e4b_qweight* w,
                             const e4b_routing* rt, int64_t tokens, int64_t M, int32_t epilogue, float alpha,
                             float limit, int32_t flags, void* out, int32_t out_dtype, const int32_t* a_exp,
                             hipStream_t stream, const LoraEpi* lora = nullptr, int out_f16_shift = 0) {
  int rc = check_weight(w);
  if (rc) return rc;
  rc = check_routing(rt, M);
  if (rc) return rc;
  if (!act_dtype_ok(act_dtype)) return fail(E4B_EINVAL, "act_dtype must be bf16 or fp16 (got %d)", act_dtype);
  if (out_dtype != act_dtype && out_dtype != E4B_FP32)
    return fail(E4B_EINVAL, "out_dtype must be the activation dtype or fp32 (got %d)", out_dtype);
  if (epilogue < E4B_EPI_NONE || epilogue > E4B_EPI_GPTOSS) return fail(E4B_EINVAL, "bad epilogue %d", epilogue);
  const bool pair = is_gated_epi(epilogue);
  if (pair && (w->n % 2)) return fail(E4B_EINVAL, "gated epilogue needs an even n (got %lld)", (long long)w->n);
  if (epilogue == E4B_EPI_GPTOSS && !w->bias) return fail(E4B_EINVAL, "gpt-oss epilogue needs the gate_up bias");
  if (M < 0 || tokens < 0) return fail(E4B_EINVAL, "negative sizes");
  if (M == 0) return E4B_OK;
  if (!a || !out) return fail(E4B_EINVAL, "a/out is NULL");
  if (!aligned16(a)) return fail(E4B_EINVAL, "activations must be 16-byte aligned");
  if (gather_k < 0) return fail(E4B_EINVAL, "gather_k must be >= 0");
  bool gemv;
  if (flags == E4B_PATH_GEMV) gemv = true;
  else if (flags == E4B_PATH_MFMA) gemv = false;
  else if (flags == E4B_PATH_AUTO) gemv = tokens <= 4;
  else return fail(E4B_EINVAL, "bad flags %d", flags);
  if (!gemv && rt->tile_m != e4b::kTileM && rt->tile_m != e4b::kTileMSmall && rt->tile_m != e4b::kTileMBig)
    return fail(E4B_EINVAL, "routing tile_m=%d but the MFMA GEMM takes %d, %d or %d", rt->tile_m, e4b::kTileMBig,
                e4b::kTileM, e4b::kTileMSmall);

  e4b::GemmArgs args;
  args.a = static_cast<const uint16_t*>(a);
  args.gather_k = gather_k;
  args.w = *w;
  args.rt = *rt;
  args.M = M;
  args.epi = epilogue;
  args.alpha = alpha;
  args.limit = limit;
  args.out = out;
  args.n_out = pair ? w->n / 2 : w->n;
  args.out_f32 = out_dtype == E4B_FP32;
  const bool f16c = a_exp != nullptr;
  if (f16c && (gemv || act_dtype != E4B_BF16 || w->format == E4B_FMT_MXFP4 || !w->shift))
    return fail(E4B_EINVAL, "the fp16 matrix-core mode needs the MFMA path, bf16 activations and NF4 weight shifts");
  args.a_exp = a_exp;
  if (out_f16_shift && (!f16c || out_dtype != E4B_FP32 || epilogue != E4B_EPI_NONE || w->bias || lora ||
                        !e4b::lora_gemm_fits(rt->tile_m, w->k)))
    return fail(E4B_EINVAL, "fp16 down rows need the fp16 mode over 256-row tiles or 32-row tiles with k %% 256 == "
                            "0, fp32 rows, and no epilogue, bias or LoRA");
  args.out_f16_shift = out_f16_shift;
  args.lt = nullptr;
  args.lb = nullptr;
  args.lbdt = E4B_FP32;
  args.lr = 0;
  args.lscale = 0.0f;
  if (lora) {
    if (!f16c || !e4b::lora_gemm_fits(rt->tile_m, w->k))
      return fail(E4B_EINVAL, "the LoRA epilogue needs the fp16 mode over 256-row tiles or 32-row tiles with k %% 256 == 0");
    args.lt = lora->t;
    args.lb = lora->b;
    args.lbdt = lora->dtype;
    args.lr = lora->rank;
    args.lscale = lora->scaling;
  }
  const int64_t max_active = std::min<int64_t>(w->num_experts, M);
  return act_dtype == E4B_BF16 ? launch_gemm_dt<E4B_BF16>(args, gemv, max_active, stream)
                               : launch_gemm_dt<E4B_FP16>(args, gemv, max_active, stream);
}

int e4b_grouped_gemm(const void* a, int32_t act_dtype, int32_t gather_k, const e4b_qweight* w, const e4b_routing* rt,
                     int64_t tokens, int64_t M, int32_t epilogue, float alpha, float limit, int32_t flags, void* out,
                     int32_t out_dtype, hipStream_t stream) {
  return grouped_gemm_impl(a, act_dtype, gather_k, w, rt, tokens, M, epilogue, alpha, limit, flags, out, out_dtype,
                           nullptr, stream);
}

int e4b_weight_shift(const e4b_qweight* w, int32_t* shift, hipStream_t stream) {
  int rc = check_weight(w);
  if (rc) return rc;
  if (w->format == E4B_FMT_MXFP4) return fail(E4B_EUNSUPPORTED, "MXFP4 weights need no shift (exact in bf16)");
  if (!shift) return fail(E4B_EINVAL, "shift is NULL");
  const int E = w->num_experts;
  if (E > 65535) return fail(E4B_EUNSUPPORTED, "num_experts=%d above 65535 (one grid row per expert)", E);
  hipLaunchKernelGGL(e4b::weight_shift_init_kernel, dim3((E + e4b::kScaleThreads - 1) / e4b::kScaleThreads),
                     dim3(e4b::kScaleThreads), 0, stream, shift, E);
  rc = check_launch("weight_shift_init_kernel");
  if (rc) return rc;
  const int64_t nb = w->n * (w->k / 64);
  const dim3 grid(static_cast<unsigned>((nb + e4b::kShiftSpan - 1) / e4b::kShiftSpan), static_cast<unsigned>(E));
  if (w->format == E4B_FMT_NF4)
    hipLaunchKernelGGL((e4b::weight_shift_kernel<E4B_FMT_NF4>), grid, dim3(e4b::kScaleThreads), 0, stream, *w, shift);
  else
    hipLaunchKernelGGL((e4b::weight_shift_kernel<E4B_FMT_NF4_DQ>), grid, dim3(e4b::kScaleThreads), 0, stream, *w,
                       shift);
  return check_launch("weight_shift_kernel");
}

namespace {

// Validation of the shared LoRA arguments (the B side's too when lora_b / out_features are
// given: out_features >= 0), then, for M > 0, t = x . A^T for every routed row.
int lora_a_pass(const void* x, int32_t x_dtype, int32_t gather_k, const e4b_routing* rt, int64_t M,
                int32_t num_experts, const void* lora_a, const void* lora_b, int32_t adapter_dtype, int32_t rank,
                int64_t in_features, int64_t out_features, int32_t delta_dtype, float* t_workspace,
                const void* out, hipStream_t stream) {
  const bool b_side = out_features >= 0;
  if (!act_dtype_ok(x_dtype)) return fail(E4B_EINVAL, "x_dtype must be bf16 or fp16 (got %d)", x_dtype);
  if (!any_dtype_ok(adapter_dtype) || !any_dtype_ok(delta_dtype)) return fail(E4B_EINVAL, "bad adapter/delta dtype");
  if (M < 0 || M > 0x7fffffffLL) return fail(E4B_EINVAL, "bad row count %lld", (long long)M);
  if (num_experts <= 0 || num_experts > 1024) return fail(E4B_EUNSUPPORTED, "num_experts=%d outside [1, 1024]", num_experts);
  if (rank <= 0 || rank > e4b::kLoraMaxRank) return fail(E4B_EUNSUPPORTED, "rank=%d outside [1, %d]", rank, e4b::kLoraMaxRank);
  if (in_features <= 0 || in_features % 8 != 0 || (b_side && out_features <= 0))
    return fail(E4B_EINVAL, "in_features (%lld) must be a positive multiple of 8, out_features (%lld) positive",
                (long long)in_features, (long long)out_features);
  if (gather_k < 0) return fail(E4B_EINVAL, "gather_k must be >= 0");
  if (!rt || !rt->offsets || (gather_k > 0 && !rt->sorted_flat)) return fail(E4B_EINVAL, "routing offsets / order are NULL");
  if (M == 0) return E4B_OK;
  if (!x || !lora_a || !t_workspace || (b_side && (!lora_b || !out))) return fail(E4B_EINVAL, "NULL pointer");
  if (!aligned16(x) || !aligned16(lora_a)) return fail(E4B_EINVAL, "x and lora_a must be 16-byte aligned");
  // lora_a: 8-row tiles once there are enough rows to fill the chip with them, else 1-row tiles.
  const int rgroups = static_cast<int>(cdiv(rank, e4b::kLoraRanksPerBlock));
  const bool big = M > 2048;
  const dim3 ga(static_cast<unsigned>(cdiv(M, big ? 8 : 1) * rgroups));
#define E4B_LA(XD, AD)                                                                                         \
  if (x_dtype == XD && adapter_dtype == AD) {                                                                  \
    if (big)                                                                                                   \
      hipLaunchKernelGGL((e4b::lora_a_kernel<XD, AD, 8>), ga, dim3(e4b::kLoraThreads), 0, stream,              \
                         static_cast<const uint16_t*>(x), gather_k, rt->sorted_flat, rt->offsets, num_experts, \
                         lora_a, rank, in_features, t_workspace, M, rgroups);                                  \
    else                                                                                                       \
      hipLaunchKernelGGL((e4b::lora_a_kernel<XD, AD, 1>), ga, dim3(e4b::kLoraThreads), 0, stream,              \
                         static_cast<const uint16_t*>(x), gather_k, rt->sorted_flat, rt->offsets, num_experts, \
                         lora_a, rank, in_features, t_workspace, M, rgroups);                                  \
  }
  E4B_LA(E4B_BF16, E4B_BF16) E4B_LA(E4B_BF16, E4B_FP16) E4B_LA(E4B_BF16, E4B_FP32)
  E4B_LA(E4B_FP16, E4B_BF16) E4B_LA(E4B_FP16, E4B_FP16) E4B_LA(E4B_FP16, E4B_FP32)
#undef E4B_LA
  return check_launch("lora_a_kernel");
}

int lora_tile_rows(int64_t M) { return M <= 512 ? 1 : (M <= 8192 ? 8 : e4b::kLoraMaxTileRows); }

// out[m, :] += delta_dtype(scaling * t[m, :] . B[e_m, :, :]^T) for the routed rows (M > 0, the
// arguments validated).
int lora_b_pass(const float* t_workspace, const e4b_routing* rt, int64_t M, int32_t num_experts, const void* lora_b,
                int32_t adapter_dtype, int32_t rank, int64_t out_features, float scaling, int32_t delta_dtype,
                float* out, hipStream_t stream) {
  // lora_b_add: row tiles sized so that small batches still spread over many blocks.
  const int64_t ncb = cdiv(out_features, e4b::kLoraThreads);
  const int tile_rows = lora_tile_rows(M);
  if (cdiv(M, tile_rows) * ncb > 0x7fffffffLL) return fail(E4B_EUNSUPPORTED, "LoRA delta grid too large");
  const dim3 gb(static_cast<unsigned>(cdiv(M, tile_rows) * ncb));
#define E4B_LB(AD, OD)                                                                                          \
  if (adapter_dtype == AD && delta_dtype == OD) {                                                               \
    if (rank <= 16)                                                                                             \
      hipLaunchKernelGGL((e4b::lora_b_add_kernel<AD, OD, 16>), gb, dim3(e4b::kLoraThreads), 0, stream,          \
                         t_workspace, rt->offsets, num_experts, lora_b, rank, out_features, scaling, out, M,   \
                         tile_rows, ncb);                                                                       \
    else if (rank <= 32)                                                                                        \
      hipLaunchKernelGGL((e4b::lora_b_add_kernel<AD, OD, 32>), gb, dim3(e4b::kLoraThreads), 0, stream,          \
                         t_workspace, rt->offsets, num_experts, lora_b, rank, out_features, scaling, out, M,   \
                         tile_rows, ncb);                                                                       \
    else                                                                                                        \
      hipLaunchKernelGGL((e4b::lora_b_add_kernel<AD, OD, e4b::kLoraMaxRank>), gb, dim3(e4b::kLoraThreads), 0,   \
                         stream, t_workspace, rt->offsets, num_experts, lora_b, rank, out_features, scaling,   \
                         out, M, tile_rows, ncb);                                                               \
  }
  E4B_LB(E4B_BF16, E4B_BF16) E4B_LB(E4B_BF16, E4B_FP16) E4B_LB(E4B_BF16, E4B_FP32)
  E4B_LB(E4B_FP16, E4B_BF16) E4B_LB(E4B_FP16, E4B_FP16) E4B_LB(E4B_FP16, E4B_FP32)
  E4B_LB(E4B_FP32, E4B_BF16) E4B_LB(E4B_FP32, E4B_FP16) E4B_LB(E4B_FP32, E4B_FP32)
#undef E4B_LB
  return check_launch("lora kernels");
}

}  // namespace

int e4b_lora_delta(const void* x, int32_t x_dtype, int32_t gather_k, const e4b_routing* rt, int64_t M,
                   int32_t num_experts, const void* lora_a, const void* lora_b, int32_t adapter_dtype,
                   int32_t rank, int64_t in_features, int64_t out_features, float scaling,
                   int32_t delta_dtype, float* t_workspace, float* out, hipStream_t stream) {
  const int st = lora_a_pass(x, x_dtype, gather_k, rt, M, num_experts, lora_a, lora_b, adapter_dtype, rank,
                             in_features, out_features, delta_dtype, t_workspace, out, stream);
  if (st != E4B_OK || M == 0) return st;
  return lora_b_pass(t_workspace, rt, M, num_experts, lora_b, adapter_dtype, rank, out_features, scaling, delta_dtype,
                     out, stream);
}

int e4b_lora_t(const void* x, int32_t x_dtype, int32_t gather_k, const e4b_routing* rt, int64_t M,
               int32_t num_experts, const void* lora_a, int32_t adapter_dtype, int32_t rank, int64_t in_features,
               float* t, hipStream_t stream) {
  return lora_a_pass(x, x_dtype, gather_k, rt, M, num_experts, lora_a, nullptr, adapter_dtype, rank, in_features, -1,
                     E4B_FP32, t, nullptr, stream);
}

int e4b_lora_t_add(const float* t, const e4b_routing* rt, int64_t M, int32_t num_experts, const void* lora_b,
                   int32_t adapter_dtype, int32_t rank, int64_t out_features, float scaling, int32_t delta_dtype,
                   float* out, hipStream_t stream) {
  if (!any_dtype_ok(adapter_dtype) || !any_dtype_ok(delta_dtype)) return fail(E4B_EINVAL, "bad adapter/delta dtype");
  if (M < 0 || M > 0x7fffffffLL) return fail(E4B_EINVAL, "bad row count %lld", (long long)M);
  if (num_experts <= 0 || num_experts > 1024) return fail(E4B_EUNSUPPORTED, "num_experts=%d outside [1, 1024]", num_experts);
  if (rank <= 0 || rank > e4b::kLoraMaxRank) return fail(E4B_EUNSUPPORTED, "rank=%d outside [1, %d]", rank, e4b::kLoraMaxRank);
  if (out_features <= 0) return fail(E4B_EINVAL, "out_features must be positive");
  if (!rt || !rt->offsets) return fail(E4B_EINVAL, "routing offsets are NULL");
  if (M == 0) return E4B_OK;
  if (!t || !lora_b || !out) return fail(E4B_EINVAL, "NULL pointer");
  return lora_b_pass(t, rt, M, num_experts, lora_b, adapter_dtype, rank, out_features, scaling, delta_dtype, out,
                     stream);
}

int e4b_lora_wgrad(const float* u, int32_t rank, const void* a, int32_t a_dtype, int32_t gather_k,
                   const e4b_routing* rt, int64_t M, int32_t num_experts, int64_t cols, float scale, float* out,
                   hipStream_t stream) {
  if (!act_dtype_ok(a_dtype)) return fail(E4B_EINVAL, "a_dtype must be bf16 or fp16 (got %d)", a_dtype);
  if (M < 0 || M > 0x7fffffffLL) return fail(E4B_EINVAL, "bad row count %lld", (long long)M);
  if (num_experts <= 0 || num_experts > 65535) return fail(E4B_EUNSUPPORTED, "num_experts=%d outside [1, 65535]", num_experts);
  if (rank <= 0 || rank > e4b::kLoraMaxRank) return fail(E4B_EUNSUPPORTED, "rank=%d outside [1, %d]", rank, e4b::kLoraMaxRank);
  if (cols <= 0) return fail(E4B_EINVAL, "cols must be positive");
  if (gather_k < 0) return fail(E4B_EINVAL, "gather_k must be >= 0");
  if (!rt || !rt->offsets || (gather_k > 0 && !rt->sorted_flat)) return fail(E4B_EINVAL, "routing offsets / order are NULL");
  if (!out || (M > 0 && (!u || !a))) return fail(E4B_EINVAL, "NULL pointer");
  if (cdiv(cols, e4b::kWgradThreads) > 0x7fffffffLL) return fail(E4B_EUNSUPPORTED, "too many columns");
  // every expert's block writes its rows of out (zeros for an expert without rows)
  const dim3 grid(static_cast<unsigned>(cdiv(cols, e4b::kWgradThreads)), static_cast<unsigned>(num_experts));
#define E4B_WG(XD, RB)                                                                                            \
  hipLaunchKernelGGL((e4b::lora_wgrad_kernel<XD, RB>), grid, dim3(e4b::kWgradThreads), 0, stream, u, rank,       \
                     static_cast<const uint16_t*>(a), gather_k, rt->sorted_flat, rt->offsets, cols, scale, out)
#define E4B_WG_R(XD)                                     \
  if (rank <= 16) E4B_WG(XD, 16);                        \
  else if (rank <= 32) E4B_WG(XD, 32);                   \
  else E4B_WG(XD, e4b::kLoraMaxRank);
  if (a_dtype == E4B_BF16) { E4B_WG_R(E4B_BF16) }
  else { E4B_WG_R(E4B_FP16) }
#undef E4B_WG_R
#undef E4B_WG
  return check_launch("lora_wgrad_kernel");
}

int e4b_grouped_dgrad(const void* grad, int32_t grad_dtype, const e4b_qweight* w, const e4b_routing* rt, int64_t M,
                      float* out, hipStream_t stream) {
  int rc = check_weight(w);
  if (rc) return rc;
  rc = check_routing(rt, M);
  if (rc) return rc;
  if (!act_dtype_ok(grad_dtype)) return fail(E4B_EINVAL, "grad_dtype must be bf16 or fp16 (got %d)", grad_dtype);
  if (w->format == E4B_FMT_MXFP4) return fail(E4B_EUNSUPPORTED, "the grouped dgrad takes NF4 / NF4_DQ weights");
  if (w->n % 64 != 0) return fail(E4B_EUNSUPPORTED, "the grouped dgrad needs n (%lld) divisible by 64", (long long)w->n);
  if (rt->tile_m != e4b::kTileM && rt->tile_m != e4b::kTileMSmall)
    return fail(E4B_EINVAL, "routing tile_m=%d but the dgrad takes %d or %d", rt->tile_m, e4b::kTileM,
                e4b::kTileMSmall);
  if (M < 0) return fail(E4B_EINVAL, "negative row count");
  if (M == 0) return E4B_OK;
  if (!grad || !out) return fail(E4B_EINVAL, "NULL pointer");
  if (!aligned16(grad)) return fail(E4B_EINVAL, "grad must be 16-byte aligned");
  e4b::DgradArgs a;
  a.g = static_cast<const uint16_t*>(grad);
  a.w = *w;
  a.rt = *rt;
  a.out = out;
  const int bm = rt->tile_m;
  const int64_t grid = e4b::kXcds * cdiv(rt->max_tiles, e4b::kXcds) * cdiv(w->k, e4b::dgrad_cols(bm));
  if (grid > 0x7fffffffLL) return fail(E4B_EUNSUPPORTED, "dgrad grid too large");
#define E4B_DG(DT, FMT, BM)                                                                                       \
  hipLaunchKernelGGL((e4b::dgrad_mfma_kernel<DT, FMT, BM>), dim3(static_cast<unsigned>(grid)),                   \
                     dim3(e4b::dgrad_threads(BM)), 0, stream, a)
#define E4B_DG_BM(DT, FMT)                                  \
  if (bm == e4b::kTileM) E4B_DG(DT, FMT, e4b::kTileM);      \
  else E4B_DG(DT, FMT, e4b::kTileMSmall);
  if (grad_dtype == E4B_BF16 && w->format == E4B_FMT_NF4) { E4B_DG_BM(E4B_BF16, E4B_FMT_NF4) }
  else if (grad_dtype == E4B_BF16) { E4B_DG_BM(E4B_BF16, E4B_FMT_NF4_DQ) }
  else if (w->format == E4B_FMT_NF4) { E4B_DG_BM(E4B_FP16, E4B_FMT_NF4) }
  else { E4B_DG_BM(E4B_FP16, E4B_FMT_NF4_DQ) }
#undef E4B_DG_BM
#undef E4B_DG
  return check_launch("dgrad_mfma_kernel");
}

int e4b_lora_delta_epilogue(const void* x, int32_t x_dtype, int32_t gather_k, const e4b_routing* rt, int64_t M,
                            int32_t num_experts, const void* lora_a, const void* lora_b, int32_t adapter_dtype,
                            int32_t rank, int64_t in_features, int64_t out_features, float scaling,
                            int32_t delta_dtype, float* t_workspace, const float* proj, int32_t epilogue,
                            float limit, void* h, int32_t h_dtype, hipStream_t stream) {
  if (!act_dtype_ok(h_dtype)) return fail(E4B_EINVAL, "h_dtype must be bf16 or fp16 (got %d)", h_dtype);
  if (delta_dtype != h_dtype && delta_dtype != E4B_FP32)
    return fail(E4B_EINVAL, "delta_dtype must be h_dtype or fp32 (got %d)", delta_dtype);
  const bool gated_epi = epilogue == E4B_EPI_SWIGLU || epilogue == E4B_EPI_CLAMP_SWIGLU;
  if (!gated_epi && epilogue != E4B_EPI_ACT)
    return fail(E4B_EUNSUPPORTED, "epilogue %d: only SWIGLU, CLAMP_SWIGLU and ACT", epilogue);
  if (gated_epi && out_features % 2 != 0) return fail(E4B_EINVAL, "gated epilogue needs an even out_features");
  const int st = lora_a_pass(x, x_dtype, gather_k, rt, M, num_experts, lora_a, lora_b, adapter_dtype, rank,
                             in_features, out_features, h_dtype, t_workspace, proj, stream);
  if (st != E4B_OK || M == 0) return st;
  if (!h) return fail(E4B_EINVAL, "NULL pointer");
  const int64_t nh = gated_epi ? out_features / 2 : out_features;
  const int64_t ncb = cdiv(nh, e4b::kLoraThreads);
  const int tile_rows = lora_tile_rows(M);
  if (cdiv(M, tile_rows) * ncb > 0x7fffffffLL) return fail(E4B_EUNSUPPORTED, "LoRA delta grid too large");
  const dim3 gb(static_cast<unsigned>(cdiv(M, tile_rows) * ncb));
#define E4B_LE(AD, OD, HD, RB, G)                                                                                  \
  hipLaunchKernelGGL((e4b::lora_b_epilogue_kernel<AD, OD, HD, RB, G>), gb, dim3(e4b::kLoraThreads), 0, stream,     \
                     t_workspace, rt->offsets, num_experts, lora_b, rank, nh, out_features, scaling, proj, epilogue, \
                     limit, static_cast<uint16_t*>(h), M, tile_rows, ncb)
#define E4B_LE_R(AD, OD, HD, G)                             \
  if (rank <= 16) E4B_LE(AD, OD, HD, 16, G);                \
  else if (rank <= 32) E4B_LE(AD, OD, HD, 32, G);           \
  else E4B_LE(AD, OD, HD, e4b::kLoraMaxRank, G);
#define E4B_LE_OD(AD, OD, HD)                               \
  if (gated_epi) { E4B_LE_R(AD, OD, HD, true) }             \
  else { E4B_LE_R(AD, OD, HD, false) }
#define E4B_LE_DT(AD, HD)                                   \
  if (adapter_dtype == AD && h_dtype == HD) {               \
    if (delta_dtype == E4B_FP32) { E4B_LE_OD(AD, E4B_FP32, HD) } \
    else { E4B_LE_OD(AD, HD, HD) }                          \
  }
  E4B_LE_DT(E4B_BF16, E4B_BF16) E4B_LE_DT(E4B_BF16, E4B_FP16)
  E4B_LE_DT(E4B_FP16, E4B_BF16) E4B_LE_DT(E4B_FP16, E4B_FP16)
  E4B_LE_DT(E4B_FP32, E4B_BF16) E4B_LE_DT(E4B_FP32, E4B_FP16)
#undef E4B_LE_DT
#undef E4B_LE_OD
#undef E4B_LE_R
#undef E4B_LE
  return check_launch("lora_b_epilogue_kernel");
}

int e4b_combine(const void* down, int32_t down_dtype, const int32_t* inv, const void* top_k_weights,
                int32_t weight_dtype, int64_t tokens, int32_t top_k, int64_t hidden, void* out, int32_t out_dtype,
                hipStream_t stream) {
  if (!any_dtype_ok(down_dtype)) return fail(E4B_EINVAL, "bad down dtype %d", down_dtype);
  if (!any_dtype_ok(weight_dtype) || !any_dtype_ok(out_dtype)) return fail(E4B_EINVAL, "bad weight/out dtype");
  if (tokens < 0 || top_k <= 0 || hidden <= 0) return fail(E4B_EINVAL, "bad sizes");
  if (tokens == 0) return E4B_OK;
  if (!down || !inv || !top_k_weights || !out) return fail(E4B_EINVAL, "NULL pointer");
  if (hidden % 8 == 0 && !aligned16(down)) return fail(E4B_EINVAL, "down must be 16-byte aligned");
  switch (down_dtype) {
    case E4B_FP32:
      launch_combine_dt<E4B_FP32>(down, inv, top_k_weights, weight_dtype, tokens, top_k, hidden, out, out_dtype, stream);
      break;
    case E4B_BF16:
      launch_combine_dt<E4B_BF16>(down, inv, top_k_weights, weight_dtype, tokens, top_k, hidden, out, out_dtype, stream);
      break;
    default:
      launch_combine_dt<E4B_FP16>(down, inv, top_k_weights, weight_dtype, tokens, top_k, hidden, out, out_dtype, stream);
      break;
  }
  return check_launch("combine_kernel");
}

int e4b_decode_gate_up(const void* hidden, int32_t act_dtype, int64_t tokens, const int64_t* top_k_index,
                       int32_t top_k, const e4b_qweight* w1, int32_t epilogue, float alpha, float limit, void* h,
                       hipStream_t stream) {
  int rc = check_weight(w1);
  if (rc) return rc;
  if (!act_dtype_ok(act_dtype)) return fail(E4B_EINVAL, "act_dtype must be bf16 or fp16 (got %d)", act_dtype);
  if (epilogue < E4B_EPI_NONE || epilogue > E4B_EPI_GPTOSS) return fail(E4B_EINVAL, "bad epilogue %d", epilogue);
  const bool pair = is_gated_epi(epilogue);
  if (pair && (w1->n % 2)) return fail(E4B_EINVAL, "gated epilogue needs an even n");
  if (epilogue == E4B_EPI_GPTOSS && !w1->bias) return fail(E4B_EINVAL, "gpt-oss epilogue needs the gate_up bias");
  if (tokens < 0 || top_k <= 0) return fail(E4B_EINVAL, "bad tokens/top_k");
  if (tokens == 0) return E4B_OK;
  const int64_t M = tokens * top_k;
  if (!decode_supported(M, w1->num_experts, w1, true))
    return fail(E4B_EUNSUPPORTED, "decode path needs tokens*top_k <= %d, E <= %d and k <= 4096 (got M=%lld E=%d)",
                e4b::kDecMaxRows, e4b::kDecMaxExperts, (long long)M, w1->num_experts);
  if (!hidden || !top_k_index || !h) return fail(E4B_EINVAL, "NULL pointer");
  if (!aligned16(hidden) || !aligned16(h)) return fail(E4B_EINVAL, "hidden / h must be 16-byte aligned");
  e4b::DecodeArgs a{};
  a.x = static_cast<const uint16_t*>(hidden);
  a.topk = top_k_index;
  a.tokens = static_cast<int>(tokens);
  a.k = top_k;
  a.E = w1->num_experts;
  a.w = *w1;
  a.epi = epilogue;
  a.alpha = alpha;
  a.limit = limit;
  a.out = h;
  a.odt = act_dtype;
  a.n_out = pair ? w1->n / 2 : w1->n;
  launch_decode<true>(a, act_dtype, std::min<int64_t>(w1->num_experts, M), M, stream);
  return check_launch("decode_up_kernel");
}

int e4b_decode_down_combine(const void* h, int32_t act_dtype, int64_t tokens, const int64_t* top_k_index,
                            const void* top_k_weights, int32_t weight_dtype, int32_t top_k, const e4b_qweight* w2,
                            void* out, int32_t out_dtype, hipStream_t stream) {
  int rc = check_weight(w2);
  if (rc) return rc;
  if (!act_dtype_ok(act_dtype)) return fail(E4B_EINVAL, "act_dtype must be bf16 or fp16 (got %d)", act_dtype);
  if (!any_dtype_ok(weight_dtype) || !any_dtype_ok(out_dtype)) return fail(E4B_EINVAL, "bad weight/out dtype");
  if (tokens < 0 || top_k <= 0) return fail(E4B_EINVAL, "bad tokens/top_k");
  if (tokens == 0) return E4B_OK;
  const int64_t M = tokens * top_k;
  if (!decode_supported(M, w2->num_experts, w2, false))
    return fail(E4B_EUNSUPPORTED, "decode path needs tokens*top_k <= %d, E <= %d and k <= 4096 (got M=%lld E=%d)",
                e4b::kDecMaxRows, e4b::kDecMaxExperts, (long long)M, w2->num_experts);
  if (!h || !top_k_index || !top_k_weights || !out) return fail(E4B_EINVAL, "NULL pointer");
  if (!aligned16(h)) return fail(E4B_EINVAL, "h must be 16-byte aligned");
  e4b::DecodeArgs a{};
  a.x = static_cast<const uint16_t*>(h);
  a.topk = top_k_index;
  a.topk_w = top_k_weights;
  a.wdt = weight_dtype;
  a.tokens = static_cast<int>(tokens);
  a.k = top_k;
  a.E = w2->num_experts;
  a.w = *w2;
  a.epi = E4B_EPI_NONE;
  a.out = out;
  a.odt = out_dtype;
  a.n_out = w2->n;
  launch_decode<false>(a, act_dtype, 0, M, stream);
  return check_launch("decode_down_kernel");
}

size_t e4b_moe_workspace_bytes(int64_t tokens, int32_t top_k, int32_t num_experts, int64_t n1, int64_t n2,
                               int32_t epilogue, int32_t act_dtype) {
  (void)act_dtype;
  const int64_t M = tokens * top_k;
  const int64_t h_cols = is_gated_epi(epilogue) ? n1 / 2 : n1;
  size_t b = 0;
  b += align256(sizeof(int32_t) * M);                                  // sorted_flat
  b += align256(sizeof(int32_t) * M);                                  // inv
  b += align256(sizeof(int32_t) * (num_experts + 1));                  // offsets
  b += align256(sizeof(int32_t) * num_experts);                        // active
  b += align256(sizeof(int32_t) * 2 * max_tiles_for(M, num_experts, mfma_tile_for(M, num_experts)));  // tiles
  b += align256(sizeof(int32_t) * 4);                                  // meta
  b += align256(sizeof(int32_t) * e4b_route_scratch_ints(M, num_experts));  // route scratch
  if (mfma_tile_for(M, num_experts) == e4b::kTileM) {                  // prefill re-tiling
    b += align256(sizeof(int32_t) * 2 * max_big_tiles(M, num_experts)) + align256(sizeof(int32_t) * 4);
    b += align256(sizeof(int32_t) * 2 * max_small_tiles(M, num_experts)) + align256(sizeof(int32_t) * 4);
  }
  b += align256(sizeof(uint16_t) * M * h_cols);                        // h
  b += align256(sizeof(float) * M * n2);                               // down rows (fp32)
  b += align256(sizeof(int32_t) * tokens) + align256(sizeof(int32_t) * M);  // fp16 mode row exponents
  b += align256(sizeof(uint16_t) * tokens * n2);  // fp16 mode: scaled tokens (hidden = w1->k = w2->n)
  return b;
}

// side_ok: the prefill's 32-row tiles may run on the device's second stream (not for the
// allocation-free entry point).
static int moe_forward_impl(const void* hidden, int32_t act_dtype, int64_t tokens, const int64_t* top_k_index,
                            const void* top_k_weights, int32_t weight_dtype, int32_t top_k, const e4b_qweight* w1,
                            const e4b_qweight* w2, int32_t epilogue, float alpha, float limit, int32_t flags,
                            void* workspace, size_t workspace_bytes, void* out, int32_t out_dtype, hipStream_t stream,
                            bool side_ok) {
  int rc = check_weight(w1);
  if (rc) return rc;
  rc = check_weight(w2);
  if (rc) return rc;
  if (w1->num_experts != w2->num_experts) return fail(E4B_EINVAL, "w1/w2 expert counts differ");
  const bool pair = is_gated_epi(epilogue);
  const int64_t h_cols = pair ? w1->n / 2 : w1->n;
  if (h_cols != w2->k)
    return fail(E4B_EINVAL, "gate_up output (%lld) does not match down k (%lld)", (long long)h_cols,
                (long long)w2->k);
  if (w1->k != w2->n)
    return fail(E4B_EINVAL, "gate_up input (%lld) and down output (%lld) must both be the hidden size",
                (long long)w1->k, (long long)w2->n);
  if (tokens < 0 || top_k <= 0) return fail(E4B_EINVAL, "bad tokens/top_k");
  if (tokens == 0) return E4B_OK;
  const int E = w1->num_experts;
  const int64_t M = tokens * top_k;
  const size_t need = e4b_moe_workspace_bytes(tokens, top_k, E, w1->n, w2->n, epilogue, act_dtype);
  if (!workspace || workspace_bytes < need)
    return fail(E4B_ESPACE, "workspace %zu bytes < %zu needed", workspace_bytes, need);
  if (!aligned16(workspace)) return fail(E4B_EINVAL, "workspace must be 16-byte aligned");
  if (!act_dtype_ok(act_dtype)) return fail(E4B_EINVAL, "act_dtype must be bf16 or fp16 (got %d)", act_dtype);
  if (!any_dtype_ok(weight_dtype) || !any_dtype_ok(out_dtype)) return fail(E4B_EINVAL, "bad weight/out dtype");
  if (epilogue < E4B_EPI_NONE || epilogue > E4B_EPI_GPTOSS) return fail(E4B_EINVAL, "bad epilogue %d", epilogue);
  if (w1->format != w2->format) return fail(E4B_EINVAL, "w1 and w2 use different formats");
  if (epilogue == E4B_EPI_GPTOSS && !w1->bias) return fail(E4B_EINVAL, "gpt-oss epilogue needs the gate_up bias");
  if (!top_k_index || !top_k_weights || !hidden || !out) return fail(E4B_EINVAL, "NULL pointer");
  if (!aligned16(hidden)) return fail(E4B_EINVAL, "hidden must be 16-byte aligned");

  if (flags < E4B_PATH_AUTO || flags > E4B_PATH_MFMA) return fail(E4B_EINVAL, "bad flags %d", flags);
  // Decode path: routing recomputed in LDS, combine fused into the down projection; two
  // launches.
  const bool decode_ok = decode_supported(M, E, w1, true) && decode_supported(M, E, w2, false);
  const bool use_decode = decode_ok && ((flags == E4B_PATH_AUTO && tokens <= 8) || flags == E4B_PATH_GEMV);
  if (use_decode) {
    void* h = workspace;
    rc = e4b_decode_gate_up(hidden, act_dtype, tokens, top_k_index, top_k, w1, epilogue, alpha, limit, h, stream);
    if (rc) return rc;
    return e4b_decode_down_combine(h, act_dtype, tokens, top_k_index, top_k_weights, weight_dtype, top_k, w2, out,
                                   out_dtype, stream);
  }

  char* p = static_cast<char*>(workspace);
  auto take = [&](size_t bytes) {
    char* q = p;
    p += align256(bytes);
    return q;
  };
  e4b_routing rt;
  rt.sorted_flat = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * M));
  rt.inv = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * M));
  rt.offsets = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * (E + 1)));
  rt.active = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * E));
  rt.tile_m = mfma_tile_for(M, E);
  rt.max_tiles = static_cast<int32_t>(max_tiles_for(M, E, rt.tile_m));
  rt.tiles = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * 2 * rt.max_tiles));
  rt.meta = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * 4));
  rt.scratch = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * e4b_route_scratch_ints(M, E)));
  // fp16 matrix-core mode: both GEMMs on the MFMA path, bf16 activations, NF4 weight shifts
  const bool gemv_path = flags == E4B_PATH_GEMV || (flags == E4B_PATH_AUTO && tokens <= 4);
  const bool f16c = !gemv_path && act_dtype == E4B_BF16 && w1->format != E4B_FMT_MXFP4 && w1->shift && w2->shift;
  // Prefill-sized groups on the MFMA path run at two tile heights: big tiles -- 256 rows (the
  // eight-wave wide kernel) in the fp16 mode and for MXFP4 weights with bf16 activations; 128
  // rows otherwise -- and one 32-row tile for an expert whose last tile would hold at most 32
  // rows (the long Zipf tail of experts with a handful of rows each), whose cost is mostly the
  // streaming and decoding of its expert's weights.
  const bool split = rt.tile_m == e4b::kTileM && flags != E4B_PATH_GEMV;
  const bool wide = f16c || (act_dtype == E4B_BF16 && w1->format == E4B_FMT_MXFP4);
  e4b_routing rbig = rt, rsmall = rt;
  if (split) {
    rbig.tile_m = wide ? e4b::kTileMBig : e4b::kTileM;
    rbig.max_tiles = static_cast<int32_t>(max_tiles_for(M, E, rbig.tile_m));
    rbig.tiles = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * 2 * rbig.max_tiles));
    rbig.meta = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * 4));
    rsmall.tile_m = e4b::kTileMSmall;
    rsmall.max_tiles = static_cast<int32_t>(max_small_tiles(M, E));
    rsmall.tiles = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * 2 * rsmall.max_tiles));
    rsmall.meta = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * 4));
  }
  void* h = take(sizeof(uint16_t) * M * h_cols);
  void* down = take(sizeof(float) * M * w2->n);
  int32_t* xexp = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * tokens));
  int32_t* hexp = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * M));
  uint16_t* x16 = reinterpret_cast<uint16_t*>(take(sizeof(uint16_t) * tokens * w1->k));
  const int32_t* up_exp = f16c ? xexp : nullptr;
  int32_t* h_exp = f16c ? hexp : nullptr;
  // fp16 mode at prefill sizes (down k a multiple of 256: the wide and narrow kernels): the down
  // rows leave the GEMM as fp16 with the operand scales left on, times 2^-c. Both operands stay
  // within 2^15 in magnitude, so |sum| <= k 2^30 and c = 16 + ceil(log2 k) keeps every value
  // within 2^14 (fp16's range), with fp16's 11 significant bits down to 2^-14: half the bytes of
  // fp32 rows, written once and read once by the combine. (Mid-size batches keep fp32 rows: their
  // rows are few, and the combine's scale lookups cost more than the bytes saved.)
  int f16_shift = 0;
  if (f16c && split && e4b::lora_gemm_fits(e4b::kTileMSmall, w2->k)) {
    int lg = 0;
    while ((int64_t(1) << lg) < w2->k) ++lg;
    f16_shift = 16 + lg;
  }
  // the gate_up GEMM reads the tokens as scaled fp16 rows in fp16 mode
  const void* up_a = f16c ? static_cast<const void*>(x16) : hidden;

  // fp16 mode: the token row exponents and scaled fp16 rows ride in the routing's first launch;
  // a prefill's two tile lists come from the routing's table step
  const RowExpArgs rx{static_cast<const uint16_t*>(hidden), w1->k, xexp, x16};
  rc = route_impl(top_k_index, tokens, top_k, E, &rt, f16c ? &rx : nullptr, stream,
                  e4b::SplitTiles{rbig, rsmall, split ? 1 : 0});
  if (rc) return rc;
  // fp16 mode: h row exponents, and h rewritten in place as scaled fp16 rows for the down GEMM
  auto h_to_f16 = [&]() {
    if (!f16c) return 0;
    e4b::launch_row_exp(static_cast<const uint16_t*>(h), M, h_cols, hexp, static_cast<uint16_t*>(h), nullptr, 0,
                        stream);
    return check_launch("row_exp_kernel");
  };
  if (split) {
    // the two tile heights write disjoint rows: the 32-row tiles go to the side stream (forked
    // after everything they read, joined before anything reads what they write)
    SideLease lease(stream, side_ok);
    auto both = [&](int site, auto&& launch) {
      return run_tile_heights(lease.get(), stream, &rbig, &rsmall, site, launch);
    };
    rc = both(E4B_PROBE_GATE_UP_BIG, [&](const e4b_routing* r, hipStream_t s) {
      return grouped_gemm_impl(up_a, act_dtype, top_k, w1, r, tokens, M, epilogue, alpha, limit, flags, h, act_dtype,
                               up_exp, s);
    });
    if (rc) return rc;
    rc = h_to_f16();
    if (rc) return rc;
    rc = both(E4B_PROBE_DOWN_BIG, [&](const e4b_routing* r, hipStream_t s) {
      return grouped_gemm_impl(h, act_dtype, 0, w2, r, tokens, M, E4B_EPI_NONE, alpha, limit, flags, down, E4B_FP32,
                               h_exp, s, nullptr, f16_shift);
    });
    if (rc) return rc;
  } else {
    rc = grouped_gemm_impl(up_a, act_dtype, top_k, w1, &rt, tokens, M, epilogue, alpha, limit, flags, h, act_dtype,
                           up_exp, stream);
    if (rc) return rc;
    rc = h_to_f16();
    if (rc) return rc;
    rc = grouped_gemm_impl(h, act_dtype, 0, w2, &rt, tokens, M, E4B_EPI_NONE, alpha, limit, flags, down, E4B_FP32,
                           h_exp, stream, nullptr, f16_shift);
    if (rc) return rc;
  }
  if (f16_shift) {
    const e4b::CombineScale cs{hexp, top_k_index, w2->shift, f16_shift};
    launch_combine_dt<E4B_FP16, true>(down, rt.inv, top_k_weights, weight_dtype, tokens, top_k, w2->n, out, out_dtype,
                                      stream, cs);
    return check_launch("combine_kernel");
  }
  return e4b_combine(down, E4B_FP32, rt.inv, top_k_weights, weight_dtype, tokens, top_k, w2->n, out, out_dtype,
                     stream);
}

int e4b_moe_forward(const void* hidden, int32_t act_dtype, int64_t tokens, const int64_t* top_k_index,
                    const void* top_k_weights, int32_t weight_dtype, int32_t top_k, const e4b_qweight* w1,
                    const e4b_qweight* w2, int32_t epilogue, float alpha, float limit, int32_t flags, void* workspace,
                    size_t workspace_bytes, void* out, int32_t out_dtype, hipStream_t stream) {
  return moe_forward_impl(hidden, act_dtype, tokens, top_k_index, top_k_weights, weight_dtype, top_k, w1, w2,
                          epilogue, alpha, limit, flags, workspace, workspace_bytes, out, out_dtype, stream, true);
}

int e4b_set_probe(int32_t site, hipEvent_t before, hipEvent_t after) {
  if (site < E4B_PROBE_OFF || site > E4B_PROBE_DOWN_TAIL) return fail(E4B_EINVAL, "bad probe site %d", site);
  if (site != E4B_PROBE_OFF && (!before || !after)) return fail(E4B_EINVAL, "NULL probe event");
  std::lock_guard<std::mutex> lk(g_probe_mu);
  g_probe_ev[0] = site == E4B_PROBE_OFF ? nullptr : before;
  g_probe_ev[1] = site == E4B_PROBE_OFF ? nullptr : after;
  g_probe_site.store(site, std::memory_order_relaxed);
  return E4B_OK;
}

static_assert(e4b::kDecLoraMaxRank == e4b::kLoraMaxRank, "one rank limit for both LoRA paths");

}  // extern "C"

namespace {

// Whether the grouped LoRA forward runs in the fp16 mode with the deltas in the GEMM epilogues.
bool lora_fused_ok(int32_t act_dtype, const e4b_qweight* w1, const e4b_qweight* w2) {
  return act_dtype == E4B_BF16 && w1->format != E4B_FMT_MXFP4 && w1->shift && w2->shift &&
         e4b::lora_gemm_fits(e4b::kTileMSmall, w1->k) && e4b::lora_gemm_fits(e4b::kTileMSmall, w2->k);
}

// t = x . A^T for the sorted rows of rt's tiles on the matrix cores (bf16 x, in a multiple of 64,
// which the narrow kernel's k limit of that path implies): 64-row parts of 128-row tiles, whole
// 32-row tiles, the ranks in 16-rank blocks.
int lora_t_mfma(const void* x, int32_t gather_k, const e4b_routing& rt, const void* A, int32_t adt, int rank,
                int64_t in, float* t, hipStream_t stream) {
  if (in <= 0 || in % e4b::kLoraTK != 0)
    return fail(E4B_EINVAL, "in_features=%lld not a multiple of %d", (long long)in, e4b::kLoraTK);
  const int bm = rt.tile_m % 64 == 0 ? 64 : 32;
  if (rt.tile_m <= 0 || rt.tile_m % bm != 0) return fail(E4B_EINVAL, "tile_m=%d", rt.tile_m);
  const int64_t blocks = int64_t(rt.max_tiles) * (rt.tile_m / bm);
  if (blocks > 0x7fffffffLL) return fail(E4B_EUNSUPPORTED, "LoRA t grid too large");
  const dim3 grid(static_cast<unsigned>(blocks));
  const int nsm = rank <= 16 ? 1 : (rank <= 32 ? 2 : 4);
#define E4B_TM(AD, BM, NS)                                                                                    \
  if (adt == AD && bm == BM && nsm == NS)                                                                    \
    hipLaunchKernelGGL((e4b::lora_t_mfma_kernel<AD, BM, NS>), grid, dim3(BM / 16 * e4b::kWave), 0, stream,     \
                       static_cast<const uint16_t*>(x), gather_k, rt, A, rank, in, t);
#define E4B_TM_AD(AD) E4B_TM(AD, 64, 1) E4B_TM(AD, 64, 2) E4B_TM(AD, 64, 4) E4B_TM(AD, 32, 1) E4B_TM(AD, 32, 2) \
  E4B_TM(AD, 32, 4)
  E4B_TM_AD(E4B_BF16) E4B_TM_AD(E4B_FP16) E4B_TM_AD(E4B_FP32)
#undef E4B_TM_AD
#undef E4B_TM
  return check_launch("lora_t_mfma_kernel");
}

// The workspace of that path, carved from p when p is not NULL; returns its size. Routing (and for
// prefill-sized batches the 256- / 32-row re-tiling), token and h row exponents, the scaled tokens,
// h, the fp32 down rows and one fp32 t [M, rank] (gate_up's, then down's).
size_t carve_lora_fused(char* p, int64_t tokens, int64_t M, int E, int64_t h_cols, int64_t k1, int64_t n2, int rank,
                        e4b_routing* rt, e4b_routing* rbig, e4b_routing* rsmall, bool* split, int32_t** xexp,
                        int32_t** hexp, uint16_t** x16, void** h, void** down, float** t) {
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* q = p ? p + off : nullptr;
    off += align256(bytes);
    return q;
  };
  e4b_routing a{}, b{}, c{};
  a.sorted_flat = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * M));
  a.inv = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * M));
  a.offsets = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * (E + 1)));
  a.active = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * E));
  a.tile_m = mfma_tile_for(M, E);
  a.max_tiles = static_cast<int32_t>(max_tiles_for(M, E, a.tile_m));
  a.tiles = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * 2 * a.max_tiles));
  a.meta = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * 4));
  a.scratch = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * e4b_route_scratch_ints(M, E)));
  const bool sp = a.tile_m == e4b::kTileM;  // prefill-sized: 256-row tiles plus 32-row tails
  b = c = a;
  if (sp) {
    b.tile_m = e4b::kTileMBig;
    b.max_tiles = static_cast<int32_t>(max_tiles_for(M, E, b.tile_m));
    b.tiles = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * 2 * b.max_tiles));
    b.meta = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * 4));
    c.tile_m = e4b::kTileMSmall;
    c.max_tiles = static_cast<int32_t>(max_small_tiles(M, E));
    c.tiles = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * 2 * c.max_tiles));
    c.meta = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * 4));
  }
  int32_t* xe = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * tokens));
  int32_t* he = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * M));
  uint16_t* xs = reinterpret_cast<uint16_t*>(take(sizeof(uint16_t) * tokens * k1));
  void* hh = take(sizeof(uint16_t) * M * h_cols);
  void* dn = take(sizeof(float) * M * n2);
  float* tt = reinterpret_cast<float*>(take(sizeof(float) * M * rank));
  if (p) {
    *rt = a;
    *rbig = b;
    *rsmall = c;
    *split = sp;
    *xexp = xe;
    *hexp = he;
    *x16 = xs;
    *h = hh;
    *down = dn;
    *t = tt;
  }
  return off;
}

}  // namespace

extern "C" {

size_t e4b_moe_lora_workspace_bytes(int64_t tokens, int32_t top_k, int32_t num_experts, int64_t n1, int64_t n2,
                                    int32_t epilogue, int32_t act_dtype, int32_t rank) {
  (void)act_dtype;
  const int64_t M = tokens * top_k;
  const int64_t h_cols = is_gated_epi(epilogue) ? n1 / 2 : n1;
  const size_t t = align256(sizeof(float) * M * std::max(rank, 1));
  const size_t h = align256(sizeof(uint16_t) * M * h_cols);
  const size_t dec = h + 2 * t;  // h, t of the gate_up and of the down projection
  size_t g = 0;
  g += 2 * align256(sizeof(int32_t) * M);                               // sorted_flat, inv
  g += align256(sizeof(int32_t) * (num_experts + 1)) + align256(sizeof(int32_t) * num_experts);
  g += align256(sizeof(int32_t) * 2 * max_tiles_for(M, num_experts, mfma_tile_for(M, num_experts)));
  g += align256(sizeof(int32_t) * 4) + align256(sizeof(int32_t) * e4b_route_scratch_ints(M, num_experts));
  g += align256(sizeof(float) * M * n1) + h + align256(sizeof(float) * M * n2) + t;  // up, h, down, t
  // the fp16-mode path (k1 = n2, the hidden size)
  const size_t f = carve_lora_fused(nullptr, tokens, M, num_experts, h_cols, n2, n2, std::max(rank, 1), nullptr,
                                    nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr);
  return std::max(dec, std::max(g, f));
}

int e4b_moe_lora_forward(const void* hidden, int32_t act_dtype, int64_t tokens, const int64_t* top_k_index,
                         const void* top_k_weights, int32_t weight_dtype, int32_t top_k, const e4b_qweight* w1,
                         const e4b_qweight* w2, const e4b_lora* lora, int32_t epilogue, float limit, int32_t flags,
                         void* workspace, size_t workspace_bytes, void* out, int32_t out_dtype, hipStream_t stream) {
  int rc = check_weight(w1);
  if (rc) return rc;
  rc = check_weight(w2);
  if (rc) return rc;
  if (!lora) return fail(E4B_EINVAL, "lora is NULL");
  if (w1->num_experts != w2->num_experts) return fail(E4B_EINVAL, "w1/w2 expert counts differ");
  if (w1->format != w2->format) return fail(E4B_EINVAL, "w1 and w2 use different formats");
  if (w1->format == E4B_FMT_MXFP4) return fail(E4B_EUNSUPPORTED, "LoRA adapters wrap the NF4 formats only");
  const bool pair = epilogue == E4B_EPI_SWIGLU || epilogue == E4B_EPI_CLAMP_SWIGLU;
  if (!pair && epilogue != E4B_EPI_ACT)
    return fail(E4B_EUNSUPPORTED, "epilogue %d: the LoRA forward takes SWIGLU, CLAMP_SWIGLU and ACT", epilogue);
  if (pair && (w1->n % 2)) return fail(E4B_EINVAL, "gated epilogue needs an even n");
  const int64_t h_cols = pair ? w1->n / 2 : w1->n;
  if (h_cols != w2->k || w1->k != w2->n)
    return fail(E4B_EINVAL, "w1 [%lld, %lld] and w2 [%lld, %lld] do not chain", (long long)w1->n, (long long)w1->k,
                (long long)w2->n, (long long)w2->k);
  const int r = lora->rank;
  if (r <= 0 || r > e4b::kLoraMaxRank) return fail(E4B_EUNSUPPORTED, "rank=%d outside [1, %d]", r, e4b::kLoraMaxRank);
  if (!any_dtype_ok(lora->dtype)) return fail(E4B_EINVAL, "bad adapter dtype %d", lora->dtype);
  if (!act_dtype_ok(act_dtype)) return fail(E4B_EINVAL, "act_dtype must be bf16 or fp16 (got %d)", act_dtype);
  if (!any_dtype_ok(weight_dtype) || !any_dtype_ok(out_dtype)) return fail(E4B_EINVAL, "bad weight/out dtype");
  if (flags < E4B_PATH_AUTO || flags > E4B_PATH_MFMA) return fail(E4B_EINVAL, "bad flags %d", flags);
  if (tokens < 0 || top_k <= 0) return fail(E4B_EINVAL, "bad tokens/top_k");
  if (tokens == 0) return E4B_OK;
  const int E = w1->num_experts;
  const int64_t M = tokens * top_k;
  const size_t need = e4b_moe_lora_workspace_bytes(tokens, top_k, E, w1->n, w2->n, epilogue, act_dtype, r);
  if (!workspace || workspace_bytes < need)
    return fail(E4B_ESPACE, "workspace %zu bytes < %zu needed", workspace_bytes, need);
  if (!hidden || !top_k_index || !top_k_weights || !out || !lora->a1 || !lora->b1 || !lora->a2 || !lora->b2)
    return fail(E4B_EINVAL, "NULL pointer");
  if (!aligned16(hidden) || !aligned16(workspace) || !aligned16(lora->a1) || !aligned16(lora->a2))
    return fail(E4B_EINVAL, "hidden, workspace and the A matrices must be 16-byte aligned");

  char* p = static_cast<char*>(workspace);
  auto take = [&](size_t bytes) {
    char* q = p;
    p += align256(bytes);
    return q;
  };
  const bool decode_ok = decode_supported(M, E, w1, true) && decode_supported(M, E, w2, false);
  if (decode_ok && ((flags == E4B_PATH_AUTO && tokens <= 8) || flags == E4B_PATH_GEMV)) {
    // t1 = A1 . x per flat row -> gate_up GEMV + delta + epilogue -> t2 = A2 . h -> down GEMV +
    // delta + combine: four launches, no routing tables.
    void* h = take(sizeof(uint16_t) * M * h_cols);
    float* t1 = reinterpret_cast<float*>(take(sizeof(float) * M * r));
    float* t2 = reinterpret_cast<float*>(take(sizeof(float) * M * r));
    auto t_rows = [&](const void* x, int gather_k, const void* A, int64_t in, float* t) {
      const dim3 grid(static_cast<unsigned>(M), static_cast<unsigned>(cdiv(r, e4b::kLoraThreads / e4b::kWave)));
#define E4B_LT(XD, AD)                                                                                            \
  if (act_dtype == XD && lora->dtype == AD)                                                                       \
    hipLaunchKernelGGL((e4b::lora_t_rows_kernel<XD, AD>), grid, dim3(e4b::kLoraThreads), 0, stream,               \
                       static_cast<const uint16_t*>(x), gather_k, top_k_index, E, A, r, in, t);
      E4B_LT(E4B_BF16, E4B_BF16) E4B_LT(E4B_BF16, E4B_FP16) E4B_LT(E4B_BF16, E4B_FP32)
      E4B_LT(E4B_FP16, E4B_BF16) E4B_LT(E4B_FP16, E4B_FP16) E4B_LT(E4B_FP16, E4B_FP32)
#undef E4B_LT
      return check_launch("lora_t_rows_kernel");
    };
    e4b::DecodeArgs a{};
    a.topk = top_k_index;
    a.tokens = static_cast<int>(tokens);
    a.k = top_k;
    a.E = E;
    a.lbdt = lora->dtype;
    a.lr = r;
    a.lscale = lora->scaling;
    rc = t_rows(hidden, top_k, lora->a1, w1->k, t1);
    if (rc) return rc;
    a.x = static_cast<const uint16_t*>(hidden);
    a.w = *w1;
    a.epi = epilogue;
    a.alpha = 1.0f;
    a.limit = limit;
    a.out = h;
    a.odt = act_dtype;
    a.n_out = h_cols;
    a.lt = t1;
    a.lb = lora->b1;
    launch_decode<true>(a, act_dtype, std::min<int64_t>(E, M), M, stream);
    rc = check_launch("decode_up_kernel (LoRA)");
    if (rc) return rc;
    rc = t_rows(h, 0, lora->a2, w2->k, t2);
    if (rc) return rc;
    a.x = static_cast<const uint16_t*>(h);
    a.topk_w = top_k_weights;
    a.wdt = weight_dtype;
    a.w = *w2;
    a.epi = E4B_EPI_NONE;
    a.out = out;
    a.odt = out_dtype;
    a.n_out = w2->n;
    a.lt = t2;
    a.lb = lora->b2;
    launch_decode<false>(a, act_dtype, 0, M, stream);
    return check_launch("decode_down_kernel (LoRA)");
  }

  // Grouped path in the fp16 matrix-core mode with each delta inside its GEMM's epilogue (bf16
  // activations, NF4 weights carrying shifts, both projections' k taken by the 32-row narrow
  // kernel): t1 = x . A1^T; gate_up GEMM + lscale t1 . B1^T + epilogue -> h; t2 = h . A2^T; h as
  // scaled fp16 rows; down GEMM + lscale t2 . B2^T -> fp32 rows; combine. No fp32 gate_up rows
  // and no pass over the down rows: the deltas ride the GEMM tiles' accumulators.
  const bool gemv_path = flags == E4B_PATH_GEMV || (flags == E4B_PATH_AUTO && tokens <= 4);
  if (!gemv_path && lora_fused_ok(act_dtype, w1, w2)) {
    e4b_routing rt, rbig, rsmall;
    bool split = false;
    int32_t *xexp, *hexp;
    uint16_t* x16;
    void *h, *down;
    float* t;
    carve_lora_fused(p, tokens, M, E, h_cols, w1->k, w2->n, r, &rt, &rbig, &rsmall, &split, &xexp, &hexp, &x16, &h,
                     &down, &t);
    const RowExpArgs rx{static_cast<const uint16_t*>(hidden), w1->k, xexp, x16};
    rc = route_impl(top_k_index, tokens, top_k, E, &rt, &rx, stream, e4b::SplitTiles{rbig, rsmall, split ? 1 : 0});
    if (rc) return rc;
    // the 32-row tiles of a split run on a side stream, as in e4b_moe_forward
    SideLease lease(stream, split);
    auto tiles = [&](int site, auto&& launch) {
      return split ? run_tile_heights(lease.get(), stream, &rbig, &rsmall, site, launch) : launch(&rt, stream);
    };
    rc = lora_t_mfma(hidden, top_k, rt, lora->a1, lora->dtype, r, w1->k, t, stream);
    if (rc) return rc;
    const LoraEpi l1{t, lora->b1, lora->dtype, r, lora->scaling};
    rc = tiles(E4B_PROBE_GATE_UP_BIG, [&](const e4b_routing* rp, hipStream_t s) {
      return grouped_gemm_impl(x16, act_dtype, top_k, w1, rp, tokens, M, epilogue, 1.0f, limit, E4B_PATH_MFMA, h,
                               act_dtype, xexp, s, &l1);
    });
    if (rc) return rc;
    // t2 from the bf16 h, before h is rewritten as scaled fp16 rows for the down GEMM
    rc = lora_t_mfma(h, 0, rt, lora->a2, lora->dtype, r, w2->k, t, stream);
    if (rc) return rc;
    e4b::launch_row_exp(static_cast<const uint16_t*>(h), M, h_cols, hexp, static_cast<uint16_t*>(h), nullptr, 0,
                        stream);
    rc = check_launch("row_exp_kernel");
    if (rc) return rc;
    const LoraEpi l2{t, lora->b2, lora->dtype, r, lora->scaling};
    rc = tiles(E4B_PROBE_DOWN_BIG, [&](const e4b_routing* rp, hipStream_t s) {
      return grouped_gemm_impl(h, act_dtype, 0, w2, rp, tokens, M, E4B_EPI_NONE, 1.0f, limit, E4B_PATH_MFMA, down,
                               E4B_FP32, hexp, s, &l2);
    });
    if (rc) return rc;
    return e4b_combine(down, E4B_FP32, rt.inv, top_k_weights, weight_dtype, tokens, top_k, w2->n, out, out_dtype,
                       stream);
  }

  // Grouped path otherwise: route once; gate_up GEMM to fp32 rows, its delta fused with the
  // activation, down GEMM to fp32 rows plus its delta, combine. The deltas stay fp32 until h / out
  // are rounded.
  e4b_routing rt;
  rt.sorted_flat = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * M));
  rt.inv = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * M));
  rt.offsets = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * (E + 1)));
  rt.active = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * E));
  rt.tile_m = mfma_tile_for(M, E);
  rt.max_tiles = static_cast<int32_t>(max_tiles_for(M, E, rt.tile_m));
  rt.tiles = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * 2 * rt.max_tiles));
  rt.meta = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * 4));
  rt.scratch = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * e4b_route_scratch_ints(M, E)));
  float* up = reinterpret_cast<float*>(take(sizeof(float) * M * w1->n));
  void* h = take(sizeof(uint16_t) * M * h_cols);
  float* down = reinterpret_cast<float*>(take(sizeof(float) * M * w2->n));
  float* t = reinterpret_cast<float*>(take(sizeof(float) * M * r));
  rc = e4b_route(top_k_index, tokens, top_k, E, &rt, stream);
  if (rc) return rc;
  rc = grouped_gemm_impl(hidden, act_dtype, top_k, w1, &rt, tokens, M, E4B_EPI_NONE, 1.0f, limit, flags, up, E4B_FP32,
                         nullptr, stream);
  if (rc) return rc;
  rc = e4b_lora_delta_epilogue(hidden, act_dtype, top_k, &rt, M, E, lora->a1, lora->b1, lora->dtype, r, w1->k, w1->n,
                               lora->scaling, E4B_FP32, t, up, epilogue, limit, h, act_dtype, stream);
  if (rc) return rc;
  rc = grouped_gemm_impl(h, act_dtype, 0, w2, &rt, tokens, M, E4B_EPI_NONE, 1.0f, limit, flags, down, E4B_FP32,
                         nullptr, stream);
  if (rc) return rc;
  rc = e4b_lora_delta(h, act_dtype, 0, &rt, M, E, lora->a2, lora->b2, lora->dtype, r, w2->k, w2->n, lora->scaling,
                      E4B_FP32, t, down, stream);
  if (rc) return rc;
  return e4b_combine(down, E4B_FP32, rt.inv, top_k_weights, weight_dtype, tokens, top_k, w2->n, out, out_dtype,
                     stream);
}

}  // extern "C"

namespace {

// The workspace of e4b_moe_forward_noalloc: a file-scope device array, one per device for the
// life of the process. Host code uses the address hipGetSymbolAddress gives on each device,
// never the array's name.
__device__ __align__(256) unsigned char scratch[E4B_NOALLOC_WORKSPACE_BYTES];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's `scratch`, taken on the first call on that device.
int scratch_address(void** ptr) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return check_launch("hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(E4B_EUNSUPPORTED, "device %d beyond %d devices", dev, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !p) {
      (void)hipGetLastError();
      return fail(E4B_ELAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(err));
    }
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return E4B_OK;
}

}  // namespace

extern "C" {

int e4b_moe_forward_noalloc(const void* hidden, int32_t act_dtype, int64_t tokens, const int64_t* top_k_index,
                            const void* top_k_weights, int32_t weight_dtype, int32_t top_k, const e4b_qweight* w1,
                            const e4b_qweight* w2, int32_t epilogue, float alpha, float limit, int32_t flags,
                            void* out, int32_t out_dtype, hipStream_t stream) {
  if (!w1 || !w2) return fail(E4B_EINVAL, "weight descriptor is NULL");
  if (tokens < 0 || top_k <= 0) return fail(E4B_EINVAL, "bad tokens/top_k");
  const size_t need = e4b_moe_workspace_bytes(tokens, top_k, w1->num_experts, w1->n, w2->n, epilogue, act_dtype);
  if (need > size_t(E4B_NOALLOC_WORKSPACE_BYTES))
    return fail(E4B_ESPACE, "this call needs %zu bytes of workspace; e4b_moe_forward_noalloc holds %zu",
                need, size_t(E4B_NOALLOC_WORKSPACE_BYTES));
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc) return rc;
  return moe_forward_impl(hidden, act_dtype, tokens, top_k_index, top_k_weights, weight_dtype, top_k, w1, w2, epilogue,
                          alpha, limit, flags, ws, size_t(E4B_NOALLOC_WORKSPACE_BYTES), out, out_dtype, stream, false);
}

}  // extern "C"
