/* e4b_amd.h -- C ABI of the MI355X (gfx950) frozen-expert MoE forward.
 *
 * The drop-in boundary for the hot path that experts4bit-qlora's `enable_fast(model)` routes
 * `ExpertsNbit` / `Experts4bit` modules through (pjordanandrsn/experts4bit-qlora v0.19.1).
 * Plain pointers and sizes only: every device pointer is HIP device memory, every call is
 * asynchronous on `stream`, nothing allocates device memory (callers pass outputs and any
 * workspace), and no C++ exception crosses the ABI. Each function returns E4B_OK (0) or a
 * negative status; `e4b_last_error()` then describes the failure (per host thread).
 *
 * Weight layouts (per expert, row = one output feature, `k` input features contiguous):
 *   NF4      packed u8 [E, n, k/2], FIRST element of a pair in the HIGH nibble;
 *            absmax fp32 [E, n*k/64]  (one scale per 64 consecutive elements of a row).
 *   NF4_DQ   as NF4, but absmax is u8 codes [E, n*k/64] into `code2` (256 fp32), with
 *            absmax2 fp32 [E, ceil(n*k/64/256)] and offset fp32 [E]:
 *            absmax[b] = fp32(fp32(code2[q[b]] * absmax2[b/256]) + offset).
 *   MXFP4    packed u8 [E, n, k/2], FIRST element in the LOW nibble (e2m1);
 *            absmax = e8m0 u8 [E, n, k/32] (value * 2^(s-127)).
 * Activations are bf16 or fp16 (the module's compute dtype); every GEMM accumulates in fp32.
 */
#ifndef E4B_AMD_H
#define E4B_AMD_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum e4b_status {
  E4B_OK = 0,
  E4B_EINVAL = -1,       /* bad argument (null pointer, shape, alignment, enum) */
  E4B_EUNSUPPORTED = -2, /* valid but not implemented (e.g. k not a multiple of 64) */
  E4B_ELAUNCH = -3,      /* a kernel launch failed (see e4b_last_error) */
  E4B_ESPACE = -4        /* workspace too small */
};

enum e4b_format { E4B_FMT_NF4 = 0, E4B_FMT_NF4_DQ = 1, E4B_FMT_MXFP4 = 2 };
enum e4b_dtype { E4B_BF16 = 0, E4B_FP16 = 1, E4B_FP32 = 2 };

/* Activation applied between the two projections (fused into the gate_up GEMM). */
enum e4b_epilogue {
  E4B_EPI_NONE = 0,         /* plain GEMM output (the reference's `gemm_4bit_grouped`) */
  E4B_EPI_SWIGLU = 1,       /* silu(gate) * up, gate = rows [0, n/2), up = rows [n/2, n) */
  E4B_EPI_ACT = 2,          /* silu(proj)  (has_gate = False) */
  E4B_EPI_CLAMP_SWIGLU = 3, /* silu(min(gate, L)) * clamp(up, -L, L) in fp32 (L <= 0: no clamp) */
  E4B_EPI_GPTOSS = 4        /* (clamp(up,-L,L) + 1) * (g * sigmoid(alpha * g)), g = min(gate, L),
                               after adding the per-expert gate_up bias */
};

/* Kernel-path selection flags for the grouped GEMMs (0 = automatic by token count). */
enum e4b_flags { E4B_PATH_AUTO = 0, E4B_PATH_GEMV = 1, E4B_PATH_MFMA = 2 };

typedef struct e4b_qweight {
  int32_t format;        /* e4b_format */
  int32_t num_experts;   /* E */
  int64_t n;             /* output features per expert */
  int64_t k;             /* input features per expert (multiple of 64) */
  const uint8_t* packed; /* [E, n, k/2] */
  const void* absmax;    /* NF4: fp32 [E, n*k/64]; NF4_DQ: u8 [E, n*k/64]; MXFP4: u8 [E, n, k/32] */
  const float* absmax2;  /* NF4_DQ only: fp32 [E, ceil(n*k/64/256)] */
  const float* offset;   /* NF4_DQ only: fp32 [E] */
  const float* code;     /* NF4 / NF4_DQ: fp32 [16] 4-bit code (the module's `code` buffer) */
  const float* code2;    /* NF4_DQ only: fp32 [256] second-level code */
  const void* bias;      /* optional [E, n] in the activation dtype (gpt-oss), else NULL */
  const int32_t* shift;  /* optional, NF4 / NF4_DQ: [E] per-expert power-of-two exponents from
                            e4b_weight_shift. When both projections carry them, e4b_moe_forward
                            runs its bf16 matrix-core GEMMs in fp16 (see there); NULL: not */
} e4b_qweight;

/* Device-side routing of M = tokens * top_k (token, slot) assignments. */
typedef struct e4b_routing {
  int32_t* sorted_flat; /* [M]     flat index (token*k + slot) of each expert-sorted row */
  int32_t* inv;         /* [M]     sorted row of each flat index (-1: dropped, id out of range) */
  int32_t* offsets;     /* [E + 1] exclusive prefix of per-expert row counts */
  int32_t* active;      /* [E]     ascending ids of experts with >= 1 row */
  int32_t* tiles;       /* [2 * max_tiles] (expert, first sorted row) of each tile_m-row tile */
  int32_t* meta;        /* [4]     num_tiles, num_active, num_dropped, tile_m */
  int32_t max_tiles;    /* capacity of `tiles`: >= ceil(M / tile_m) + min(E, M) */
  int32_t tile_m;       /* rows per tile (the MFMA path takes 128 or 32) */
  int32_t* scratch;     /* [e4b_route_scratch_ints(M, E)] per-chunk counts of the chunked route
                           (M > 4096); may be NULL when that size is 0 */
} e4b_routing;

/* Library version string and the last error message of the calling host thread. */
const char* e4b_version(void);
const char* e4b_last_error(void);

/* Rows per tile (128) of the grouped MFMA GEMM for prefill-sized groups; e4b_routing.tile_m
 * may also be 32, which the GEMM runs with 32-row tiles. */
int32_t e4b_mfma_tile_m(void);

/* Dequantize experts [expert_begin, expert_begin + expert_count) to a dense row-major
 * [count, n, k] tensor in out_dtype (E4B_BF16 / E4B_FP16 / E4B_FP32). Bit-exact: one fp32
 * product code[nib] * absmax, one round-to-nearest-even into out_dtype.
 * Replaces: ExpertsNbit._dequantize_expert (experts4bit_qlora/_vendor/experts.py:428-457,
 * bitsandbytes dequantize_4bit; pure-torch form engines/cold_engine.py:104-115) and, for
 * MXFP4, formats/mxfp4.py:35-105 dequantize_mxfp4 before its final transpose. */
int e4b_dequant(const e4b_qweight* w, int32_t expert_begin, int32_t expert_count, int32_t out_dtype,
                void* out, hipStream_t stream);

/* Per-expert weight exponents for the fp16 matrix-core mode of e4b_moe_forward: shift[e] =
 * 141 - max(E_e, 20), E_e the largest biased fp32 exponent of expert e's block scales (the
 * decoded ones for NF4_DQ), so every |code * absmax| * 2^shift[e] is below 2^15 and the scaled
 * weights sit in fp16's normal range. shift is [E] int32 on the device. NF4 / NF4_DQ only.
 * Has no counterpart in the reference: it is derived data of the weights, computed once per
 * weight version (the Python layer caches it with the kernel descriptors). */
int e4b_weight_shift(const e4b_qweight* w, int32_t* shift, hipStream_t stream);

/* int32 scratch the route needs for M = tokens * top_k routed rows over E experts: 0 up to
 * 4096 rows (one workgroup routes them), else ceil(M / 256) * (E + 1) (four launches over
 * 256-row chunks). */
int64_t e4b_route_scratch_ints(int64_t M, int32_t num_experts);

/* Token -> expert permutation, bit-exact to a stable argsort of top_k_index.reshape(-1).
 * Replaces: engines/fast.py:125-133 (argsort(stable), //k, %k, bincount, nonzero, .tolist());
 * nothing is copied to the host. Ids outside [0, E) are dropped (counted in meta[2]). */
int e4b_route(const int64_t* top_k_index, int64_t tokens, int32_t top_k, int32_t num_experts,
              const e4b_routing* rt, hipStream_t stream);

/* Routing of row groups with host sizes and device expert ids: group g holds the input rows
 * [sum(sizes[:g]), sum(sizes[:g+1])) for expert expert_ids[g] (int64, on the device, read only
 * there). An expert's groups are concatenated in group order; sorted_flat maps each sorted row to
 * its input row, inv each input row to its sorted row (-1 when the id is outside [0, E): those
 * rows are dropped and counted in meta[2]). The sizes travel as kernel arguments: nothing is
 * copied to or from host memory, so a decode loop with fixed sizes never synchronises.
 * groups <= 512; rt->max_tiles >= ceil(M / tile_m) + min(E, groups).
 * Replaces: the device-id grouped call of engines/pipelined.py:502-508 (gemm_4bit_grouped with
 * `sizes` on the host and the ids as a device tensor). */
int e4b_route_groups(const int64_t* sizes, int32_t groups, const int64_t* expert_ids, int32_t num_experts,
                     const e4b_routing* rt, hipStream_t stream);

/* Address-table row gather: for each slot s < slots, unless ident[s] == have[s] (the slot
 * already holds that row), copies n_bytes from the absolute address src_addr[s] (device memory
 * or host memory mapped into the device's address space) to dst + s * row_bytes + dst_off.
 * ident, have and src_addr are int64 device arrays. bytes_copied (optional, device) accumulates
 * the bytes moved. Replaces: _gather_rows_addr and its launch in engines/pipelined.py:117-151,
 * 408-417, with the traffic accounting of :471-487. */
int e4b_gather_rows(void* dst, int64_t row_bytes, int64_t dst_off, const int64_t* src_addr, const int64_t* ident,
                    const int64_t* have, int32_t slots, int64_t n_bytes, unsigned long long* bytes_copied,
                    hipStream_t stream);

/* Grouped GEMM over the expert-sorted rows: out[r, :] = epilogue(a_row(r) @ deq(W[e(r)]).T).
 * a_row(r) = a[sorted_flat[r] / gather_k] when gather_k > 0 (the gather of fast.py:135 fused
 * into the A loads), else a[r]. out is [M, n] (E4B_EPI_NONE, E4B_EPI_ACT) or [M, n/2] (gated
 * epilogues), in out_dtype: the activation dtype (one rounding of the fp32 result) or E4B_FP32.
 * The per-expert bias (w->bias) is added to the fp32 projection before the epilogue, as gpt-oss
 * does; the epilogue itself runs in fp32.
 * Replaces: nf4_grouped.gemm_4bit_grouped (engines/fast.py:137-143, 150-156, 220-226, 242-248)
 * and mxfp4_grouped.gemm_mxfp4_grouped (engines/nvme_experts.py:852-865), plus the epilogue
 * of lora.py:102-128 / hot_residency.py:72-80 fused into the same launch. */
int e4b_grouped_gemm(const void* a, int32_t act_dtype, int32_t gather_k, const e4b_qweight* w,
                     const e4b_routing* rt, int64_t tokens, int64_t M, int32_t epilogue, float alpha,
                     float limit, int32_t flags, void* out, int32_t out_dtype, hipStream_t stream);

/* Deterministic weighted combine back to token order:
 * out[t, :] = out_dtype( sum_{s<k} float(down[inv[t*k+s], :]) * float(top_k_weights[t, s]) ),
 * the slots summed in slot order in fp32 -- unique writes + a fixed-axis sum, never atomics.
 * down is [M, hidden] in down_dtype (bf16, fp16 or fp32).
 * Replaces: engines/fast.py:158 and _scatter_combine at fast.py:260-278. */
int e4b_combine(const void* down, int32_t down_dtype, const int32_t* inv, const void* top_k_weights,
                int32_t weight_dtype, int64_t tokens, int32_t top_k, int64_t hidden, void* out,
                int32_t out_dtype, hipStream_t stream);

/* Low-rank (LoRA) delta added to a grouped projection's fp32 rows, all expert groups at once:
 * for every expert-sorted row m below rt->offsets[E] (expert e: offsets[e] <= m < offsets[e+1])
 *   out[m, n] += delta_dtype( scaling * sum_j t[m, j] * lora_b[e, n, j] ),
 *   t[m, j] = sum_c x_m[c] * lora_a[e, j, c]   (fp32; t_workspace is [M, rank] fp32),
 * x_m = x[sorted_flat[m] / gather_k] when gather_k > 0 (token rows, as for gate_up), else x[m].
 * lora_a is [E, rank, in_features], lora_b [E, out_features, rank], both in adapter_dtype (bf16,
 * fp16 or fp32); x is in x_dtype (bf16 or fp16); out is [M, out_features] fp32; rank <= 64,
 * in_features a multiple of 8, num_experts <= 1024. Rows past offsets[E] are untouched.
 * Replaces: the per-expert Python loop of `up[s:t] += _lora(a_cat[s:t], A[e], B[e])` at
 * engines/fast.py:229-233 and 249-253 (lora.py:251-256 `_lora`), and its host sync on the
 * group sizes. */
int e4b_lora_delta(const void* x, int32_t x_dtype, int32_t gather_k, const e4b_routing* rt, int64_t M,
                   int32_t num_experts, const void* lora_a, const void* lora_b, int32_t adapter_dtype,
                   int32_t rank, int64_t in_features, int64_t out_features, float scaling,
                   int32_t delta_dtype, float* t_workspace, float* out, hipStream_t stream);

// The gate_up projection's LoRA delta fused with the activation, for the fused LoRA forward's
// first projection: the same t = x . A^T pass as e4b_lora_delta (same arguments and limits,
// the delta rounded to delta_dtype: h_dtype as the reference's `_lora` casts it back, or E4B_FP32
// to keep it unrounded), then for every routed row g = proj[m, n] + delta[m, n] and,
// for the gated epilogues, u = proj[m, n + out/2] + delta[m, n + out/2] (the `proj.chunk(2, -1)`
// halves), h[m, n] = h_dtype(SWIGLU / CLAMP_SWIGLU(g, u; limit) or ACT(g)). `proj` (fp32
// [M, out_features]) is only read; h is [M, out_features / 2] (gated) or [M, out_features].
// Replaces fast.py:229-233 followed by the base's `_epilogue` (lora.py:102-128) and its cast.
int e4b_lora_delta_epilogue(const void* x, int32_t x_dtype, int32_t gather_k, const e4b_routing* rt, int64_t M,
                            int32_t num_experts, const void* lora_a, const void* lora_b, int32_t adapter_dtype,
                            int32_t rank, int64_t in_features, int64_t out_features, float scaling,
                            int32_t delta_dtype, float* t_workspace, const float* proj, int32_t epilogue,
                            float limit, void* h, int32_t h_dtype, hipStream_t stream);

/* The two halves of e4b_lora_delta, for the training lane's backward (same arguments and
 * limits): t[m, :] = x_m . A[e_m]^T for the routed rows (t fp32 [M, rank]), and
 * out[m, :] += delta_dtype(scaling * t[m, :] . B[e_m]^T) (B [E, out_features, rank]).
 * Replaces: the `F.linear(x, A)` and `F.linear(., B)` halves of lora.py:251-256 `_lora`, per
 * expert group, inside nf4_qlora.fused_grouped_lora's forward and backward (grouped-nf4-gemm,
 * external; called at engines/fast.py:509-518, 531-540). */
int e4b_lora_t(const void* x, int32_t x_dtype, int32_t gather_k, const e4b_routing* rt, int64_t M,
               int32_t num_experts, const void* lora_a, int32_t adapter_dtype, int32_t rank, int64_t in_features,
               float* t, hipStream_t stream);
int e4b_lora_t_add(const float* t, const e4b_routing* rt, int64_t M, int32_t num_experts, const void* lora_b,
                   int32_t adapter_dtype, int32_t rank, int64_t out_features, float scaling, int32_t delta_dtype,
                   float* out, hipStream_t stream);

/* Per-expert LoRA weight gradient: out[e, j, c] = scale * sum over expert e's routed rows m (in
 * sorted order) of u[m, j] * a_m[c], out fp32 [E, rank, cols] (every expert written, zeros
 * where an expert has no rows). u fp32 [M, rank]; a_m = row sorted_flat[m] / gather_k of a
 * (gather_k > 0) or row m, a [*, cols] in a_dtype. dL/dA[e] = scaling * (g . B[e])^T x and
 * dL/dB[e]^T = scaling * t^T g of a projection's adapter.
 * Replaces: the adapter gradients of nf4_qlora.fused_grouped_lora's backward (grouped-nf4-gemm,
 * external; engines/fast.py:509-540), i.e. autograd through lora.py:251-256 per expert. */
int e4b_lora_wgrad(const float* u, int32_t rank, const void* a, int32_t a_dtype, int32_t gather_k,
                   const e4b_routing* rt, int64_t M, int32_t num_experts, int64_t cols, float scale, float* out,
                   hipStream_t stream);

/* Grouped input gradient of a frozen projection: out[m, :] = grad[m, :] . deq(W[e_m]) for the
 * expert-sorted rows (grad [M, w->n] in grad_dtype, out fp32 [M, w->k]); the weights are the
 * forward's dequantized values (one fp32 product code * absmax, one rounding to grad_dtype),
 * fp32 accumulation on the matrix cores, nothing materialised. rt->tile_m 128 or 32 (the row
 * tiles); NF4 / NF4_DQ; w->n a multiple of 64.
 * Replaces: the `grad_out @ deq(W)` of nf4_qlora.fused_grouped_lora's backward -- its per-expert
 * recompute-decode loop, or the single-launch dgrad kernel that engines/fast.py:426-452 selects
 * with `dgrad_kernel=True` (grouped-nf4-gemm >= 0.7.0, external). */
int e4b_grouped_dgrad(const void* grad, int32_t grad_dtype, const e4b_qweight* w, const e4b_routing* rt, int64_t M,
                      float* out, hipStream_t stream);

/* Decode path, first half: routing of top_k_index recomputed on the device (no route launch),
 * gate_up GEMV with the fused epilogue. h is [tokens * top_k, h_cols] in act_dtype, row
 * t * top_k + s holding token t's activation for slot s (flat order, not expert order).
 * Needs tokens * top_k <= 64, E <= 256, w1->k <= 4096 (E4B_EUNSUPPORTED otherwise).
 * Replaces: engines/fast.py:125-148 (sort, gather, gemm_4bit_grouped gate_up, _epilogue) for
 * small batches. */
int e4b_decode_gate_up(const void* hidden, int32_t act_dtype, int64_t tokens, const int64_t* top_k_index,
                       int32_t top_k, const e4b_qweight* w1, int32_t epilogue, float alpha, float limit,
                       void* h, hipStream_t stream);

/* Decode path, second half: down GEMV over every routed row plus the deterministic k-slot
 * combine, fused (out[t] = sum over s in slot order of (h[t*k+s] @ W2[e].T + bias) * w[t, s]).
 * Same limits as e4b_decode_gate_up.
 * Replaces: engines/fast.py:150-160 (gemm_4bit_grouped down, router-weight gather) and
 * _scatter_combine at fast.py:260-278. */
int e4b_decode_down_combine(const void* h, int32_t act_dtype, int64_t tokens, const int64_t* top_k_index,
                            const void* top_k_weights, int32_t weight_dtype, int32_t top_k,
                            const e4b_qweight* w2, void* out, int32_t out_dtype, hipStream_t stream);

/* Bytes of workspace e4b_moe_forward needs for these sizes. */
size_t e4b_moe_workspace_bytes(int64_t tokens, int32_t top_k, int32_t num_experts, int64_t n1,
                               int64_t n2, int32_t epilogue, int32_t act_dtype);

/* The whole frozen-expert forward: route -> gate_up (+epilogue, h rounded once to act_dtype)
 * -> down (+bias, fp32 sums) -> combine (one rounding into out_dtype).
 * hidden [tokens, w1->k] in act_dtype; top_k_index [tokens, top_k] int64; top_k_weights
 * [tokens, top_k] in weight_dtype; out [tokens, w2->n] in out_dtype.
 * Small batches (tokens <= 8, or flags == E4B_PATH_GEMV within the decode limits) take the
 * decode path, two launches (gate_up, then down + combine); larger ones route once and run the
 * grouped GEMMs.
 * fp16 matrix-core mode (bf16 activations, NF4 / NF4_DQ weights whose descriptors both carry
 * `shift`): the GEMMs multiply fp16 operands -- every weight fp16(fl32(code * absmax) *
 * 2^shift[e]) (one rounding of the fp32 product, 2^-11 relative, where bf16 weights carry
 * 2^-8), every activation row scaled by a power of two that puts its largest value in
 * [2^14, 2^15) (exact for bf16 values), the scales removed from the fp32 sums before the
 * epilogue -- so the layer keeps the decode path's accuracy at any batch. h is still rounded
 * once to act_dtype. At prefill sizes with w2->k a multiple of 256 the down rows are kept as
 * fp16 (11 significant bits) with the operand scales left on, times 2^-(16 + ceil(log2 k)) so
 * that they stay within fp16's range, and the combine takes the scales off in the router
 * weights; elsewhere they stay fp32. Without `shift` the GEMMs use the bf16 dequantized weights
 * themselves.
 * Replaces: engines/fast.py:100-160 fused_experts_forward (the bare-module forward that
 * enable_fast binds, fast.py:371-372), with no device->host synchronisation. */
int e4b_moe_forward(const void* hidden, int32_t act_dtype, int64_t tokens, const int64_t* top_k_index,
                    const void* top_k_weights, int32_t weight_dtype, int32_t top_k, const e4b_qweight* w1,
                    const e4b_qweight* w2, int32_t epilogue, float alpha, float limit, int32_t flags,
                    void* workspace, size_t workspace_bytes, void* out, int32_t out_dtype,
                    hipStream_t stream);

/* e4b_moe_forward without a workspace argument and without any allocation: the workspace is a
 * device array of E4B_NOALLOC_WORKSPACE_BYTES that the library holds on every device it runs on
 * until the process ends. Calls whose e4b_moe_workspace_bytes exceeds it fail with E4B_ESPACE
 * (at Qwen3-30B-A3B geometry that allows 800 tokens at top-8). All calls on one device share the array:
 * calls that overlap in time on one device (e.g. on two streams) race; calls in one stream's
 * order do not. The array is not cleared between calls (nothing the forward reads from it
 * has to start at zero).
 * No counterpart in the reference: for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). */
#define E4B_NOALLOC_WORKSPACE_BYTES (64u << 20)
int e4b_moe_forward_noalloc(const void* hidden, int32_t act_dtype, int64_t tokens, const int64_t* top_k_index,
                            const void* top_k_weights, int32_t weight_dtype, int32_t top_k, const e4b_qweight* w1,
                            const e4b_qweight* w2, int32_t epilogue, float alpha, float limit, int32_t flags,
                            void* out, int32_t out_dtype, hipStream_t stream);

/* Per-expert low-rank adapters of both projections (the ExpertsLoRA parameters, lora.py:172-175):
 * gate_up gains scaling * (x . A1[e]^T) . B1[e]^T, down gains scaling * (h . A2[e]^T) . B2[e]^T. */
typedef struct e4b_lora {
  const void* a1;  /* [E, rank, w1->k]  gate_up_lora_A */
  const void* b1;  /* [E, w1->n, rank]  gate_up_lora_B */
  const void* a2;  /* [E, rank, w2->k]  down_lora_A */
  const void* b2;  /* [E, w2->n, rank]  down_lora_B */
  int32_t dtype;   /* e4b_dtype of all four (bf16, fp16 or fp32) */
  int32_t rank;    /* 1..64 */
  float scaling;   /* alpha / rank */
} e4b_lora;

/* Bytes of workspace e4b_moe_lora_forward needs for these sizes (either path). */
size_t e4b_moe_lora_workspace_bytes(int64_t tokens, int32_t top_k, int32_t num_experts, int64_t n1, int64_t n2,
                                    int32_t epilogue, int32_t act_dtype, int32_t rank);

/* The whole frozen-expert forward with per-expert LoRA deltas, in one call: arguments as
 * e4b_moe_forward plus `lora`; epilogue SWIGLU, CLAMP_SWIGLU or ACT; NF4 / NF4_DQ weights.
 * Both deltas stay fp32 until h (act_dtype) and out (out_dtype) are rounded, as the base's
 * projections do.
 * Decode path (tokens <= 8 within the decode limits, or flags == E4B_PATH_GEMV): four
 * launches -- t1 = x . A1^T per routed row; the gate_up GEMV with scaling * t1 . B1[e, n, :]
 * added to each column's fp32 sum before the epilogue; t2 = h . A2^T; the down GEMV with its
 * delta added the same way, then the combine. Otherwise, with bf16 activations and both
 * weights carrying `shift` (and both k multiples of 256 up to 16384): route; t1 = x . A1^T on
 * the matrix cores; the gate_up grouped GEMM in the fp16 matrix-core mode whose tile
 * accumulators start as the tile's scaling * t1 . B1^T (t and B split into bf16 hi / lo
 * pairs: ~16 significant bits of the delta); the epilogue into h; t2 = h . A2^T; the down GEMM
 * the same way into fp32 rows; combine. Other larger batches: grouped GEMMs to fp32 rows, the
 * deltas of every expert group added on the device (as e4b_lora_delta_epilogue and
 * e4b_lora_delta), combine. No device->host synchronisation on any path.
 * Replaces: engines/fast.py:163-257 fused_experts_lora_forward (the ExpertsLoRA forward that
 * enable_fast binds, fast.py:328-329), whose groups are sliced on the host after a .tolist(). */
int e4b_moe_lora_forward(const void* hidden, int32_t act_dtype, int64_t tokens, const int64_t* top_k_index,
                         const void* top_k_weights, int32_t weight_dtype, int32_t top_k, const e4b_qweight* w1,
                         const e4b_qweight* w2, const e4b_lora* lora, int32_t epilogue, float limit, int32_t flags,
                         void* workspace, size_t workspace_bytes, void* out, int32_t out_dtype, hipStream_t stream);

/* Launch sites of the prefill path that e4b_set_probe can watch: the 256-row (big) tile launch
 * of each projection and its 32-row tail launch (which runs on the library's second stream when
 * one is free). */
enum e4b_probe_site {
  E4B_PROBE_OFF = 0,
  E4B_PROBE_GATE_UP_BIG = 1,
  E4B_PROBE_GATE_UP_TAIL = 2,
  E4B_PROBE_DOWN_BIG = 3,
  E4B_PROBE_DOWN_TAIL = 4
};

/* Measurement hook for benchmarks and profilers. While a site is set, every e4b_moe_forward /
 * e4b_moe_lora_forward whose routed rows are re-tiled into 256- and 32-row tiles runs both tile
 * heights on the caller's stream (no second stream, so each launch runs alone) and records
 * `before` on that stream right before the watched launch and `after` right after it, so
 * hipEventElapsedTime(before, after) is the launch's device time once `after` has completed.
 * E4B_PROBE_OFF clears it. One setting per process; the caller keeps both events alive while it
 * is set. Meant for eager calls (records made during a graph capture become graph nodes, whose
 * elapsed time did not follow the replays when measured). Has no counterpart in the reference:
 * it exists so that a benchmark can time one kernel of the fused forward with HIP events on the
 * stream that kernel is launched on. */
int e4b_set_probe(int32_t site, hipEvent_t before, hipEvent_t after);

#ifdef __cplusplus
}
#endif

#endif /* E4B_AMD_H */
