/* C restatement of the integer and dequant pieces of the frozen-expert MoE path.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (through oracle/c_oracle.py) to cross-check the
 * numpy restatement and to run byte-exact checks at full configuration sizes. The product
 * library never links it. Built with -ffp-contract=off so no product is fused into an FMA.
 *
 * Sources restated (pjordanandrsn/experts4bit-qlora v0.19.1):
 *   orc_dequant_4bit      experts4bit_qlora/engines/cold_engine.py:104-115 (high nibble first,
 *                         code[idx] * absmax in fp32) and _vendor/experts.py:428-457.
 *   orc_dequant_absmax_dq bitsandbytes nested QuantState (absmax = code2[q]*absmax2 + offset);
 *                         not in the reference (compress_statistics=False, _vendor/experts.py:415).
 *   orc_dequant_mxfp4     experts4bit_qlora/formats/mxfp4.py:84-99 (low nibble first, ldexp).
 *   orc_route             experts4bit_qlora/engines/fast.py:125-133 (stable argsort, bincount).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static const float kFp4Values[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                                     -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

uint16_t orc_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* n values; out_kind 0 = fp32 values, 1 = bf16 bits (uint16). */
void orc_dequant_4bit(const uint8_t* packed, const float* absmax, const float* code, int64_t n,
                      int blocksize, int out_kind, void* out) {
  for (int64_t i = 0; i < n; ++i) {
    uint8_t b = packed[i >> 1];
    uint8_t nib = (i & 1) ? (b & 0xF) : (b >> 4);
    float v = code[nib] * absmax[i / blocksize];
    if (out_kind == 0) ((float*)out)[i] = v;
    else ((uint16_t*)out)[i] = orc_f32_to_bf16(v);
  }
}

void orc_dequant_absmax_dq(const uint8_t* q, const float* absmax2, float offset, const float* code2,
                           int64_t nb, int blocksize2, float* out) {
  for (int64_t b = 0; b < nb; ++b) {
    float p = code2[q[b]] * absmax2[b / blocksize2];
    out[b] = p + offset;
  }
}

/* rows x K values, row-major; blocks [rows, K/2], scales [rows, K/32]. */
void orc_dequant_mxfp4(const uint8_t* blocks, const uint8_t* scales, int64_t rows, int64_t K,
                       int out_kind, void* out) {
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t k = 0; k < K; ++k) {
      uint8_t b = blocks[r * (K / 2) + k / 2];
      uint8_t nib = (k & 1) ? (b >> 4) : (b & 0xF);
      int e = (int)scales[r * (K / 32) + k / 32] - 127;
      float v = ldexpf(kFp4Values[nib], e);
      if (out_kind == 0) ((float*)out)[r * K + k] = v;
      else ((uint16_t*)out)[r * K + k] = orc_f32_to_bf16(v);
    }
  }
}

/* Stable counting sort of M expert ids in [0, E). Returns 0, or -1 on an out-of-range id.
 * order[r] = flat index of the r-th sorted row; inv[flat] = r; offsets[E+1] exclusive prefix. */
int orc_route(const int64_t* idx, int64_t M, int E, int64_t* order, int64_t* inv, int64_t* offsets) {
  for (int e = 0; e <= E; ++e) offsets[e] = 0;
  for (int64_t i = 0; i < M; ++i) {
    if (idx[i] < 0 || idx[i] >= E) return -1;
    offsets[idx[i] + 1]++;
  }
  for (int e = 0; e < E; ++e) offsets[e + 1] += offsets[e];
  /* cursor per expert: reuse a stack array when small */
  int64_t cursor_small[1024];
  int64_t* cursor = cursor_small;
  if (E > 1024) return -2;
  for (int e = 0; e < E; ++e) cursor[e] = offsets[e];
  for (int64_t i = 0; i < M; ++i) {
    int64_t r = cursor[idx[i]]++;
    order[r] = i;
    inv[i] = r;
  }
  return 0;
}
