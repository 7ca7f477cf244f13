/*
 * TEST INFRASTRUCTURE ONLY — CPU restatement of the reference's weight codecs.
 *
 * This file is the checker for the product's codecs and HIP dequantization.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it; the product path never does.
 *
 * Restated from the reference (zihaomu/UMA-QMoE):
 *   Q4   src/uma_qmoe/q4.py:12-14     symmetric [-7, 7], reserved -8
 *        src/uma_qmoe/q4.py:96-114    pack: low nibble first, two's complement
 *        src/uma_qmoe/q4.py:117-133   unpack: rejects -8 and a nonzero odd tail
 *        src/uma_qmoe/q4.py:136-165   quantize: scale = absmax/7 (f32), 0 -> 1.0,
 *                                     q = clip(rint(w / scale), -7, 7)
 *        src/uma_qmoe/q4.py:168-179   dequantize: q * scale in f32, scales must be
 *                                     finite and positive
 *   Q8   src/uma_qmoe/target_pack.py:92-112   scale = absmax/127, clip +-127
 *        src/uma_qmoe/target_pack.py:164-175  dequantize
 *   BF16 src/uma_qmoe/target_pack.py:78-89    RNE (w + 0x7FFF + lsb) >> 16
 *        src/uma_qmoe/bf16.py (NaN handling pinned by tests/unit/test_bf16.py:44-63)
 *
 * numpy semantics reproduced exactly: float32 division by a Python int is a
 * float32 division (NEP 50), np.rint is round-half-to-even, which is rintf()
 * under the default rounding mode.
 *
 * Return codes: 0 ok, 1 value out of range / reserved code, 2 nonzero tail
 * padding, 3 bad scale, 4 bad argument.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

int orc_q4_pack(const int8_t* values, int64_t n, uint8_t* out) {
  if (n <= 0) return 4;
  for (int64_t i = 0; i < n; ++i)
    if (values[i] < -7 || values[i] > 7) return 1;
  for (int64_t b = 0; b < (n + 1) / 2; ++b) {
    uint8_t lo = (uint8_t)(values[2 * b] & 0xF);
    uint8_t hi = (2 * b + 1 < n) ? (uint8_t)(values[2 * b + 1] & 0xF) : 0;
    out[b] = (uint8_t)(lo | (hi << 4));
  }
  return 0;
}

static int8_t nibble_to_signed(uint8_t nib) {
  return (int8_t)(nib >= 8 ? (int)nib - 16 : (int)nib);
}

int orc_q4_unpack(const uint8_t* packed, int64_t n, int8_t* out) {
  if (n <= 0) return 4;
  for (int64_t i = 0; i < n; ++i) {
    uint8_t byte = packed[i / 2];
    uint8_t nib = (i & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 0xF);
    int8_t v = nibble_to_signed(nib);
    if (v == -8) return 1;
    out[i] = v;
  }
  if ((n & 1) && (packed[n / 2] >> 4) != 0) return 2;
  return 0;
}

/* Group-wise symmetric quantization shared by Q4 (qmax 7) and Q8 (qmax 127). */
static void quantize_groups(const float* src, int64_t n, int64_t group,
                            int qmax, int8_t* q, float* scales) {
  int64_t groups = (n + group - 1) / group;
  for (int64_t g = 0; g < groups; ++g) {
    float absmax = 0.0f;
    for (int64_t i = g * group; i < (g + 1) * group && i < n; ++i) {
      float a = fabsf(src[i]);
      if (a > absmax) absmax = a;
    }
    float s = absmax / (float)qmax;
    if (s == 0.0f) s = 1.0f;
    scales[g] = s;
    for (int64_t i = g * group; i < (g + 1) * group && i < n; ++i) {
      float r = rintf(src[i] / s);
      if (r < (float)-qmax) r = (float)-qmax;
      if (r > (float)qmax) r = (float)qmax;
      q[i] = (int8_t)r;
    }
  }
}

int orc_q4_quantize(const float* src, int64_t n, int64_t group, int8_t* q_scratch,
                    uint8_t* packed, float* scales) {
  if (n <= 0 || group <= 0) return 4;
  for (int64_t i = 0; i < n; ++i)
    if (!isfinite(src[i])) return 1;
  quantize_groups(src, n, group, 7, q_scratch, scales);
  return orc_q4_pack(q_scratch, n, packed);
}

static int check_scales(const float* scales, int64_t groups) {
  for (int64_t g = 0; g < groups; ++g)
    if (!isfinite(scales[g]) || !(scales[g] > 0.0f)) return 3;
  return 0;
}

int orc_q4_dequantize(const uint8_t* packed, const float* scales, int64_t n,
                      int64_t group, int8_t* q_scratch, float* out) {
  if (n <= 0 || group <= 0) return 4;
  int rc = orc_q4_unpack(packed, n, q_scratch);
  if (rc) return rc;
  rc = check_scales(scales, (n + group - 1) / group);
  if (rc) return rc;
  for (int64_t i = 0; i < n; ++i) out[i] = (float)q_scratch[i] * scales[i / group];
  return 0;
}

int orc_q8_quantize(const float* src, int64_t n, int64_t group, int8_t* q,
                    float* scales) {
  if (n <= 0 || group <= 0) return 4;
  for (int64_t i = 0; i < n; ++i)
    if (!isfinite(src[i])) return 1;
  quantize_groups(src, n, group, 127, q, scales);
  return 0;
}

int orc_q8_dequantize(const int8_t* q, const float* scales, int64_t n,
                      int64_t group, float* out) {
  if (n <= 0 || group <= 0) return 4;
  int rc = check_scales(scales, (n + group - 1) / group);
  if (rc) return rc;
  for (int64_t i = 0; i < n; ++i) out[i] = (float)q[i] * scales[i / group];
  return 0;
}

/* f32 -> bf16 round-to-nearest-even; NaN stays a quiet NaN with its sign. */
void orc_f32_to_bf16(const float* src, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) {
    uint32_t w;
    memcpy(&w, &src[i], 4);
    if ((w & 0x7F800000u) == 0x7F800000u && (w & 0x007FFFFFu)) {
      out[i] = (uint16_t)((w >> 16) | 0x0040u);
      continue;
    }
    uint32_t rounding = 0x7FFFu + ((w >> 16) & 1u);
    out[i] = (uint16_t)((w + rounding) >> 16);
  }
}

void orc_bf16_to_f32(const uint16_t* src, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) {
    uint32_t w = (uint32_t)src[i] << 16;
    memcpy(&out[i], &w, 4);
  }
}
