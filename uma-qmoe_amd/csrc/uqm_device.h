// Device-side building blocks shared by the UMA-QMoE MI355X kernels.
//
// Weight encodings (the canonical TargetPack/ExpertPack byte formats, read
// directly; nothing is dequantized to memory):
//   Q4   two's-complement nibbles, low nibble = even element, FP32 scale per
//        group of `group` elements along the flattened tensor
//        (reference: src/uma_qmoe/q4.py:96-179)
//   Q8   int8 codes, FP32 scale per group (src/uma_qmoe/target_pack.py:92-112)
//   BF16 raw little-endian bf16 (src/uma_qmoe/target_pack.py:78-89)
//
// Every kernel streams weights in 16-byte "chunks" (one 128-bit load per
// lane). A chunk holds 32 Q4, 16 Q8 or 8 BF16 weights, and never straddles a
// scale group because group % elements-per-chunk == 0 is enforced on the host.
//
// Dequantization is fused into the dot product with the bf16 magic-number
// trick: OR-ing a 4-bit field into the mantissa of bf16 128.0 (0x4300) gives
// exactly 128 + field, so v_dot2_f32_bf16 can consume packed weights after one
// AND-OR per pair; the constant offset is removed with a per-chunk activation
// sum that is computed once per token, not once per weight row.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace uqm {

enum Encoding : int { kQ4 = 0, kQ8 = 1, kBF16 = 2 };

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

constexpr int kWave = 64;

template <int ENC>
struct Enc;
template <>
struct Enc<kQ4> {
  static constexpr int kElems = 32;   // weights per 16-byte chunk
  static constexpr int kXWords = 16;  // bf16 pairs of activations per chunk
  static constexpr bool kScaled = true;
  static constexpr int kBitsPerWeight = 4;
};
template <>
struct Enc<kQ8> {
  static constexpr int kElems = 16;
  static constexpr int kXWords = 8;
  static constexpr bool kScaled = true;
  static constexpr int kBitsPerWeight = 8;
};
template <>
struct Enc<kBF16> {
  static constexpr int kElems = 8;
  static constexpr int kXWords = 4;
  static constexpr bool kScaled = false;
  static constexpr int kBitsPerWeight = 16;
};

// ---------------------------------------------------------------- bf16 ----
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// Round-to-nearest-even f32 -> bf16; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

// v_perm_b32: byte selectors 0-3 pick from `lo`, 4-7 from `hi`.
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }
__device__ __forceinline__ float sigmoidf_(float g) { return 1.0f / (1.0f + __expf(-g)); }

// ------------------------------------------------ activation fragments ----
// One lane's view of the activations under one weight chunk, re-paired to
// match the order in which the weight fields are unpacked.
//   Q4  dword d of the chunk holds elements 8d..8d+7; field j (bits 4j..4j+3)
//       and field j+4 (bits 16+4j..) are unpacked together, so pair
//       (d, j) = (x[8d+j], x[8d+j+4]).
//   Q8  dword d holds elements 4d..4d+3; pair A = (x[4d], x[4d+2]),
//       pair B = (x[4d+1], x[4d+3]) (low and high nibbles reuse the same pair).
//   BF16 natural pairs.
// `off` carries the constant-offset correction (see dot_chunk).
template <int ENC>
struct XFrag {
  uint32_t w[Enc<ENC>::kXWords];
  float off;
};

// raw: the chunk's activations as bf16 pairs in natural order
// (kElems/2 dwords). Builds the fragment for one token.
template <int ENC>
__device__ __forceinline__ void make_frag(const uint32_t* raw, XFrag<ENC>& f) {
  float s = 0.f;
  if constexpr (ENC == kQ4) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t a = raw[4 * d + 0], b = raw[4 * d + 1], c = raw[4 * d + 2], e = raw[4 * d + 3];
      f.w[4 * d + 0] = perm(c, a, 0x05040100u);
      f.w[4 * d + 1] = perm(c, a, 0x07060302u);
      f.w[4 * d + 2] = perm(e, b, 0x05040100u);
      f.w[4 * d + 3] = perm(e, b, 0x07060302u);
      s += bf16lo(a) + bf16hi(a) + bf16lo(b) + bf16hi(b) + bf16lo(c) + bf16hi(c) + bf16lo(e) + bf16hi(e);
    }
    f.off = -136.0f * s;  // value = 128 + (s ^ 8) = 136 + s for every Q4 field
  } else if constexpr (ENC == kQ8) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t a = raw[2 * d + 0], b = raw[2 * d + 1];
      f.w[2 * d + 0] = perm(b, a, 0x05040100u);
      f.w[2 * d + 1] = perm(b, a, 0x07060302u);
      s += bf16lo(a) + bf16hi(a) + bf16lo(b) + bf16hi(b);
    }
    f.off = -2304.0f * s;  // lo + 16*hi sums carry 128 + 16*128 + the +128 bias
  } else {
#pragma unroll
    for (int d = 0; d < 4; ++d) f.w[d] = raw[d];
    f.off = 0.f;
  }
}

// Dot product of one 16-byte weight chunk with one fragment, before scaling.
//   Q4: field u = nibble ^ 8 = q + 8; bf16(0x4300 | u) = 136 + q.
//       sum x*(136+q) + off = sum x*q.
//   Q8: byte u = code ^ 0x80 = q + 128 = 16*hi + lo;
//       sum x*(128+lo) + 16*sum x*(128+hi) + off = sum x*q.
template <int ENC>
__device__ __forceinline__ float dot_chunk(const uint4 wv, const XFrag<ENC>& f) {
  const uint32_t w4[4] = {wv.x, wv.y, wv.z, wv.w};
  if constexpr (ENC == kQ4) {
    float acc = f.off;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t u = w4[d] ^ 0x88888888u;
      acc = dot2((u & 0x000F000Fu) | 0x43004300u, f.w[4 * d + 0], acc);
      acc = dot2(((u >> 4) & 0x000F000Fu) | 0x43004300u, f.w[4 * d + 1], acc);
      acc = dot2(((u >> 8) & 0x000F000Fu) | 0x43004300u, f.w[4 * d + 2], acc);
      acc = dot2(((u >> 12) & 0x000F000Fu) | 0x43004300u, f.w[4 * d + 3], acc);
    }
    return acc;
  } else if constexpr (ENC == kQ8) {
    float lo = 0.f, hi = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t u = w4[d] ^ 0x80808080u;
      lo = dot2((u & 0x000F000Fu) | 0x43004300u, f.w[2 * d + 0], lo);
      lo = dot2(((u >> 8) & 0x000F000Fu) | 0x43004300u, f.w[2 * d + 1], lo);
      hi = dot2(((u >> 4) & 0x000F000Fu) | 0x43004300u, f.w[2 * d + 0], hi);
      hi = dot2(((u >> 12) & 0x000F000Fu) | 0x43004300u, f.w[2 * d + 1], hi);
    }
    return lo + 16.0f * hi + f.off;
  } else {
    float acc = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) acc = dot2(w4[d], f.w[d], acc);
    return acc;
  }
}

// ------------------------------------------------------- reductions ----
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Reduces V = 2^m per-lane values over the wave with V-1+6-m shuffles.
// On return every lane holds the full sum of value index lane >> (6 - m).
template <int V>
__device__ __forceinline__ float wave_multi_sum(float (&v)[V]) {
  static_assert((V & (V - 1)) == 0 && V >= 1 && V <= 64, "V must be a power of two <= 64");
  const int lane = threadIdx.x & (kWave - 1);
  float buf[V];
#pragma unroll
  for (int i = 0; i < V; ++i) buf[i] = v[i];
  int n = V;
  int o = 32;
#pragma unroll
  for (; n > 1; n >>= 1, o >>= 1) {
    const bool upper = (lane & o) != 0;
#pragma unroll
    for (int i = 0; i < n / 2; ++i) {
      const float keep = upper ? buf[i + n / 2] : buf[i];
      const float send = upper ? buf[i] : buf[i + n / 2];
      buf[i] = keep + __shfl_xor(send, o, kWave);
    }
  }
  float r = buf[0];
#pragma unroll
  for (; o > 0; o >>= 1) r += __shfl_xor(r, o, kWave);
  return r;
}

__device__ __forceinline__ uint4 ldg16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

}  // namespace uqm
