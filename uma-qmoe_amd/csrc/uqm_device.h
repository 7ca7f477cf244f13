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

// Two floats -> a packed bf16 pair (lo in the low half), round to nearest
// even, in one instruction (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2_t;
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

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
  // ((w >> s) & 0x000F000F) ^ K puts two fields into the low bits of two bf16
  // halves whose high bits read 0x43 (128.0), flipping field bit 3 where K
  // has 0x8: one shift and one v_bitop3 per bf16 pair.
  constexpr uint32_t kM = 0x000F000Fu;
  if constexpr (ENC == kQ4) {
    constexpr uint32_t kK = 0x43084308u;  // field u = nibble ^ 8
    float acc = f.off;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t w = w4[d];
      acc = dot2((w & kM) ^ kK, f.w[4 * d + 0], acc);
      acc = dot2(((w >> 4) & kM) ^ kK, f.w[4 * d + 1], acc);
      acc = dot2(((w >> 8) & kM) ^ kK, f.w[4 * d + 2], acc);
      acc = dot2(((w >> 12) & kM) ^ kK, f.w[4 * d + 3], acc);
    }
    return acc;
  } else if constexpr (ENC == kQ8) {
    // byte ^ 0x80 = 16 * hi + lo: the low nibble is unchanged, bit 3 of the
    // high nibble flips.
    constexpr uint32_t kLo = 0x43004300u, kHi = 0x43084308u;
    float lo = 0.f, hi = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t w = w4[d];
      lo = dot2((w & kM) ^ kLo, f.w[2 * d + 0], lo);
      lo = dot2(((w >> 8) & kM) ^ kLo, f.w[2 * d + 1], lo);
      hi = dot2(((w >> 4) & kM) ^ kHi, f.w[2 * d + 0], hi);
      hi = dot2(((w >> 12) & kM) ^ kHi, f.w[2 * d + 1], hi);
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
// Cross-lane exchanges on the VALU (no LDS round trip): DPP within rows of
// 16 lanes, the gfx950 permlane swaps across rows. xor_partner<O> returns
// the value of a partner lane whose index differs from this lane's in bit
// log2(O) and agrees in every higher bit: lane ^ O for O = 1, 2, 16, 32
// (quad_perm, permlane16/32_swap), lane ^ 7 for O = 4 (row_half_mirror) and
// lane ^ 15 for O = 8 (row_mirror). That is all a butterfly reduction needs,
// and, once a reduction has left one value per group of lanes, it reads the
// neighbouring group's value.
template <int O>
__device__ __forceinline__ float xor_partner(float v) {
  const int u = __float_as_int(v);
  if constexpr (O == 1) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, u, 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
  } else if constexpr (O == 2) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, u, 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
  } else if constexpr (O == 4) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, u, 0x141, 0xF, 0xF, false));  // row_half_mirror
  } else if constexpr (O == 8) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, u, 0x140, 0xF, 0xF, false));  // row_mirror
  } else if constexpr (O == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);  // r[0]: even rows, r[1]: odd rows
    return __int_as_float((threadIdx.x & 16) ? r[0] : r[1]);
  } else {
    static_assert(O == 32, "O must be a power of two <= 32");
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);  // r[0]: low half, r[1]: high half
    return __int_as_float((threadIdx.x & 32) ? r[0] : r[1]);
  }
}

__device__ __forceinline__ float wave_sum(float v) {
  v += xor_partner<32>(v);
  v += xor_partner<16>(v);
  v += xor_partner<8>(v);
  v += xor_partner<4>(v);
  v += xor_partner<2>(v);
  v += xor_partner<1>(v);
  return v;
}

template <int O>
__device__ __forceinline__ float wave_max_step(float v) {
  return fmaxf(v, xor_partner<O>(v));
}
__device__ __forceinline__ float wave_max(float v) {
  v = wave_max_step<32>(v);
  v = wave_max_step<16>(v);
  v = wave_max_step<8>(v);
  v = wave_max_step<4>(v);
  v = wave_max_step<2>(v);
  return wave_max_step<1>(v);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#define UQM_MAXSTEP(O) v = max(v, static_cast<uint32_t>(__float_as_int(xor_partner<O>(__int_as_float(static_cast<int>(v))))))
  UQM_MAXSTEP(32);
  UQM_MAXSTEP(16);
  UQM_MAXSTEP(8);
  UQM_MAXSTEP(4);
  UQM_MAXSTEP(2);
  UQM_MAXSTEP(1);
#undef UQM_MAXSTEP
  return v;
}

// Order-preserving 16-bit key of a bf16 value: larger value, larger key; -0
// and +0 share a key; NaN sorts above +inf (as a descending torch.sort puts
// it first). Keys of non-NaN values are >= 0x007F, so 0 marks "taken".
__device__ __forceinline__ uint32_t bf16_key(uint16_t u) {
  if ((u & 0x7FFFu) > 0x7F80u) return 0xFFFFu;
  if (u == 0x8000u) u = 0;
  return (u & 0x8000u) ? (~u & 0xFFFFu) : (u | 0x8000u);
}
// bf16_key of the bf16 bits u (low 16 bits) with selects only, no branches:
// the same key for every value (any NaN pattern maps to 0xFFFF).
__device__ __forceinline__ uint32_t bf16_key_select(uint32_t u) {
  const uint32_t mag = u & 0x7FFFu;
  const uint32_t k = ((u & 0x8000u) != 0u && mag != 0u) ? 0x7FFFu - mag : 0x8000u | mag;
  return mag > 0x7F80u ? 0xFFFFu : k;
}
__device__ __forceinline__ float bf16_of_key(uint32_t key) {
  const uint32_t u = (key & 0x8000u) ? (key & 0x7FFFu) : (~key & 0xFFFFu);
  return bf16_to_f32(static_cast<uint16_t>(u));
}

// Halving butterfly stage with partner distance O over n live values.
template <int O, int N>
__device__ __forceinline__ void multi_sum_stage(float* buf) {
  const bool upper = (threadIdx.x & O) != 0;
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const float keep = upper ? buf[i + N / 2] : buf[i];
    const float send = upper ? buf[i] : buf[i + N / 2];
    buf[i] = keep + xor_partner<O>(send);
  }
}

// Reduces V = 2^m per-lane values over the wave with V-1+6-m exchanges.
// On return every lane holds the full sum of value index lane >> (6 - m).
template <int V>
__device__ __forceinline__ float wave_multi_sum(float (&v)[V]) {
  static_assert((V & (V - 1)) == 0 && V >= 1 && V <= 64, "V must be a power of two <= 64");
  float buf[V];
#pragma unroll
  for (int i = 0; i < V; ++i) buf[i] = v[i];
  if constexpr (V >= 2) multi_sum_stage<32, V>(buf);
  if constexpr (V >= 4) multi_sum_stage<16, V / 2>(buf);
  if constexpr (V >= 8) multi_sum_stage<8, V / 4>(buf);
  if constexpr (V >= 16) multi_sum_stage<4, V / 8>(buf);
  if constexpr (V >= 32) multi_sum_stage<2, V / 16>(buf);
  if constexpr (V >= 64) multi_sum_stage<1, V / 32>(buf);
  float r = buf[0];
  if constexpr (V < 2) r += xor_partner<32>(r);
  if constexpr (V < 4) r += xor_partner<16>(r);
  if constexpr (V < 8) r += xor_partner<8>(r);
  if constexpr (V < 16) r += xor_partner<4>(r);
  if constexpr (V < 32) r += xor_partner<2>(r);
  if constexpr (V < 64) r += xor_partner<1>(r);
  return r;
}

__device__ __forceinline__ uint4 ldg16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

}  // namespace uqm
