// Expert-grouped batched GEMV for the decode regime (few tokens per expert).
//
// Replaces the reference's per-output-element GEMV kernels
// (src/uma_qmoe/native/packed_q4_kernel.cu:72-152 q4/q8 linear, :156-231
// gate+up+SwiGLU, :1369-1426 down+route) with one CDNA4 design:
//   * a wavefront owns FPW weight rows; each lane streams one 16-byte chunk of
//     every row per step (global_load_dwordx4), so a row's bytes are read by
//     consecutive lanes, fully coalesced, exactly once per launch;
//   * dequantization is fused into v_dot2_f32_bf16 (see uqm_device.h), with
//     the FP32 group scale applied once per chunk;
//   * the activations of the (<= NT) routes that share the expert are staged
//     once per workgroup in LDS, already re-paired for the dot products, so one
//     pass over the weights serves every route of that expert;
//   * the per-lane partial sums of all FPW*NT*NMAT outputs are reduced together
//     with a halving butterfly (V-1+6-log2 V shuffles instead of 6V).
#include "uqm_internal.h"

namespace uqm {

template <int ENC, int NMAT, int NT, int FPW, int SU, int MODE>
__global__ __launch_bounds__(256) void expert_gemv_kernel(GemvArgs a) {
  using E = Enc<ENC>;
  constexpr int kWaves = 4;
  constexpr int kXQuads = E::kXWords / 4;
  constexpr int V = NMAT * FPW * NT;
  static_assert(V <= 64, "too many outputs per wave");

  extern __shared__ __align__(16) unsigned char lds[];

  const int slot = blockIdx.y;
  if (a.active_count != nullptr && slot >= *a.active_count) return;
  const int expert = a.active_experts != nullptr ? a.active_experts[slot] : slot;
  int rbeg, rend;
  if (a.expert_offsets != nullptr) {
    rbeg = a.expert_offsets[expert];
    rend = a.expert_offsets[expert + 1];
  } else {
    rbeg = 0;
    rend = a.n_routes;
  }
  if (rbeg >= rend) return;

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t C = a.K / E::kElems;  // 16-byte chunks per row
  const int64_t row_bytes = a.K * E::kBitsPerWeight / 8;
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * kWaves + wave) * FPW;

  uint4* xq = reinterpret_cast<uint4*>(lds);                       // [NT][kXQuads][C]
  float* xoff = reinterpret_cast<float*>(lds + sizeof(uint4) * NT * kXQuads * C);  // [NT][C]

  for (int rb = rbeg; rb < rend; rb += NT) {
    const int nt = min(NT, rend - rb);
    __syncthreads();
    // Stage the activation fragments of this route group.
    for (int64_t idx = threadIdx.x; idx < NT * C; idx += blockDim.x) {
      const int t = static_cast<int>(idx / C);
      const int64_t c = idx - t * C;
      XFrag<ENC> f;
      if (t < nt) {
        const int route = a.route_order != nullptr ? a.route_order[rb + t] : rb + t;
        const uint16_t* xr = a.x + static_cast<int64_t>(route / a.x_div) * a.ldx + c * E::kElems;
        uint32_t raw[E::kElems / 2];
#pragma unroll
        for (int q = 0; q < E::kElems / 8; ++q) {
          const uint4 v = ldg16(xr + 8 * q);
          raw[4 * q + 0] = v.x;
          raw[4 * q + 1] = v.y;
          raw[4 * q + 2] = v.z;
          raw[4 * q + 3] = v.w;
        }
        make_frag<ENC>(raw, f);
      } else {
#pragma unroll
        for (int j = 0; j < E::kXWords; ++j) f.w[j] = 0u;
        f.off = 0.f;
      }
#pragma unroll
      for (int q = 0; q < kXQuads; ++q)
        xq[(t * kXQuads + q) * C + c] = make_uint4(f.w[4 * q], f.w[4 * q + 1], f.w[4 * q + 2], f.w[4 * q + 3]);
      xoff[t * C + c] = f.off;
    }
    __syncthreads();

    float acc[NMAT][FPW][NT];
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
      for (int f = 0; f < FPW; ++f)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[m][f][t] = 0.f;

    if (row0 < a.rows) {
      const int64_t cpl = (C + 63) / 64;
      for (int64_t i0 = 0; i0 < cpl; i0 += SU) {
        uint4 wv[NMAT][FPW][SU];
        float sv[NMAT][FPW][SU];
#pragma unroll
        for (int u = 0; u < SU; ++u) {
          const int64_t c = lane + 64 * (i0 + u);
#pragma unroll
          for (int f = 0; f < FPW; ++f) {
            const int64_t r = row0 + f;
            const bool ok = c < C && r < a.rows;
            const int64_t grow = static_cast<int64_t>(expert) * a.rows + r;
#pragma unroll
            for (int m = 0; m < NMAT; ++m) {
              const uint8_t* rowp = (m == 0 && a.w_tail != nullptr && r >= a.tail_from)
                                        ? a.w_tail + (r - a.tail_from) * row_bytes
                                        : a.w[m] + grow * row_bytes;
              wv[m][f][u] = ok ? ldg16(rowp + c * 16) : make_uint4(0, 0, 0, 0);
              if constexpr (E::kScaled)
                sv[m][f][u] = ok ? a.s[m][expert * a.scales_per_expert + (r * a.K + c * E::kElems) / a.group] : 0.f;
              else
                sv[m][f][u] = 1.f;
            }
          }
        }
#pragma unroll
        for (int u = 0; u < SU; ++u) {
          const int64_t c = lane + 64 * (i0 + u);
          if (c < C) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
              XFrag<ENC> fr;
#pragma unroll
              for (int q = 0; q < kXQuads; ++q) {
                const uint4 v = xq[(t * kXQuads + q) * C + c];
                fr.w[4 * q + 0] = v.x;
                fr.w[4 * q + 1] = v.y;
                fr.w[4 * q + 2] = v.z;
                fr.w[4 * q + 3] = v.w;
              }
              fr.off = xoff[t * C + c];
#pragma unroll
              for (int m = 0; m < NMAT; ++m)
#pragma unroll
                for (int f = 0; f < FPW; ++f) {
                  const float d = dot_chunk<ENC>(wv[m][f][u], fr);
                  if constexpr (E::kScaled)
                    acc[m][f][t] = fmaf(d, sv[m][f][u], acc[m][f][t]);
                  else
                    acc[m][f][t] += d;
                }
            }
          }
        }
      }
    }

    float vals[V];
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
      for (int f = 0; f < FPW; ++f)
#pragma unroll
        for (int t = 0; t < NT; ++t) vals[(m * FPW + f) * NT + t] = acc[m][f][t];
    float r = wave_multi_sum<V>(vals);
    constexpr int kLog2V = (V >= 64) ? 6 : (V >= 32) ? 5 : (V >= 16) ? 4 : (V >= 8) ? 3 : (V >= 4) ? 2 : (V >= 2) ? 1 : 0;
    const int j = lane >> (6 - kLog2V);
    float other = 0.f;
    if constexpr (NMAT == 2) other = xor_partner<32>(r);
    const bool writer = (lane & ((64 >> kLog2V) - 1)) == 0;
    const int t = j % NT;
    const int f = (j / NT) % FPW;
    const int m = j / (NT * FPW);
    const int64_t row = row0 + f;
    if (writer && m == 0 && t < nt && row < a.rows) {
      const int route = a.route_order != nullptr ? a.route_order[rb + t] : rb + t;
      if constexpr (MODE == kModeSilu) {
        const float g = round_bf16(r);
        const float u = round_bf16(other);
        reinterpret_cast<uint16_t*>(a.out)[static_cast<int64_t>(route) * a.ldo + row] = f32_to_bf16(silu(g) * u);
      } else if constexpr (MODE == kModeF32) {
        reinterpret_cast<float*>(a.out)[static_cast<int64_t>(route) * a.ldo + row] = r;
      } else {
        reinterpret_cast<uint16_t*>(a.out)[static_cast<int64_t>(route) * a.ldo + row] = f32_to_bf16(r);
      }
    }
  }
}

template <int ENC>
constexpr int default_su() {
  return ENC == kQ4 ? 1 : ENC == kQ8 ? 2 : 4;
}

template <int ENC, int NMAT, int NT, int FPW, int MODE>
static hipError_t launch_gemv_fpw(const GemvArgs& a, int grid_y, hipStream_t stream) {
  using E = Enc<ENC>;
  const int64_t C = a.K / E::kElems;
  const size_t lds = (sizeof(uint4) * (E::kXWords / 4) + sizeof(float)) * NT * C;
  const int64_t waves = (a.rows + FPW - 1) / FPW;
  const dim3 grid(static_cast<unsigned>((waves + 3) / 4), static_cast<unsigned>(grid_y));
  hipLaunchKernelGGL((expert_gemv_kernel<ENC, NMAT, NT, FPW, default_su<ENC>(), MODE>), grid, dim3(256), lds, stream, a);
  return hipGetLastError();
}

template <int ENC, int NMAT, int NT, int MODE>
static hipError_t launch_gemv_nt(const GemvArgs& a, int grid_y, int fpw, hipStream_t stream) {
  if (fpw == 1) return launch_gemv_fpw<ENC, NMAT, NT, 1, MODE>(a, grid_y, stream);
  if (fpw == 2) return launch_gemv_fpw<ENC, NMAT, NT, 2, MODE>(a, grid_y, stream);
  return launch_gemv_fpw<ENC, NMAT, NT, 4, MODE>(a, grid_y, stream);
}

template <int ENC, int NMAT, int MODE>
static hipError_t launch_gemv_enc(const GemvArgs& a, int grid_y, int nt, int fpw, hipStream_t stream) {
  if (nt <= 1) return launch_gemv_nt<ENC, NMAT, 1, MODE>(a, grid_y, fpw, stream);
  if (nt <= 2) return launch_gemv_nt<ENC, NMAT, 2, MODE>(a, grid_y, fpw, stream);
  return launch_gemv_nt<ENC, NMAT, 4, MODE>(a, grid_y, fpw, stream);
}

size_t gemv_lds_bytes(int enc, int64_t K, int nt) {
  int xw = enc == kQ4 ? 16 : enc == kQ8 ? 8 : 4;
  int el = enc == kQ4 ? 32 : enc == kQ8 ? 16 : 8;
  int ntp = nt <= 1 ? 1 : nt <= 2 ? 2 : 4;
  return (sizeof(uint4) * (xw / 4) + sizeof(float)) * ntp * (K / el);
}

// Picks rows-per-wave so that the launch has enough waves to cover the chip.
static int pick_fpw(int64_t rows, int grid_y, int nmat) {
  const int64_t waves1 = rows * grid_y;
  if (nmat == 2) return waves1 >= 4 * 4096 ? 4 : (waves1 >= 2 * 4096 ? 2 : 1);
  return waves1 >= 4 * 4096 ? 4 : (waves1 >= 2 * 4096 ? 2 : 1);
}

hipError_t launch_expert_gemv(int enc, int nmat, int mode, const GemvArgs& args, int grid_y, int nt,
                              hipStream_t stream) {
  GemvArgs a = args;
  if (enc != kBF16) {
    if (a.group <= 0) return hipErrorInvalidValue;
    a.scales_per_expert = (a.rows * a.K + a.group - 1) / a.group;
  }
  const int fpw = pick_fpw(a.rows, grid_y, nmat);
  if (nmat == 2) {
    if (mode != kModeSilu) return hipErrorInvalidValue;
    if (enc == kQ4) return launch_gemv_enc<kQ4, 2, kModeSilu>(a, grid_y, nt, fpw, stream);
    if (enc == kQ8) return launch_gemv_enc<kQ8, 2, kModeSilu>(a, grid_y, nt, fpw, stream);
    return launch_gemv_enc<kBF16, 2, kModeSilu>(a, grid_y, nt, fpw, stream);
  }
  if (mode == kModeF32) {
    if (enc == kQ4) return launch_gemv_enc<kQ4, 1, kModeF32>(a, grid_y, nt, fpw, stream);
    if (enc == kQ8) return launch_gemv_enc<kQ8, 1, kModeF32>(a, grid_y, nt, fpw, stream);
    return launch_gemv_enc<kBF16, 1, kModeF32>(a, grid_y, nt, fpw, stream);
  }
  if (mode == kModeBF16) {
    if (enc == kQ4) return launch_gemv_enc<kQ4, 1, kModeBF16>(a, grid_y, nt, fpw, stream);
    if (enc == kQ8) return launch_gemv_enc<kQ8, 1, kModeBF16>(a, grid_y, nt, fpw, stream);
    return launch_gemv_enc<kBF16, 1, kModeBF16>(a, grid_y, nt, fpw, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace uqm
