// Expert-grouped streaming GEMV for batched decode (a few tokens per expert).
//
// Replaces, for multi-token calls whose experts see few routes each (batch
// decode), the reference's per-expert GEMV launches (src/uma_qmoe/native/
// packed_q4_kernel.cu:72-152 and the per-expert Python loop of
// src/uma_qmoe/native_backend.py:319-372, 722-753).
//
// Work units are (active expert, output row) pairs in one flat range that a
// persistent grid splits evenly over its waves; a wave's share is a run of
// consecutive rows of one or two experts. For each expert in its run the
// wave loads the activations of up to NT of the expert's routes into
// registers (as dot-product fragments, once), then streams its rows: every
// lane reads whole 16-byte chunks, so one Q4 row of 2048 weights is a single
// coalesced 1 KB load, RB rows (of NMAT matrices) per round trip. The unpacked
// weight fields are shared by the NT routes' dot products, the per-lane sums
// of all RB x NMAT x NT outputs are reduced together by one halving butterfly,
// and one lane per output writes it. No LDS and no barrier: the waves never
// wait for each other, and the only dependent loads are the activations at an
// expert switch. Experts with more than NT routes take one pass per group of
// NT routes over the same rows (served from L2).
//
// Outputs, indexed by route id: MODE kModeSilu (NMAT = 2, gate and up)
// writes bf16(silu(bf16 g) * bf16 u) [route, rows]; kModeF32 writes the FP32
// row sums [route, rows] that the combine kernel weights and adds.
#include "uqm_internal.h"

namespace uqm {
namespace {

__device__ __forceinline__ int first_lane_value(int v) { return __builtin_amdgcn_readfirstlane(v); }

}  // namespace

template <int ENC, int NMAT, int CPL, int NT, int RB, int MODE>
__global__ __launch_bounds__(256) void routed_stream_kernel(GemvArgs a) {
  using E = Enc<ENC>;
  constexpr int V = NMAT * RB * NT;  // outputs reduced together per round trip
  static_assert(V <= 64 && (V & (V - 1)) == 0, "outputs per round trip must be a power of two <= 64");
  constexpr int kLog2V = V >= 64 ? 6 : V >= 32 ? 5 : V >= 16 ? 4 : V >= 8 ? 3 : V >= 4 ? 2 : V >= 2 ? 1 : 0;
  const int lane = threadIdx.x & 63;
  const int wave = first_lane_value(static_cast<int>(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)));
  const int nwaves = static_cast<int>(gridDim.x * (blockDim.x >> 6));
  const int64_t rows = a.rows;
  const int64_t W = static_cast<int64_t>(*a.active_count) * rows;  // (active expert, row) work units
  int64_t q = W * wave / nwaves;
  const int64_t q_end = W * (wave + 1) / nwaves;

  const int C = static_cast<int>(a.K / E::kElems);  // 16-byte chunks per row
  const int64_t row_bytes = a.K * E::kBitsPerWeight / 8;
  const int64_t spr = E::kScaled ? a.K / a.group : 0;  // scale groups per row
  // This lane's chunks lane + 64 j; past the row end a lane reads chunk 0
  // (in bounds) and drops its products.
  int chunk[CPL], sofs[CPL];
  bool valid[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    valid[j] = c < C;
    chunk[j] = valid[j] ? c : 0;
    sofs[j] = E::kScaled ? static_cast<int>(static_cast<int64_t>(chunk[j]) * E::kElems / a.group) : 0;
  }
  // Output of value index idx = (m * RB + f) * NT + t of the butterfly.
  const int idx = lane >> (6 - kLog2V);
  const int my_t = idx % NT, my_f = (idx / NT) % RB, my_m = idx / (NT * RB);
  const bool writer = (lane & ((64 >> kLog2V) - 1)) == 0 && my_m == 0;

  while (q < q_end) {
    const int slot = static_cast<int>(q / rows);
    const int64_t r_begin = q - static_cast<int64_t>(slot) * rows;
    const int64_t r_stop = min(rows, r_begin + (q_end - q));
    const int expert = a.active_experts[slot];
    const int t_begin = a.expert_offsets[expert], t_end = a.expert_offsets[expert + 1];
    const uint8_t* wbase[NMAT];
    const float* sbase[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; ++m) {
      wbase[m] = a.w[m] + static_cast<int64_t>(expert) * rows * row_bytes;
      sbase[m] = E::kScaled ? a.s[m] + static_cast<int64_t>(expert) * a.scales_per_expert : nullptr;
    }
    // The run's rows of this expert go RB rows of every matrix per round
    // trip. (Issuing the next round trip's loads before this one's products
    // measured slower: the second buffer costs occupancy.)
    auto load_batch = [&](int64_t r0, uint4(&wv)[NMAT][RB][CPL], float(&sv)[NMAT][RB][CPL]) {
      const int n = static_cast<int>(min(static_cast<int64_t>(RB), r_stop - r0));
#pragma unroll
      for (int f = 0; f < RB; ++f) {
        const int64_t r = r0 + (f < n ? f : n - 1);  // past n: the last row again (outputs dropped)
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
#pragma unroll
          for (int j = 0; j < CPL; ++j) {
            wv[m][f][j] = ldg16(wbase[m] + r * row_bytes + chunk[j] * 16);
            if constexpr (E::kScaled)
              sv[m][f][j] = sbase[m][r * spr + sofs[j]];
            else
              sv[m][f][j] = 1.f;
          }
        }
      }
    };
    for (int tg = t_begin; tg < t_end; tg += NT) {
      const int nt = min(NT, t_end - tg);
      // activation fragments of this route group (zero beyond nt)
      int my_route = 0;
      XFrag<ENC> xf[NT][CPL];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int route = a.route_order[tg + (t < nt ? t : 0)];
        if (t == my_t) my_route = route;
        const uint16_t* xr = a.x + static_cast<int64_t>(route / a.x_div) * a.ldx;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          uint32_t raw[E::kElems / 2];
          const uint16_t* src = xr + static_cast<int64_t>(chunk[j]) * E::kElems;
#pragma unroll
          for (int u = 0; u < E::kElems / 8; ++u) {
            const uint4 v = ldg16(src + 8 * u);
            raw[4 * u] = v.x;
            raw[4 * u + 1] = v.y;
            raw[4 * u + 2] = v.z;
            raw[4 * u + 3] = v.w;
          }
          make_frag<ENC>(raw, xf[t][j]);
          if (t >= nt) {
#pragma unroll
            for (int w = 0; w < E::kXWords; ++w) xf[t][j].w[w] = 0u;
            xf[t][j].off = 0.f;
          }
        }
      }
      for (int64_t r0 = r_begin; r0 < r_stop; r0 += RB) {
        const int n = static_cast<int>(min(static_cast<int64_t>(RB), r_stop - r0));
        uint4 wv[NMAT][RB][CPL];
        float sv[NMAT][RB][CPL];
        load_batch(r0, wv, sv);
        float vals[V];
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
          for (int f = 0; f < RB; ++f)
#pragma unroll
            for (int t = 0; t < NT; ++t) {
              float acc = 0.f;
#pragma unroll
              for (int j = 0; j < CPL; ++j) {
                const float d = dot_chunk<ENC>(wv[m][f][j], xf[t][j]) * sv[m][f][j];
                acc += valid[j] ? d : 0.f;
              }
              vals[(m * RB + f) * NT + t] = acc;
            }
        const float red = wave_multi_sum<V>(vals);  // full sum of value index idx
        float up = 0.f;
        if constexpr (NMAT == 2) up = xor_partner<32>(red);  // matrix 1 is index bit kLog2V - 1 = lane bit 5
        if (writer && my_f < n && my_t < nt) {
          const int64_t o = static_cast<int64_t>(my_route) * a.ldo + r0 + my_f;
          if constexpr (MODE == kModeSilu)
            reinterpret_cast<uint16_t*>(a.out)[o] = f32_to_bf16(silu(round_bf16(red)) * round_bf16(up));
          else
            reinterpret_cast<float*>(a.out)[o] = red;
        }
      }
    }
    q += r_stop - r_begin;
  }
}

namespace {

template <int ENC, int NMAT, int CPL, int NT, int RB, int MODE>
hipError_t launch_stream_cfg(const GemvArgs& a, int64_t max_active, int cus, hipStream_t stream) {
  auto kernel = routed_stream_kernel<ENC, NMAT, CPL, NT, RB, MODE>;
  // resident workgroups per CU (same on every gfx950 device; queried once)
  static const int per_cu = [&] {
    int n = 0;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, 256, 0) == hipSuccess && n > 0 ? n : 1;
  }();
  // persistent: every resident slot once, but no more waves than row batches
  int64_t grid = static_cast<int64_t>(cus) * per_cu;
  const int64_t batches = (max_active * a.rows + RB - 1) / RB;
  if (grid * 4 > batches) grid = (batches + 3) / 4;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

template <int ENC, int NMAT, int CPL, int MODE>
hipError_t launch_stream_nt(const GemvArgs& a, int nt, int64_t max_active, int cus, hipStream_t stream) {
  // 8 chunks of 16 bytes in flight per lane and round trip
  constexpr int RB = 8 / (NMAT * CPL) > 0 ? 8 / (NMAT * CPL) : 1;
  if (nt <= 1) return launch_stream_cfg<ENC, NMAT, CPL, 1, RB, MODE>(a, max_active, cus, stream);
  if (nt <= 2) return launch_stream_cfg<ENC, NMAT, CPL, 2, RB, MODE>(a, max_active, cus, stream);
  return launch_stream_cfg<ENC, NMAT, CPL, 4, RB, MODE>(a, max_active, cus, stream);
}

template <int ENC, int NMAT, int MODE>
hipError_t launch_stream_enc(const GemvArgs& a, int nt, int64_t max_active, int cus, hipStream_t stream) {
  const int64_t C = a.K / Enc<ENC>::kElems;
  if (C <= 64) return launch_stream_nt<ENC, NMAT, 1, MODE>(a, nt, max_active, cus, stream);
  if (C <= 128) return launch_stream_nt<ENC, NMAT, 2, MODE>(a, nt, max_active, cus, stream);
  if constexpr (ENC == kBF16) {
    if (C <= 256) return launch_stream_nt<ENC, NMAT, 4, MODE>(a, nt, max_active, cus, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace

// Up to 2 chunks per lane for Q4 and Q8 (K <= 4096 and 2048), 4 for BF16
// (K <= 2048): beyond that the round trip's registers spill.
bool stream_supported(int enc, int64_t K, int64_t group) {
  const int el = enc == kQ4 ? 32 : enc == kQ8 ? 16 : 8;
  if (K <= 0 || K % el != 0 || K / el > (enc == kBF16 ? 256 : 128)) return false;
  if (enc == kBF16) return true;
  return group > 0 && group % el == 0 && K % group == 0;
}

hipError_t launch_routed_stream(int enc, int nmat, int mode, const GemvArgs& args, int nt, int64_t max_active, int cus,
                                hipStream_t stream) {
  GemvArgs a = args;
  if (!stream_supported(enc, a.K, a.group)) return hipErrorInvalidValue;
  if (a.active_experts == nullptr || a.active_count == nullptr || a.expert_offsets == nullptr ||
      a.route_order == nullptr)
    return hipErrorInvalidValue;
  if (enc != kBF16) a.scales_per_expert = (a.rows * a.K + a.group - 1) / a.group;
  if (max_active <= 0) return hipSuccess;
  if (nmat == 2) {
    if (mode != kModeSilu) return hipErrorInvalidValue;
    if (enc == kQ4) return launch_stream_enc<kQ4, 2, kModeSilu>(a, nt, max_active, cus, stream);
    if (enc == kQ8) return launch_stream_enc<kQ8, 2, kModeSilu>(a, nt, max_active, cus, stream);
    return launch_stream_enc<kBF16, 2, kModeSilu>(a, nt, max_active, cus, stream);
  }
  if (mode != kModeF32) return hipErrorInvalidValue;
  if (enc == kQ4) return launch_stream_enc<kQ4, 1, kModeF32>(a, nt, max_active, cus, stream);
  if (enc == kQ8) return launch_stream_enc<kQ8, 1, kModeF32>(a, nt, max_active, cus, stream);
  return launch_stream_enc<kBF16, 1, kModeF32>(a, nt, max_active, cus, stream);
}

}  // namespace uqm
