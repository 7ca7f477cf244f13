// Weighted scatter-combine and RMSNorm.
//
// Combine: the reference accumulates each expert's weighted BF16 output with
// index_add_ in ascending expert order (src/uma_qmoe/custom_op.py:500-504); its
// fused GPU decode kernel sums the top-k slots in FP32 and rounds once
// (src/uma_qmoe/native/packed_q4_kernel.cu:1389-1424). Here every route's
// projection is kept in FP32 at its route index, so the combine is a gather
// in slot order with one final rounding; the Qwen shared expert and its
// sigmoid gate (src/uma_qmoe/qwen_compressed_loader.py:82-85) are folded in.
//
// RMSNorm: Transformers' Qwen2MoeRMSNorm (modeling_qwen2_moe.py:65-70),
// variance in FP32, normalised value cast to BF16, then times the weight.
#include "uqm_internal.h"

namespace uqm {

// The P FP32 partials of a row segment (loads only) and their sum in order.
template <int P>
__device__ __forceinline__ void load_parts(const float* __restrict__ base, int64_t stride, float4 (&u)[P]) {
#pragma unroll
  for (int p = 0; p < P; ++p) u[p] = *reinterpret_cast<const float4*>(base + p * stride);
}
template <int P>
__device__ __forceinline__ float4 add_parts(const float4 (&u)[P]) {
  float4 v = u[0];
#pragma unroll
  for (int p = 1; p < P; ++p) {
    v.x += u[p].x;
    v.y += u[p].y;
    v.z += u[p].z;
    v.w += u[p].w;
  }
  return v;
}

// One thread: 4 outputs of one token. YP routed and SP shared-expert FP32
// partials (SP = 0: no shared expert). The loads of the first 4 route slots
// (route id, weight, the partials of its row) and of the shared expert are
// issued before any is used, so for k <= 4 the thread waits about one memory
// round trip instead of one per slot and partial (each further group of 4
// slots adds one); the row of a dropped route is read (it lies in the
// workspace) and discarded. The arithmetic is the slot-order FMA chain of the
// partials' sums, then the shared term.
template <int YP, int SP>
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ y, int64_t y_stride,
                                                      const uint16_t* __restrict__ w,
                                                      const int64_t* __restrict__ idx, int64_t k, int64_t E,
                                                      int64_t H, const float* __restrict__ ys, int64_t ys_stride,
                                                      const float* __restrict__ sg, uint16_t* __restrict__ out) {
  constexpr int kSlots = 4;
  const int64_t t = blockIdx.y;
  const int64_t o = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  if (o >= H) return;
  float4 u[kSlots][YP];
  float ws[kSlots];
  bool live[kSlots];
  auto load_group = [&](int64_t s0) {
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
      const bool in = s0 + j < k;
      const int64_t slot = t * k + (in ? s0 + j : s0);
      const int64_t e = idx[slot];
      live[j] = in && e >= 0 && e < E;
      ws[j] = bf16_to_f32(w[slot]);
      load_parts<YP>(y + slot * H + o, y_stride, u[j]);
    }
  };
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  // a dropped slot keeps acc (a select, not a branch, so that the route ids
  // load with everything else)
  auto add_group = [&]() {
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
      const float4 v = add_parts<YP>(u[j]);
      const float4 f = make_float4(fmaf(ws[j], v.x, acc.x), fmaf(ws[j], v.y, acc.y), fmaf(ws[j], v.z, acc.z),
                                   fmaf(ws[j], v.w, acc.w));
      acc.x = live[j] ? f.x : acc.x;
      acc.y = live[j] ? f.y : acc.y;
      acc.z = live[j] ? f.z : acc.z;
      acc.w = live[j] ? f.w : acc.w;
    }
  };
  load_group(0);
  float4 su[SP > 0 ? SP : 1];
  float g = 0.f;
  if constexpr (SP > 0) {
    g = sg[t];
    load_parts<SP>(ys + t * H + o, ys_stride, su);
  }
  // keep the scheduler from moving the first group's arithmetic between its loads
  __builtin_amdgcn_sched_barrier(0);
  add_group();
  for (int64_t s0 = kSlots; s0 < k; s0 += kSlots) {
    load_group(s0);
    __builtin_amdgcn_sched_barrier(0);
    add_group();
  }
  if constexpr (SP > 0) {
    const float4 v = add_parts<SP>(su);
    acc.x = fmaf(g, v.x, acc.x);
    acc.y = fmaf(g, v.y, acc.y);
    acc.z = fmaf(g, v.z, acc.z);
    acc.w = fmaf(g, v.w, acc.w);
  }
  const uint32_t lo = static_cast<uint32_t>(f32_to_bf16(acc.x)) | (static_cast<uint32_t>(f32_to_bf16(acc.y)) << 16);
  const uint32_t hi = static_cast<uint32_t>(f32_to_bf16(acc.z)) | (static_cast<uint32_t>(f32_to_bf16(acc.w)) << 16);
  *reinterpret_cast<uint2*>(out + t * H + o) = make_uint2(lo, hi);
}

namespace {

struct CombineLaunch {
  const float* y;
  int64_t y_stride;
  const uint16_t* weights;
  const int64_t* indices;
  int64_t T, k, E, H;
  const float* ys;
  int64_t ys_stride;
  const float* sg;
  uint16_t* out;
  hipStream_t stream;
};

template <int YP, int SP>
hipError_t launch_parts(const CombineLaunch& c) {
  const dim3 grid(static_cast<unsigned>((c.H / 4 + 255) / 256), static_cast<unsigned>(c.T));
  hipLaunchKernelGGL((combine_kernel<YP, SP>), grid, dim3(256), 0, c.stream, c.y, c.y_stride, c.weights, c.indices,
                     c.k, c.E, c.H, c.ys, c.ys_stride, c.sg, c.out);
  return hipGetLastError();
}

template <int YP>
hipError_t launch_shared_parts(int sp, const CombineLaunch& c) {
  switch (sp) {
    case 0: return launch_parts<YP, 0>(c);
    case 1: return launch_parts<YP, 1>(c);
    case 2: return launch_parts<YP, 2>(c);
    case 3: return launch_parts<YP, 3>(c);
    case 4: return launch_parts<YP, 4>(c);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

// At most 4 K-split partials of each projection (the workspace holds 4).
hipError_t launch_combine(const float* y, int y_parts, int64_t y_stride, const uint16_t* weights,
                          const int64_t* indices, int64_t T, int64_t k, int64_t E, int64_t H, const float* ys,
                          int ys_parts, int64_t ys_stride, const float* sg, uint16_t* out, hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  const CombineLaunch c{y, y_stride, weights, indices, T, k, E, H, ys, ys_stride, sg, out, stream};
  const int sp = ys == nullptr ? 0 : ys_parts;
  switch (y_parts) {
    case 1: return launch_shared_parts<1>(sp, c);
    case 2: return launch_shared_parts<2>(sp, c);
    case 3: return launch_shared_parts<3>(sp, c);
    case 4: return launch_shared_parts<4>(sp, c);
    default: return hipErrorInvalidValue;
  }
}

__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* __restrict__ x, int64_t H,
                                                      const uint16_t* __restrict__ weight, float eps,
                                                      uint16_t* __restrict__ out) {
  __shared__ float part[4];
  const uint16_t* xr = x + blockIdx.x * H;
  uint16_t* orow = out + blockIdx.x * H;
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < H; i += blockDim.x) {
    const float v = bf16_to_f32(xr[i]);
    ss = fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float total = part[0] + part[1] + part[2] + part[3];
  const float r = rsqrtf(total / static_cast<float>(H) + eps);
  for (int64_t i = threadIdx.x; i < H; i += blockDim.x) {
    const float nv = round_bf16(bf16_to_f32(xr[i]) * r);
    const float wv = weight != nullptr ? bf16_to_f32(weight[i]) : 1.0f;
    orow[i] = f32_to_bf16(wv * nv);
  }
}

hipError_t launch_rmsnorm(const uint16_t* x, int64_t rows, int64_t H, const uint16_t* weight, float eps,
                          uint16_t* out, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0, stream, x, H, weight, eps,
                     out);
  return hipGetLastError();
}

}  // namespace uqm

namespace uqm {

__global__ __launch_bounds__(256) void zero_fill_kernel(uint4* __restrict__ p, size_t n16) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n16;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

hipError_t launch_zero_fill(void* p, size_t bytes, hipStream_t stream) {
  if (bytes == 0) return hipSuccess;
  if ((reinterpret_cast<uintptr_t>(p) & 15u) != 0 || bytes % 16 != 0) return hipErrorInvalidValue;
  const size_t n16 = bytes / 16;
  const unsigned blocks = static_cast<unsigned>(n16 / 256 + 1 < 1024 ? n16 / 256 + 1 : 1024);
  hipLaunchKernelGGL(zero_fill_kernel, dim3(blocks), dim3(256), 0, stream, static_cast<uint4*>(p), n16);
  return hipGetLastError();
}

}  // namespace uqm

namespace uqm {

// Dequantisation of an encoded Q4 or Q8 tensor to BF16: out[i] = bf16(q_i *
// scale[i / group]), the FP32 product rounded to nearest even, as the
// reference's correctness path builds its transient experts
// (src/uma_qmoe/q4.py:168-179 dequantize_q4, src/uma_qmoe/target_pack.py:144-176
// decode_target_tensor, then .to(bfloat16) at src/uma_qmoe/custom_op.py:416-431).
// Each thread takes 8 consecutive elements: 4 packed bytes (Q4, low nibble
// first, two's complement) or 8 bytes (Q8), one scale (group % 8 == 0), one
// 16-byte store.
template <bool Q4>
__global__ __launch_bounds__(256) void dequantize_kernel(const uint8_t* __restrict__ data,
                                                         const float* __restrict__ scales, int64_t n8,
                                                         int64_t group8, uint4* __restrict__ out) {
  for (int64_t c = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; c < n8;
       c += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const float s = scales[c / group8];
    int q[8];
    if constexpr (Q4) {
      const uint32_t w = reinterpret_cast<const uint32_t*>(data)[c];
#pragma unroll
      for (int j = 0; j < 8; ++j) q[j] = static_cast<int>((w >> (4 * j)) & 0xFu) - (((w >> (4 * j)) & 0x8u) ? 16 : 0);
    } else {
      const uint2 w = reinterpret_cast<const uint2*>(data)[c];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        q[j] = static_cast<int8_t>((w.x >> (8 * j)) & 0xFFu);
        q[4 + j] = static_cast<int8_t>((w.y >> (8 * j)) & 0xFFu);
      }
    }
    uint32_t h[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      h[j] = static_cast<uint32_t>(f32_to_bf16(static_cast<float>(q[2 * j]) * s)) |
             (static_cast<uint32_t>(f32_to_bf16(static_cast<float>(q[2 * j + 1]) * s)) << 16);
    out[c] = make_uint4(h[0], h[1], h[2], h[3]);
  }
}

hipError_t launch_dequantize(bool q4, const void* data, const float* scales, int64_t elements, int64_t group,
                             void* out, hipStream_t stream) {
  if (elements <= 0) return hipSuccess;
  const int64_t n8 = elements / 8;
  const int64_t want = (n8 + 255) / 256;
  const unsigned blocks = static_cast<unsigned>(want < 8192 ? want : 8192);
  if (q4)
    hipLaunchKernelGGL(dequantize_kernel<true>, dim3(blocks), dim3(256), 0, stream, static_cast<const uint8_t*>(data),
                       scales, n8, group / 8, static_cast<uint4*>(out));
  else
    hipLaunchKernelGGL(dequantize_kernel<false>, dim3(blocks), dim3(256), 0, stream,
                       static_cast<const uint8_t*>(data), scales, n8, group / 8, static_cast<uint4*>(out));
  return hipGetLastError();
}

}  // namespace uqm
