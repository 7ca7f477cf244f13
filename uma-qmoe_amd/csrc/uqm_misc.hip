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

__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ y, int y_parts, int64_t y_stride,
                                                      const uint16_t* __restrict__ w,
                                                      const int64_t* __restrict__ idx, int64_t k, int64_t E,
                                                      int64_t H, const float* __restrict__ ys, int ys_parts,
                                                      int64_t ys_stride, const float* __restrict__ sg,
                                                      uint16_t* __restrict__ out) {
  const int64_t t = blockIdx.y;
  const int64_t o = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  if (o >= H) return;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int64_t s = 0; s < k; ++s) {
    const int64_t e = idx[t * k + s];
    if (e < 0 || e >= E) continue;
    const float ws = bf16_to_f32(w[t * k + s]);
    float4 v = *reinterpret_cast<const float4*>(y + (t * k + s) * H + o);
    for (int p = 1; p < y_parts; ++p) {
      const float4 u = *reinterpret_cast<const float4*>(y + p * y_stride + (t * k + s) * H + o);
      v.x += u.x;
      v.y += u.y;
      v.z += u.z;
      v.w += u.w;
    }
    acc.x = fmaf(ws, v.x, acc.x);
    acc.y = fmaf(ws, v.y, acc.y);
    acc.z = fmaf(ws, v.z, acc.z);
    acc.w = fmaf(ws, v.w, acc.w);
  }
  if (ys != nullptr) {
    const float g = sg[t];
    float4 v = *reinterpret_cast<const float4*>(ys + t * H + o);
    for (int p = 1; p < ys_parts; ++p) {
      const float4 u = *reinterpret_cast<const float4*>(ys + p * ys_stride + t * H + o);
      v.x += u.x;
      v.y += u.y;
      v.z += u.z;
      v.w += u.w;
    }
    acc.x = fmaf(g, v.x, acc.x);
    acc.y = fmaf(g, v.y, acc.y);
    acc.z = fmaf(g, v.z, acc.z);
    acc.w = fmaf(g, v.w, acc.w);
  }
  const uint32_t lo = static_cast<uint32_t>(f32_to_bf16(acc.x)) | (static_cast<uint32_t>(f32_to_bf16(acc.y)) << 16);
  const uint32_t hi = static_cast<uint32_t>(f32_to_bf16(acc.z)) | (static_cast<uint32_t>(f32_to_bf16(acc.w)) << 16);
  *reinterpret_cast<uint2*>(out + t * H + o) = make_uint2(lo, hi);
}

hipError_t launch_combine(const float* y, int y_parts, int64_t y_stride, const uint16_t* weights,
                          const int64_t* indices, int64_t T, int64_t k, int64_t E, int64_t H, const float* ys,
                          int ys_parts, int64_t ys_stride, const float* sg, uint16_t* out, hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((H / 4 + 255) / 256), static_cast<unsigned>(T));
  hipLaunchKernelGGL(combine_kernel, grid, dim3(256), 0, stream, y, y_parts, y_stride, weights, indices, k, E, H,
                     ys, ys_parts, ys_stride, sg, out);
  return hipGetLastError();
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
