// Counter program for the multi-token MoE paths (batch decode and prefill):
// a plain HIP program over the library's C ABI that issues a few hundred
// dispatches, so that rocprofv3 --pmc runs (which serialise and count every
// dispatch) stay short. It builds `instances` layers of one configuration
// with weights from a device-side generator (the timing does not depend on
// the values; every Q4 nibble and the bf16 patterns used decode to finite
// numbers), times `reps` rotations over them with HIP events, and prints one
// JSON line: microseconds per call, algorithmic bytes per call (each distinct
// routed expert once, plus router and shared expert) and the FLOPs.
//
//   grouped_counters [b32|c4|c5] [instances] [reps]
//
//   b32  Qwen1.5-MoE shape (H 2048, 60 experts, top-4, I 1408, shared 5632),
//        32 tokens, whole block (uqm_moe_layer: router, top-k, routed Q4
//        experts, shared expert, combine)
//   c4   the same block at 512 tokens
//   c5   128 experts, top-8, I 768, no shared expert, 256 tokens with given
//        routes (uqm_moe_forward); the routes are the top-8 of logits
//        0.905 * N(0, 1) + b_e with b_e = -1.1 * log(rank_e) over a seeded
//        ranking (Zipf s = 1.1; 0.905 = 0.02 * sqrt(2048), the spread of
//        x . w_e for x ~ N(0, 1) and w ~ N(0, 0.02))
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <numeric>
#include <random>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <vector>

#include "../../../include/uma_qmoe_hip.h"

#define CHECK(x)                                                                   \
  do {                                                                             \
    hipError_t e_ = (x);                                                           \
    if (e_ != hipSuccess) {                                                        \
      fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
      exit(1);                                                                     \
    }                                                                              \
  } while (0)
#define UQM(x)                                                                    \
  do {                                                                            \
    int rc_ = (x);                                                                \
    if (rc_ != UQM_OK) {                                                          \
      fprintf(stderr, "uqm error %d at line %d: %s\n", rc_, __LINE__, uqm_last_error()); \
      exit(1);                                                                    \
    }                                                                             \
  } while (0)

namespace {

__global__ void fill_words(uint32_t* p, size_t n, uint32_t seed, uint32_t mask, uint32_t bias) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    uint32_t h = static_cast<uint32_t>(i) * 2654435761u ^ seed;
    h ^= h >> 13;
    h *= 0x5bd1e995u;
    h ^= h >> 15;
    p[i] = (h & mask) | bias;
  }
}

// Small finite bf16 values (magnitudes in [2^-5, 2^-1)), two per word.
void fill_bf16(void* p, size_t elems, uint32_t seed) {
  hipLaunchKernelGGL(fill_words, dim3(1024), dim3(256), 0, 0, static_cast<uint32_t*>(p), elems / 2, seed,
                     0x81FF81FFu, 0x3D003D00u);
}
void fill_bytes(void* p, size_t bytes, uint32_t seed) {
  hipLaunchKernelGGL(fill_words, dim3(1024), dim3(256), 0, 0, static_cast<uint32_t*>(p), bytes / 4, seed,
                     0xFFFFFFFFu, 0u);
}
void fill_scales(float* p, size_t n) {  // 2^-8
  hipLaunchKernelGGL(fill_words, dim3(256), dim3(256), 0, 0, reinterpret_cast<uint32_t*>(p), n, 0u, 0u, 0x3B800000u);
}

template <typename T>
T* device_alloc(size_t n) {
  void* p = nullptr;
  CHECK(hipMalloc(&p, n * sizeof(T)));
  return static_cast<T*>(p);
}

struct Config {
  const char* name;
  int64_t H, E, k, I, Is, T;
};

// Zipf-biased top-k routes on the host (c5): ids [T, k] and bf16 weights
// (softmax over the biased logits, taken at the chosen ids).
void zipf_routes(const Config& c, std::vector<int64_t>& ids, std::vector<uint16_t>& w) {
  std::mt19937 gen(20260920u);
  std::vector<int> rank(c.E);
  std::iota(rank.begin(), rank.end(), 1);
  std::shuffle(rank.begin(), rank.end(), gen);
  std::normal_distribution<float> nd(0.f, 1.f);
  ids.resize(c.T * c.k);
  w.resize(c.T * c.k);
  std::vector<float> lg(c.E);
  std::vector<int> order(c.E);
  for (int64_t t = 0; t < c.T; ++t) {
    float mx = -INFINITY;
    for (int64_t e = 0; e < c.E; ++e) {
      lg[e] = 0.905f * nd(gen) - 1.1f * std::log(static_cast<float>(rank[e]));
      mx = std::max(mx, lg[e]);
    }
    double se = 0.0;
    for (int64_t e = 0; e < c.E; ++e) se += std::exp(static_cast<double>(lg[e] - mx));
    std::iota(order.begin(), order.end(), 0);
    std::partial_sort(order.begin(), order.begin() + c.k, order.end(),
                      [&](int a, int b) { return lg[a] > lg[b] || (lg[a] == lg[b] && a < b); });
    for (int64_t s = 0; s < c.k; ++s) {
      const int e = order[s];
      ids[t * c.k + s] = e;
      const float p = static_cast<float>(std::exp(static_cast<double>(lg[e] - mx)) / se);
      uint32_t u;
      memcpy(&u, &p, 4);
      w[t * c.k + s] = static_cast<uint16_t>((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
    }
  }
}

}  // namespace

int main(int argc, char** argv) {
  const char* name = argc > 1 ? argv[1] : "c4";
  Config c{};
  if (strcmp(name, "b32") == 0)
    c = {"b32", 2048, 60, 4, 1408, 5632, 32};
  else if (strcmp(name, "c4") == 0)
    c = {"c4", 2048, 60, 4, 1408, 5632, 512};
  else if (strcmp(name, "c5") == 0)
    c = {"c5", 2048, 128, 8, 768, 0, 256};
  else {
    fprintf(stderr, "usage: grouped_counters [b32|c4|c5] [instances>=1] [reps>=1]\n");
    return 2;
  }
  const int64_t G = 128;
  const bool routed_only = c.Is == 0;
  const size_t q4 = static_cast<size_t>(c.E) * c.I * c.H / 2, sc = static_cast<size_t>(c.E) * c.I * c.H / G;
  const size_t expert_bytes = 3 * (static_cast<size_t>(c.I) * c.H / 2 + static_cast<size_t>(c.I) * c.H / G * 4);
  const size_t dense_bytes = static_cast<size_t>(c.E) * c.H * 2 + (c.Is > 0 ? 3 * c.Is * c.H * 2 + c.H * 2 : 0);
  // >= 1.1 GB of weights over the rotated instances (the 256 MB MALL cannot
  // serve them), as bench.py rotates
  const int R_default = static_cast<int>(std::ceil(1.1e9 / static_cast<double>(c.E * expert_bytes + dense_bytes)));
  const int R = argc > 2 ? atoi(argv[2]) : std::max(2, R_default);
  const int reps = argc > 3 ? atoi(argv[3]) : 10;
  if (R < 1 || reps < 1) {
    fprintf(stderr, "instances and reps must be >= 1\n");
    return 2;
  }

  std::vector<uqm_layer_weights> layers(R);
  for (int r = 0; r < R; ++r) {
    uqm_layer_weights& L = layers[r];
    memset(&L, 0, sizeof(L));
    uint8_t* eg = device_alloc<uint8_t>(q4);
    uint8_t* eu = device_alloc<uint8_t>(q4);
    uint8_t* ed = device_alloc<uint8_t>(q4);
    float* s = device_alloc<float>(3 * sc);
    fill_bytes(eg, q4, 600 + r);
    fill_bytes(eu, q4, 700 + r);
    fill_bytes(ed, q4, 800 + r);
    fill_scales(s, 3 * sc);
    uint16_t* router = device_alloc<uint16_t>(c.E * c.H);
    fill_bf16(router, c.E * c.H, 100 + r);
    L.experts = {UQM_Q4, static_cast<int32_t>(G), c.E, c.H, c.I, eg, s, eu, s + sc, ed, s + 2 * sc};
    L.router = router;
    L.top_k = c.k;
    if (c.Is > 0) {
      uint16_t* seg = device_alloc<uint16_t>(c.H);
      uint16_t* sg = device_alloc<uint16_t>(c.Is * c.H);
      uint16_t* su = device_alloc<uint16_t>(c.Is * c.H);
      uint16_t* sd = device_alloc<uint16_t>(c.Is * c.H);
      fill_bf16(seg, c.H, 200 + r);
      fill_bf16(sg, c.Is * c.H, 300 + r);
      fill_bf16(su, c.Is * c.H, 400 + r);
      fill_bf16(sd, c.Is * c.H, 500 + r);
      L.has_shared = 1;
      L.shared_intermediate_size = c.Is;
      L.shared_gate = sg;
      L.shared_up = su;
      L.shared_down = sd;
      L.shared_expert_gate = seg;
    }
  }
  uint16_t* x = device_alloc<uint16_t>(c.T * c.H);
  fill_bf16(x, c.T * c.H, 7);
  uint16_t* out = device_alloc<uint16_t>(c.T * c.H);
  int64_t* idx = device_alloc<int64_t>(c.T * c.k);
  uint16_t* wts = device_alloc<uint16_t>(c.T * c.k);
  std::vector<int64_t> h_ids;
  std::vector<uint16_t> h_w;
  if (routed_only) {
    zipf_routes(c, h_ids, h_w);
    CHECK(hipMemcpy(idx, h_ids.data(), h_ids.size() * 8, hipMemcpyHostToDevice));
    CHECK(hipMemcpy(wts, h_w.data(), h_w.size() * 2, hipMemcpyHostToDevice));
  }
  const size_t ws_bytes = uqm_moe_workspace_bytes(c.T, c.H, c.I, c.Is, c.E, c.k);
  void* ws = device_alloc<char>(ws_bytes);
  CHECK(hipMemset(ws, 0, ws_bytes));
  CHECK(hipDeviceSynchronize());

  auto call = [&](int r) {
    if (routed_only)
      UQM(uqm_moe_forward(&layers[r].experts, x, c.T, idx, wts, c.k, out, ws, ws_bytes, nullptr));
    else
      UQM(uqm_moe_layer(&layers[r], x, c.T, out, nullptr, wts, idx, ws, ws_bytes, nullptr));
  };

  // distinct experts per call (the routes of the last instance; the router
  // weights of every instance come from the same generator)
  call(R - 1);
  CHECK(hipDeviceSynchronize());
  if (!routed_only) {
    h_ids.resize(c.T * c.k);
    CHECK(hipMemcpy(h_ids.data(), idx, h_ids.size() * 8, hipMemcpyDeviceToHost));
  }
  std::vector<int> count(c.E, 0);
  for (int64_t v : h_ids)
    if (v >= 0 && v < c.E) ++count[v];
  int active = 0, hot = 0, small = 0, maxc = 0;
  for (int v : count) {
    active += v > 0;
    hot += v > 100;
    small += v >= 1 && v <= 2;
    maxc = std::max(maxc, v);
  }
  const size_t algo_bytes = active * expert_bytes + dense_bytes - (routed_only ? c.E * c.H * 2 : 0);
  const double flops = 6.0 * c.H * c.I * c.T * c.k + 6.0 * c.H * c.Is * c.T + (routed_only ? 0.0 : 2.0 * c.H * c.E * c.T);

  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  for (int r = 0; r < R; ++r) call(r);
  CHECK(hipEventRecord(e0, nullptr));
  for (int i = 0; i < reps; ++i)
    for (int r = 0; r < R; ++r) call(r);
  CHECK(hipEventRecord(e1, nullptr));
  CHECK(hipEventSynchronize(e1));
  float ms = 0.f;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  const double us = 1000.0 * ms / (reps * R);
  printf("{\"config\": \"%s\", \"tokens\": %ld, \"instances\": %d, \"reps\": %d, \"us_per_call\": %.3f, "
         "\"algorithmic_bytes_per_call\": %zu, \"tb_per_s\": %.3f, \"flops_per_call\": %.4g, \"tflop_per_s\": %.2f, "
         "\"active_experts\": %d, \"experts_over_100_routes\": %d, \"experts_with_1_2_routes\": %d, "
         "\"max_routes\": %d}\n",
         c.name, static_cast<long>(c.T), R, reps, us, algo_bytes, algo_bytes / us / 1e6, flops, flops / us / 1e6, active,
         hot, small, maxc);
  return 0;
}
