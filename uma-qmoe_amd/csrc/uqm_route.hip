// Router top-k and token->expert permutation.
//
// Top-k replaces torch.topk in Transformers' Qwen2MoeTopKRouter.forward
// (models/qwen2_moe/modeling_qwen2_moe.py:330-336) with an explicit order:
// larger logit first, then lower expert id. Softmax is FP32 over the BF16
// logits; weights are cast to BF16 (optionally renormalised first).
//
// The permutation replaces the reference's argsort(stable)/bincount/cumsum
// (src/uma_qmoe/native_backend.py:530-543) with a stable counting sort: per
// 64-route chunk, eight wave ballots give every lane the mask of lanes holding
// the same expert id, so ranks come from one popcount and no comparison sort
// is needed (one workgroup up to 3072 routes, one wavefront beyond).
#include "uqm_route.h"

namespace uqm {

// Logit of column e: the bf16 value itself, or the bf16 rounding of the sum of
// the FP32 partials.
__device__ __forceinline__ float logit_of(const uint16_t* row, const float* prow, int parts, int64_t pstride, int e) {
  if (prow == nullptr) return bf16_to_f32(row[e]);
  float v = prow[e];
  for (int p = 1; p < parts; ++p) v += prow[p * pstride + e];
  return round_bf16(v);
}

// Top-k, softmax weights and shared-expert gate of token t, by one wavefront.
__device__ __forceinline__ void topk_token(int64_t t, int lane, const uint16_t* __restrict__ logits,
                                           const float* __restrict__ plog, int parts, int64_t pstride, int64_t ldl,
                                           int E, int k, int norm, uint16_t* __restrict__ weights_out,
                                           int64_t* __restrict__ indices_out, int32_t* __restrict__ route_expert,
                                           float* __restrict__ shared_gate, uint16_t* __restrict__ logits_out) {
  const uint16_t* row = plog != nullptr ? nullptr : logits + t * ldl;
  const float* prow = plog != nullptr ? plog + t * ldl : nullptr;

  // column E (the shared-expert gate logit) is loaded with the others, by
  // lane E % 64 (lane 0 when E = 256), so that the block has a single round
  // trip of loads
  float l[4];
  float gate = 0.f;
  if (shared_gate != nullptr && E >= 256 && lane == 0) gate = logit_of(row, prow, parts, pstride, E);
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = lane + 64 * i;
    const bool load = e < E || (shared_gate != nullptr && e == E);
    float v = load ? logit_of(row, prow, parts, pstride, e) : -INFINITY;
    if (e == E) {
      gate = v;
      v = -INFINITY;
    }
    l[i] = v;
    if (logits_out != nullptr && e < E) logits_out[t * E + e] = f32_to_bf16(v);
    mx = fmaxf(mx, v);
  }
  mx = wave_max(mx);
  float se = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (lane + 64 * i < E) se += __expf(l[i] - mx);
  se = wave_sum(se);

  // Top-k by k rounds of a wave max over (value key, 0xFFFF - id): the
  // largest logit wins, equal logits go to the lower expert id, NaN sorts
  // first (as in a descending torch.sort); the exchanges run on DPP and the
  // permlane swaps, not through LDS.
  uint32_t key[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = lane + 64 * i;
    key[i] = e < E ? (bf16_key(f32_to_bf16(l[i])) << 16) | static_cast<uint32_t>(0xFFFF - e) : 0u;
  }
  float my_v = 0.f;
  int my_e = -1;
  for (int s = 0; s < k; ++s) {
    uint32_t m = max(max(key[0], key[1]), max(key[2], key[3]));
    m = wave_max_u32(m);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (key[i] == m) key[i] = 0u;
    if (lane == s) {
      my_e = 0xFFFF - static_cast<int>(m & 0xFFFFu);
      my_v = bf16_of_key(m >> 16);
    }
  }
  float p = lane < k ? __expf(my_v - mx) / se : 0.f;
  if (norm) p = p / wave_sum(p);
  if (lane < k) {
    weights_out[t * k + lane] = f32_to_bf16(p);
    indices_out[t * k + lane] = my_e;
    // device-coherent store: the fused top-k + permutation launch reads the
    // ids back in another workgroup, possibly on another XCD
    if (route_expert != nullptr)
      __hip_atomic_store(route_expert + t * k + lane, my_e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (shared_gate != nullptr && lane == (E < 256 ? (E & 63) : 0)) shared_gate[t] = round_bf16(sigmoidf_(gate));
}

__global__ __launch_bounds__(256) void route_topk_kernel(const uint16_t* __restrict__ logits,
                                                         const float* __restrict__ plog, int parts, int64_t pstride,
                                                         int64_t ldl, int64_t T, int E, int k, int norm,
                                                         uint16_t* __restrict__ weights_out,
                                                         int64_t* __restrict__ indices_out,
                                                         int32_t* __restrict__ route_expert,
                                                         float* __restrict__ shared_gate,
                                                         uint16_t* __restrict__ logits_out) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + wave;
  if (t >= T) return;
  topk_token(t, lane, logits, plog, parts, pstride, ldl, E, k, norm, weights_out, indices_out, route_expert,
             shared_gate, logits_out);
}

hipError_t launch_route_topk(const uint16_t* logits, int64_t ldl, int64_t T, int64_t E, int64_t k, int norm,
                             uint16_t* weights_out, int64_t* indices_out, int32_t* route_expert,
                             float* shared_gate, hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((T + 3) / 4));
  hipLaunchKernelGGL(route_topk_kernel, grid, dim3(256), 0, stream, logits, nullptr, 1, int64_t{0}, ldl, T,
                     static_cast<int>(E), static_cast<int>(k), norm, weights_out, indices_out, route_expert,
                     shared_gate, nullptr);
  return hipGetLastError();
}

hipError_t launch_route_topk_partials(const float* plog, int parts, int64_t pstride, int64_t ldl, int64_t T,
                                      int64_t E, int64_t k, int norm, uint16_t* weights_out, int64_t* indices_out,
                                      int32_t* route_expert, float* shared_gate, uint16_t* logits_out,
                                      hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((T + 3) / 4));
  hipLaunchKernelGGL(route_topk_kernel, grid, dim3(256), 0, stream, nullptr, plog, parts, pstride, ldl, T,
                     static_cast<int>(E), static_cast<int>(k), norm, weights_out, indices_out, route_expert,
                     shared_gate, logits_out);
  return hipGetLastError();
}

// kCoherent: read route_expert with device-coherent loads (ids written by
// other workgroups of the same launch).
template <bool kCoherent = false>
__device__ __forceinline__ int load_route_id(const int32_t* route_expert, const int64_t* indices64, int64_t r,
                                             int64_t n, int E, bool& valid) {
  int64_t id = -1;
  if (r < n) {
    if (indices64 != nullptr)
      id = indices64[r];
    else if constexpr (kCoherent)
      id = __hip_atomic_load(const_cast<int32_t*>(route_expert) + r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
      id = route_expert[r];
  }
  valid = id >= 0 && id < E;
  return valid ? static_cast<int>(id) : 0;
}

// Per-expert tables from the counts cnt[0..255] (one wavefront): exclusive
// offsets into start[] (LDS) and expert_offsets[E+1], the route tiles (when
// tile_tokens > 0) and the compact list of experts that have routes.
__device__ void expert_tables(const int* cnt, int* start, int lane, int E, int32_t* __restrict__ expert_offsets,
                              int64_t* __restrict__ offsets64, int tile_tokens, int32_t* __restrict__ tiles,
                              int32_t* __restrict__ tile_count, int32_t* __restrict__ active_experts,
                              int32_t* __restrict__ active_count) {
  // Exclusive scan over 4 experts per lane.
  int c4[4];
  int local = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    c4[i] = cnt[4 * lane + i];
    local += c4[i];
  }
  int incl = local;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int v = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += v;
  }
  int pre = incl - local;
  if (tile_tokens > 0) {
    // Route tiles: ceil(count / tile_tokens) per expert, in ascending expert id.
    int nt4[4];
    int tl = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      nt4[i] = (c4[i] + tile_tokens - 1) / tile_tokens;
      tl += nt4[i];
    }
    int tincl = tl;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(tincl, o, kWave);
      if (lane >= o) tincl += v;
    }
    int tpos = tincl - tl;
    int first = pre;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      for (int j = 0; j < nt4[i]; ++j, ++tpos) {
        tiles[2 * tpos] = 4 * lane + i;
        tiles[2 * tpos + 1] = first + j * tile_tokens;
      }
      first += c4[i];
    }
    if (lane == 63) *tile_count = tincl;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = 4 * lane + i;
    if (e < E) {
      expert_offsets[e] = pre;
      if (offsets64 != nullptr) offsets64[e] = pre;
    }
    start[e] = pre;
    pre += c4[i];
  }
  const int total = __shfl(incl, 63, kWave);
  if (lane == 0) {
    expert_offsets[E] = total;
    if (offsets64 != nullptr) offsets64[E] = total;
  }
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int acc = 0;
  for (int e0 = 0; e0 < E; e0 += 64) {
    const int e = e0 + lane;
    const bool on = e < E && cnt[e] > 0;
    const uint64_t m = __ballot(on);
    if (on) active_experts[acc + __popcll(m & lt)] = e;
    acc += __popcll(m);
  }
  if (lane == 0) *active_count = acc;
}

// Mask of the lanes of this wavefront that hold the same expert id (valid
// ids only): one ballot per id bit.
__device__ __forceinline__ uint64_t same_id_lanes(int id, bool valid, int nbits) {
  uint64_t eq = __ballot(valid);
  for (int b = 0; b < nbits; ++b) {
    const bool bit = (id >> b) & 1;
    const uint64_t bal = __ballot(bit);
    eq &= bit ? bal : ~bal;
  }
  return eq;
}

// One wavefront; E <= 256. Any number of routes.
__global__ __launch_bounds__(64) void route_permute_kernel(const int32_t* __restrict__ route_expert,
                                                           const int64_t* __restrict__ indices64, int64_t n,
                                                           int E, int32_t* __restrict__ route_order,
                                                           int32_t* __restrict__ expert_offsets,
                                                           int32_t* __restrict__ active_experts,
                                                           int32_t* __restrict__ active_count,
                                                           int64_t* __restrict__ order64,
                                                           int64_t* __restrict__ offsets64, int tile_tokens,
                                                           int32_t* __restrict__ tiles,
                                                           int32_t* __restrict__ tile_count) {
  __shared__ int cnt[256];
  __shared__ int run[256];
  const int lane = threadIdx.x;
  for (int e = lane; e < 256; e += 64) cnt[e] = 0;
  __syncthreads();

  for (int64_t base = 0; base < n; base += 64) {
    bool valid;
    const int id = load_route_id(route_expert, indices64, base + lane, n, E, valid);
    if (valid) atomicAdd(&cnt[id], 1);
  }
  __syncthreads();
  expert_tables(cnt, run, lane, E, expert_offsets, offsets64, tile_tokens, tiles, tile_count, active_experts,
                active_count);
  __syncthreads();

  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int64_t base = 0; base < n; base += 64) {
    bool valid;
    const int id = load_route_id(route_expert, indices64, base + lane, n, E, valid);
    const uint64_t eq = same_id_lanes(id, valid, nbits);
    const int rank = __popcll(eq & lt);
    int start = 0;
    if (valid) start = run[id];
    __syncthreads();
    if (valid) {
      const int pos = start + rank;
      route_order[pos] = static_cast<int32_t>(base + lane);
      if (order64 != nullptr) order64[pos] = base + lane;
      if ((eq & lt) == 0) run[id] = start + __popcll(eq);
    }
    __syncthreads();
  }
}

// One workgroup of 16 wavefronts for up to kPermuteMaxRoutes routes: the
// routes are cut into 64-route chunks; every chunk's per-expert counts go to
// an LDS histogram (ballot matching gives each route its rank inside its
// chunk), a scan over the chunks per expert turns them into chunk bases, and
// each route lands at offset[e] + base[chunk][e] + rank. Same stable order
// as the one-wave kernel.
constexpr int kPermuteMaxRoutes = 3072;
constexpr int kPermuteWaves = 16;

// Body of the one-workgroup permutation (kPermuteWaves wavefronts).
template <bool kCoherent>
__device__ __forceinline__ void permute_wg(const int32_t* __restrict__ route_expert,
                                           const int64_t* __restrict__ indices64, int64_t n, int E,
                                           int32_t* __restrict__ route_order, int32_t* __restrict__ expert_offsets,
                                           int32_t* __restrict__ active_experts, int32_t* __restrict__ active_count,
                                           int64_t* __restrict__ order64, int64_t* __restrict__ offsets64,
                                           int tile_tokens, int32_t* __restrict__ tiles,
                                           int32_t* __restrict__ tile_count) {
  constexpr int kChunks = kPermuteMaxRoutes / 64;
  constexpr int kPer = kChunks / kPermuteWaves;  // chunks per wavefront
  // [chunk][expert] counts in dynamic LDS sized for the launch's chunks
  // (permute_lds_bytes), so a small permutation fits beside other kernels
  extern __shared__ int hist_dyn[];
  int (*hist)[256] = reinterpret_cast<int (*)[256]>(hist_dyn);
  __shared__ int cnt[256];
  __shared__ int start[256];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int nch = static_cast<int>((n + 63) / 64);
  for (int i = threadIdx.x; i < nch * 256; i += blockDim.x) (&hist[0][0])[i] = 0;
  __syncthreads();

  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int ids[kPer], ranks[kPer];
  bool oks[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int ch = wave + kPermuteWaves * j;
    oks[j] = false;
    ids[j] = 0;
    ranks[j] = 0;
    if (ch < nch) {  // uniform over the wavefront
      bool valid;
      const int id = load_route_id<kCoherent>(route_expert, indices64, static_cast<int64_t>(ch) * 64 + lane, n, E, valid);
      const uint64_t eq = same_id_lanes(id, valid, nbits);
      ids[j] = id;
      oks[j] = valid;
      ranks[j] = __popcll(eq & lt);
      if (valid && (eq & lt) == 0) hist[ch][id] = __popcll(eq);
    }
  }
  __syncthreads();
  // per expert: chunk bases (exclusive scan over the chunks) and the total
  for (int e = threadIdx.x; e < 256; e += blockDim.x) {
    int run = 0;
    for (int ch = 0; ch < nch; ++ch) {
      const int v = hist[ch][e];
      hist[ch][e] = run;
      run += v;
    }
    cnt[e] = e < E ? run : 0;
  }
  __syncthreads();
  if (wave == 0)
    expert_tables(cnt, start, lane, E, expert_offsets, offsets64, tile_tokens, tiles, tile_count, active_experts,
                  active_count);
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int ch = wave + kPermuteWaves * j;
    if (ch < nch && oks[j]) {
      const int pos = start[ids[j]] + hist[ch][ids[j]] + ranks[j];
      const int64_t r = static_cast<int64_t>(ch) * 64 + lane;
      route_order[pos] = static_cast<int32_t>(r);
      if (order64 != nullptr) order64[pos] = r;
    }
  }
}

// Dynamic LDS of permute_wg for n routes.
size_t permute_lds_bytes(int64_t n) { return static_cast<size_t>((n + 63) / 64) * 256 * sizeof(int); }

__global__ __launch_bounds__(64 * kPermuteWaves) void route_permute_wg_kernel(
    const int32_t* __restrict__ route_expert, const int64_t* __restrict__ indices64, int64_t n, int E,
    int32_t* __restrict__ route_order, int32_t* __restrict__ expert_offsets, int32_t* __restrict__ active_experts,
    int32_t* __restrict__ active_count, int64_t* __restrict__ order64, int64_t* __restrict__ offsets64,
    int tile_tokens, int32_t* __restrict__ tiles, int32_t* __restrict__ tile_count) {
  permute_wg<false>(route_expert, indices64, n, E, route_order, expert_offsets, active_experts, active_count, order64,
             offsets64, tile_tokens, tiles, tile_count);
}

// Top-k and permutation in one launch (up to kPermuteMaxRoutes routes): one
// token per wavefront. The route ids are written with device-coherent stores;
// once they have completed, every workgroup counts itself done on a
// device-scope counter, and the workgroup that arrives last reads the ids back
// with device-coherent loads, runs the permutation and resets the counter for
// the next launch. Nothing waits on another workgroup, and no cache is
// written back or invalidated.
__global__ __launch_bounds__(64 * kPermuteWaves) void route_topk_permute_kernel(
    const uint16_t* __restrict__ logits, const float* __restrict__ plog, int parts, int64_t pstride, int64_t ldl,
    int64_t T, int E, int k, int norm, uint16_t* __restrict__ weights_out, int64_t* __restrict__ indices_out,
    float* __restrict__ shared_gate, uint16_t* __restrict__ logits_out, RouteTables rt, int tile_tokens,
    uint32_t* __restrict__ counter) {
  __shared__ int s_last;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kPermuteWaves + wave;
  if (t < T)
    topk_token(t, lane, logits, plog, parts, pstride, ldl, E, k, norm, weights_out, indices_out, rt.route_expert,
               shared_gate, logits_out);
  __builtin_amdgcn_s_waitcnt(0);  // this wave's stores have completed
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t done = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = done == gridDim.x - 1 ? 1 : 0;
  }
  __syncthreads();
  if (s_last == 0) return;
  permute_wg<true>(rt.route_expert, nullptr, T * k, E, rt.route_order, rt.expert_offsets, rt.active_experts,
             rt.active_count, nullptr, nullptr, tile_tokens, rt.tiles, rt.tile_count);
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

bool route_topk_permute_fits(int64_t T, int64_t k) { return T > 0 && T * k <= kPermuteMaxRoutes; }

hipError_t launch_route_topk_permute(const uint16_t* logits, const float* plog, int parts, int64_t pstride,
                                     int64_t ldl, int64_t T, int64_t E, int64_t k, int norm, uint16_t* weights_out,
                                     int64_t* indices_out, float* shared_gate, uint16_t* logits_out,
                                     const RouteTables& rt, int tile_tokens, uint32_t* counter, hipStream_t stream) {
  if (!route_topk_permute_fits(T, k) || counter == nullptr) return hipErrorInvalidValue;
  if (tile_tokens > 0 && (rt.tiles == nullptr || rt.tile_count == nullptr)) return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>((T + kPermuteWaves - 1) / kPermuteWaves));
  hipLaunchKernelGGL(route_topk_permute_kernel, grid, dim3(64 * kPermuteWaves), permute_lds_bytes(T * k), stream,
                     logits, plog,
                     plog != nullptr ? parts : 1, pstride, ldl, T, static_cast<int>(E), static_cast<int>(k), norm,
                     weights_out, indices_out, shared_gate, logits_out, rt, tile_tokens, counter);
  return hipGetLastError();
}

hipError_t launch_route_permute(const int32_t* route_expert, const int64_t* indices64, int64_t n_routes,
                                int64_t E, const RouteTables& rt, int64_t* order64, int64_t* offsets64,
                                int tile_tokens, hipStream_t stream) {
  if (tile_tokens > 0 && (rt.tiles == nullptr || rt.tile_count == nullptr)) return hipErrorInvalidValue;
  if (n_routes > 64 && n_routes <= kPermuteMaxRoutes)
    hipLaunchKernelGGL(route_permute_wg_kernel, dim3(1), dim3(64 * kPermuteWaves), permute_lds_bytes(n_routes), stream,
                       route_expert, indices64,
                       n_routes, static_cast<int>(E), rt.route_order, rt.expert_offsets, rt.active_experts,
                       rt.active_count, order64, offsets64, tile_tokens, rt.tiles, rt.tile_count);
  else
    hipLaunchKernelGGL(route_permute_kernel, dim3(1), dim3(64), 0, stream, route_expert, indices64, n_routes,
                       static_cast<int>(E), rt.route_order, rt.expert_offsets, rt.active_experts, rt.active_count,
                       order64, offsets64, tile_tokens, rt.tiles, rt.tile_count);
  return hipGetLastError();
}

}  // namespace uqm
