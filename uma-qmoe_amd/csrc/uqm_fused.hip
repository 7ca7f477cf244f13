// Fused single-token MoE block for gfx950: one persistent launch per layer.
//
// A decode step of one MoE block reads ~88 MB of weights (Qwen1.5-MoE shape:
// 4 routed Q4 experts, the BF16 shared expert, the router) and does almost no
// arithmetic on them, so its time is HBM time plus every dependent memory
// round trip of the chain router -> top-k -> routed gate/up -> down that the
// streaming cannot hide. The reference runs this chain as ~12 launches with
// host syncs (src/uma_qmoe/native_backend.py:319-372; Transformers router and
// shared MLP around it, src/uma_qmoe/qwen_compressed_loader.py:67-86).
//
// Here one grid of 8-wave workgroups, one per CU, splits the CUs by role:
//
//   routed workgroups (the first `routed_blocks`, or all without a shared
//   expert) each compute the full router from the L2-resident router matrix
//   (no cross-CU hand-off for routing), run the FP32 softmax / top-k (ties to
//   the lower expert id) in LDS, then share the routed gate+up rows of the k
//   selected experts and afterwards the routed down rows, publishing
//   y_r[o] = sum_k w_k * (down_ek row o . h_k) per output row;
//   shared workgroups stream the shared expert's gate+up rows, then its down
//   rows, and write out[o] = bf16(sigmoid(x . w_g) * y_s[o] + y_r[o]).
//
// Measured on MI355X: HBM saturates with ~160 CUs streaming, so the shared
// stream keeps full bandwidth while the latency-bound routed chain runs on
// CUs whose memory queues hold no bulk traffic ahead of its loads.
//
// Hand-offs between CUs (SiLU products h, y_r) are epoch-tagged words
// written with agent-scope (sc1) stores, which are coherent across the eight
// XCD L2 caches. A consumer loads and validates them in one round trip and
// reloads until every tag carries this launch's epoch; there are no counter
// barriers and no store drains on the critical path. The epoch is a workspace
// word that every workgroup reads at start and the last workgroup to finish
// advances. Every wait is bounded: when a bound expires the kernel raises a
// sticky error word and still runs to the end, so no wave can hang the device.
// The waits need all workgroups resident at once: the grid is one 512-thread
// workgroup per CU.
//
// Within a role, work is split statically and evenly over its waves; each
// lane streams fixed 16-byte column chunks of every row (non-temporal loads:
// each weight byte is read once) against activation fragments held in
// registers. Loads are issued branch-free (out-of-row lanes re-read the row's
// first chunk and are masked in the arithmetic) and all row bookkeeping is
// wave-uniform, so every load of a batch is in flight before the first wait.
#include "uqm_internal.h"

// Phase-boundary trace hooks: no-ops here; a timing harness may define them
// (before including this file) to record per-wave timestamps. The INIT hook
// runs once at kernel entry.
#ifndef UQM_FUSED_TRACE
#define UQM_FUSED_TRACE(point)
#endif
#ifndef UQM_FUSED_TRACE_INIT
#define UQM_FUSED_TRACE_INIT
#endif

namespace uqm {

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

namespace {

// Load batches (rows per wave per round trip). Larger batches mean fewer
// dependent round trips; smaller ones keep less in flight, which keeps the
// HBM queue, and so every round trip behind it, short.
#ifndef UQM_FUSED_ROUTER_RB
#define UQM_FUSED_ROUTER_RB 8   // router rows
#endif
#ifndef UQM_FUSED_ROUTED_RB
#define UQM_FUSED_ROUTED_RB 8   // routed gate+up row pairs
#endif
#ifndef UQM_FUSED_SHARED_RB
#define UQM_FUSED_SHARED_RB 2   // shared gate+up row pairs
#endif

constexpr int kWaves = 8;                  // waves per workgroup
constexpr int kThreads = kWaves * 64;
constexpr int kRoutedLdsHeader = 2576;     // routed-role LDS before the SiLU products (16-byte aligned)
constexpr uint32_t kSpinLimit = 1u << 20;  // ~0.2 s of polling at s_sleep 8

__device__ __forceinline__ uint4 ld_stream(const uint8_t* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float ld_stream(const float* p) { return __builtin_nontemporal_load(p); }

template <typename T>
__device__ __forceinline__ T co_load(const T* p) {
  return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void co_store(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Completes every memory operation this wave issued.
__device__ __forceinline__ void drain() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

template <int V>
constexpr int log2_of() {
  int l = 0;
  while ((1 << l) < V) ++l;
  return l;
}

// ------------------------------------------------------- epoch tagging ----
// 32-bit word: bf16 value in the low half, 16-bit epoch in the high half.
__device__ __forceinline__ uint32_t tag16(uint32_t epoch, uint16_t v) { return (epoch << 16) | v; }
// 64-bit word: fp32 bits in the low half, epoch in the high half.
__device__ __forceinline__ uint64_t tag32(uint32_t epoch, float v) {
  return (static_cast<uint64_t>(epoch) << 32) | __float_as_uint(v);
}

// This lane's 16-byte column chunks of a row of C chunks: chunk lane + 64*j,
// clamped to chunk 0 beyond the row (the load stays inside the row and is
// coalesced with lane 0's), with a 0/1 mask and the offset of its scale.
template <int ENC, int CPL>
struct Cols {
  int c[CPL];
  int s[CPL];
  float m[CPL];
};

template <int ENC, int CPL>
__device__ __forceinline__ void make_cols(int C, int group, Cols<ENC, CPL>& cl) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    const bool ok = c < C;
    cl.c[j] = ok ? c : 0;
    cl.m[j] = ok ? 1.f : 0.f;
    cl.s[j] = Enc<ENC>::kScaled ? (cl.c[j] * Enc<ENC>::kElems) / group : 0;
  }
}

// Fragments of a BF16 activation row (global or LDS) for this lane's chunks.
template <int ENC, int CPL>
__device__ __forceinline__ void frags_from(const uint16_t* row, const Cols<ENC, CPL>& cl, XFrag<ENC> (&f)[CPL]) {
  using E = Enc<ENC>;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const uint16_t* src = row + static_cast<int64_t>(cl.c[j]) * E::kElems;
    uint32_t raw[E::kElems / 2];
#pragma unroll
    for (int q = 0; q < E::kElems / 8; ++q) {
      const uint4 v = *reinterpret_cast<const uint4*>(src + 8 * q);
      raw[4 * q] = v.x;
      raw[4 * q + 1] = v.y;
      raw[4 * q + 2] = v.z;
      raw[4 * q + 3] = v.w;
    }
    make_frag<ENC>(raw, f[j]);
  }
}

// One matrix row's 16-byte chunks at this lane's columns, plus their scales.
template <int ENC, int CPL>
struct RowLoad {
  uint4 w[CPL];
  float s[CPL];
};

// srow: scales of this row's first group (K % group == 0), ignored for BF16.
template <int ENC, int CPL>
__device__ __forceinline__ void issue_row(const uint8_t* row, const float* srow, const Cols<ENC, CPL>& cl,
                                          RowLoad<ENC, CPL>& r) {
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    r.w[j] = ld_stream(row + static_cast<int64_t>(cl.c[j]) * 16);
    if constexpr (Enc<ENC>::kScaled) r.s[j] = ld_stream(srow + cl.s[j]);
  }
}

template <int ENC, int CPL>
__device__ __forceinline__ float dot_row(const RowLoad<ENC, CPL>& r, const XFrag<ENC> (&f)[CPL],
                                         const Cols<ENC, CPL>& cl) {
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const float d = dot_chunk<ENC>(r.w[j], f[j]);
    acc = fmaf(d, Enc<ENC>::kScaled ? r.s[j] * cl.m[j] : cl.m[j], acc);
  }
  return acc;
}

__device__ __forceinline__ int lane_value(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }
__device__ __forceinline__ float lane_value(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Workgroup-cooperative copy of n epoch-tagged bf16 words into LDS. Reloads
// until every tag equals `epoch` (the producers' sc1 stores have landed).
__device__ void stage_tagged16(const uint32_t* src, int n, uint16_t* dst, uint32_t epoch, uint32_t* error) {
  const uint64_t* s64 = reinterpret_cast<const uint64_t*>(src);
  uint32_t* d32 = reinterpret_cast<uint32_t*>(dst);
  const int n2 = n / 2;
  for (uint32_t spins = 0;; ++spins) {
    int ok = 1;
    for (int i = threadIdx.x; i < n2; i += kThreads) {
      const uint64_t v = co_load(s64 + i);
      const uint32_t lo = static_cast<uint32_t>(v), hi = static_cast<uint32_t>(v >> 32);
      ok &= (lo >> 16) == epoch && (hi >> 16) == epoch;
      d32[i] = (lo & 0xFFFFu) | (hi << 16);
    }
    if (__syncthreads_and(ok)) return;
    if (spins > kSpinLimit) {
      if (threadIdx.x == 0) atomicOr(error, 1u);
      return;
    }
    __builtin_amdgcn_s_sleep(8);
  }
}

}  // namespace

// Template parameters: routed encoding; 16-byte chunks per lane for a BF16
// row of H (CH), an encoded row of H (CHR), an encoded row of I (CIR) and a
// BF16 row of Is (CIS, 0 without a shared expert); KMAX >= top_k.
template <int ENC, int CH, int CHR, int CIR, int CIS, int KMAX>
__global__ __launch_bounds__(kThreads) void moe_decode_fused_kernel(FusedArgs a) {
  using ER = Enc<ENC>;
  constexpr int CISX = CIS > 0 ? CIS : 1;  // array extent when there is no shared expert
  constexpr bool kShared = CIS > 0;
  extern __shared__ __align__(16) unsigned char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nb = static_cast<int>(gridDim.x);
  const int b = static_cast<int>(blockIdx.x);
  const int gw = b * kWaves + wave;  // for trace hooks
  (void)gw;
  UQM_FUSED_TRACE_INIT
  const int H = static_cast<int>(a.H), I = static_cast<int>(a.I), Is = static_cast<int>(a.Is);
  const int E = a.E, k = a.k;
  uint32_t* const sync = a.sync;
  uint32_t* const error = a.sync + kSyncError;
  const int group = ER::kScaled ? a.group : 1;
  const int nr = kShared ? a.routed_blocks : nb;  // routed workgroups

  uint32_t epoch = (co_load(sync + kSyncEpoch) + 1u) & 0xFFFFu;
  if (epoch == 0) epoch = 1;  // tag 0 never marks valid data (zero-filled workspace)
  epoch = static_cast<uint32_t>(uniform(static_cast<int>(epoch)));

  const int64_t rowH16 = static_cast<int64_t>(H) * 2, rowHR = static_cast<int64_t>(H) * ER::kBitsPerWeight / 8,
                rowIR = static_cast<int64_t>(I) * ER::kBitsPerWeight / 8, rowIS = static_cast<int64_t>(Is) * 2;
  const int hpg = H / group, ipg = I / group;  // scale groups per row

  Cols<kBF16, CH> colH16;
  make_cols<kBF16, CH>(H / 8, 1, colH16);
  XFrag<kBF16> xb[CH];
  frags_from<kBF16, CH>(a.x, colH16, xb);
  UQM_FUSED_TRACE(0);

  if (b < nr) {
    // =========================================================== routed role
    // LDS: logits [256] f32 | ranks [256] i32 | slots [64] i32 | slot weights [64] f32 |
    //      softmax max, sum | routed SiLU products [k, I] bf16
    float* lg = reinterpret_cast<float*>(lds);
    int* lrank = reinterpret_cast<int*>(lds + 1024);
    int* lslot = reinterpret_cast<int*>(lds + 2048);
    float* lsw = reinterpret_cast<float*>(lds + 2304);
    float* lstat = reinterpret_cast<float*>(lds + 2560);
    uint16_t* lhr = reinterpret_cast<uint16_t*>(lds + kRoutedLdsHeader);
    const int wr = nr * kWaves;      // routed waves
    const int rw = b * kWaves + wave;

    // Router: this workgroup computes every logit (the router rows come from
    // L2 after the first workgroup of each XCD has read them).
    constexpr int RBR = UQM_FUSED_ROUTER_RB;
    for (int r0 = wave * RBR; r0 < E; r0 += kWaves * RBR) {
      RowLoad<kBF16, CH> rl[RBR];
#pragma unroll
      for (int q = 0; q < RBR; ++q) {
        const int r = r0 + q < E ? r0 + q : r0;
        issue_row<kBF16, CH>(a.router + r * rowH16, nullptr, colH16, rl[q]);
      }
      float v[RBR];
#pragma unroll
      for (int q = 0; q < RBR; ++q) v[q] = dot_row<kBF16, CH>(rl[q], xb, colH16);
      const float sum = wave_multi_sum<RBR>(v);
      const int q = lane >> (6 - log2_of<RBR>());
      if ((lane & ((64 / RBR) - 1)) == 0 && r0 + q < E) lg[r0 + q] = round_bf16(sum);
    }
    if (threadIdx.x < 256) lrank[threadIdx.x] = 0;
    if (threadIdx.x < 64) {
      lslot[threadIdx.x] = 0;  // defined even if NaN logits leave a rank unused
      lsw[threadIdx.x] = 0.f;
    }
    __syncthreads();

    // Top-k by ranking, spread over the workgroup: rank(e) = #larger logits
    // + #equal logits with a lower id (ties go to the lower expert id). Item
    // (e, c) counts over the c-th eighth of the logits.
    for (int it = threadIdx.x; it < E * 8; it += kThreads) {
      const int e = it % E, c = it / E;
      const float le = lg[e];
      int cnt = 0;
      for (int j = c * E / 8; j < (c + 1) * E / 8; ++j) {
        const float lj = lg[j];
        cnt += static_cast<int>(lj > le) | (static_cast<int>(lj == le) & static_cast<int>(j < e));
      }
      if (cnt) atomicAdd(&lrank[e], cnt);
    }
    if (wave == 0) {  // FP32 softmax statistics
      float mx = -INFINITY;
      for (int e = lane; e < E; e += 64) mx = fmaxf(mx, lg[e]);
      mx = wave_max(mx);
      float se = 0.f;
      for (int e = lane; e < E; e += 64) se += __expf(lg[e] - mx);
      se = wave_sum(se);
      if (lane == 0) {
        lstat[0] = mx;
        lstat[1] = se;
      }
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += kThreads) {
      const int r = lrank[e];
      if (r < k) {
        lslot[r] = e;
        lsw[r] = __expf(lg[e] - lstat[0]) / lstat[1];
      }
    }
    __syncthreads();
    const int route_e = lane < k ? lslot[lane] : 0;
    float p = lane < k ? lsw[lane] : 0.f;
    if (a.norm) p = p / wave_sum(p);
    const uint16_t wb = f32_to_bf16(p);
    const float route_w = lane < k ? bf16_to_f32(wb) : 0.f;
    if (b == 0 && wave == 0) {
      if (lane < k) {
        if (a.weights_out != nullptr) a.weights_out[lane] = wb;
        if (a.indices_out != nullptr) a.indices_out[lane] = route_e;
      }
      if (a.logits_out != nullptr)
        for (int e = lane; e < E; e += 64) a.logits_out[e] = f32_to_bf16(lg[e]);
    }
    UQM_FUSED_TRACE(1);

    // Routed gate+up rows q = slot * I + i, split over the routed waves.
    {
      Cols<ENC, CHR> colHR;
      make_cols<ENC, CHR>(H / ER::kElems, group, colHR);
      XFrag<ENC> xr[CHR];
      frags_from<ENC, CHR>(a.x, colHR, xr);
      const int64_t spe = static_cast<int64_t>(I) * hpg;  // gate/up scales per expert
      const int nq = k * I;
      const int qa = uniform(static_cast<int>(static_cast<int64_t>(rw) * nq / wr));
      const int qb = uniform(static_cast<int>(static_cast<int64_t>(rw + 1) * nq / wr));
      constexpr int RB = UQM_FUSED_ROUTED_RB;
      int slot = qa / I;
      int row = qa - slot * I;
      for (int q0 = qa; q0 < qb; q0 += RB) {
        const int n = qb - q0 < RB ? qb - q0 : RB;
        RowLoad<ENC, CHR> rl[RB][2];
        const int first_slot = slot, first_row = row;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          const int sl = rb < n ? slot : first_slot;  // rows past the range re-read the first row
          const int i = rb < n ? row : first_row;
          const int64_t e = lane_value(route_e, sl);
          const int64_t grow = e * I + i;
          issue_row<ENC, CHR>(a.eg + grow * rowHR, a.egs + e * spe + static_cast<int64_t>(i) * hpg, colHR, rl[rb][0]);
          issue_row<ENC, CHR>(a.eu + grow * rowHR, a.eus + e * spe + static_cast<int64_t>(i) * hpg, colHR, rl[rb][1]);
          if (rb < n && ++row == I) {
            row = 0;
            ++slot;
          }
        }
        constexpr int V = 2 * RB;
        float v[V];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          v[2 * rb] = dot_row<ENC, CHR>(rl[rb][0], xr, colHR);
          v[2 * rb + 1] = dot_row<ENC, CHR>(rl[rb][1], xr, colHR);
        }
        const float sum = wave_multi_sum<V>(v);
        constexpr int kL = log2_of<V>();
        const float partner = xor_partner<64 / V>(sum);
        const int idx = lane >> (6 - kL);
        const bool writer = (lane & ((64 >> kL) - 1)) == 0 && (idx & 1) == 0;
        const int rb = idx >> 1;
        if (writer && rb < n)
          co_store<uint32_t>(a.hr + q0 + rb, tag16(epoch, f32_to_bf16(silu(round_bf16(sum)) * round_bf16(partner))));
      }
    }
    UQM_FUSED_TRACE(2);

    // Routed down rows: y_r[o] = sum_s w_s * (down_{e_s} row o . h_s).
    {
      Cols<ENC, CIR> colIR;
      make_cols<ENC, CIR>(I / ER::kElems, group, colIR);
      const int64_t spd = static_cast<int64_t>(H) * ipg;  // down scales per expert
      const int oa = uniform(static_cast<int>(static_cast<int64_t>(rw) * H / wr));
      const int ob = uniform(static_cast<int>(static_cast<int64_t>(rw + 1) * H / wr));
      // rows per batch: about 32 chunk loads per lane in flight
      constexpr int RB = KMAX * CIR <= 8 ? 4 : (KMAX * CIR <= 16 ? 2 : 1);
      RowLoad<ENC, CIR> rr[RB][KMAX];
      auto issue_rows = [&](int o0, int n) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          const int o = rb < n ? o0 + rb : o0;
#pragma unroll
          for (int s = 0; s < KMAX; ++s) {
            if (s < k) {
              const int64_t e = lane_value(route_e, s);
              issue_row<ENC, CIR>(a.ed + (e * H + o) * rowIR, a.eds + e * spd + static_cast<int64_t>(o) * ipg,
                                  colIR, rr[rb][s]);
            }
          }
        }
      };
      if (oa < ob) issue_rows(oa, ob - oa < RB ? ob - oa : RB);
      UQM_FUSED_TRACE(3);
      stage_tagged16(a.hr, k * I, lhr, epoch, error);
      UQM_FUSED_TRACE(4);
      for (int o0 = oa; o0 < ob; o0 += RB) {
        const int n = ob - o0 < RB ? ob - o0 : RB;
        if (o0 > oa) issue_rows(o0, n);
        float y[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) y[rb] = 0.f;
#pragma unroll
        for (int s = 0; s < KMAX; ++s) {
          if (s < k) {
            XFrag<ENC> fr[CIR];
            frags_from<ENC, CIR>(lhr + s * I, colIR, fr);
            float v[RB];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) v[rb] = dot_row<ENC, CIR>(rr[rb][s], fr, colIR);
            const float sum = wave_multi_sum<RB>(v);
            const float w = lane_value(route_w, s);
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) y[rb] = fmaf(w, lane_value(sum, rb * (64 / RB)), y[rb]);
          }
        }
        if (lane < n) {
          float yo = y[0];
#pragma unroll
          for (int rb = 1; rb < RB; ++rb)
            if (lane == rb) yo = y[rb];
          if constexpr (kShared)
            co_store<uint64_t>(a.yr + o0 + lane, tag32(epoch, yo));
          else
            a.out[o0 + lane] = f32_to_bf16(yo);
        }
      }
    }
    UQM_FUSED_TRACE(5);
  } else if constexpr (kShared) {
    // =========================================================== shared role
    uint16_t* lhs = reinterpret_cast<uint16_t*>(lds);  // [Is] shared SiLU product
    float* lsg = reinterpret_cast<float*>(lds + ((2 * static_cast<size_t>(Is) + 15) & ~static_cast<size_t>(15)));
    const int ws = (nb - nr) * kWaves;  // shared waves
    const int sw = (b - nr) * kWaves + wave;

    // Shared gate+up rows, two row pairs per load batch.
    {
      const int pa = uniform(static_cast<int>(static_cast<int64_t>(sw) * Is / ws));
      const int pb = uniform(static_cast<int>(static_cast<int64_t>(sw + 1) * Is / ws));
      constexpr int RB = UQM_FUSED_SHARED_RB;
      for (int r0 = pa; r0 < pb; r0 += RB) {
        const int n = pb - r0 < RB ? pb - r0 : RB;
        RowLoad<kBF16, CH> rl[RB][2];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          const int64_t r = rb < n ? r0 + rb : r0;  // rows past the range re-read row r0
          issue_row<kBF16, CH>(a.sg_w + r * rowH16, nullptr, colH16, rl[rb][0]);
          issue_row<kBF16, CH>(a.su_w + r * rowH16, nullptr, colH16, rl[rb][1]);
        }
        constexpr int V = 2 * RB;
        float v[V];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          v[2 * rb] = dot_row<kBF16, CH>(rl[rb][0], xb, colH16);
          v[2 * rb + 1] = dot_row<kBF16, CH>(rl[rb][1], xb, colH16);
        }
        const float sum = wave_multi_sum<V>(v);
        constexpr int kL = log2_of<V>();
        const float partner = xor_partner<64 / V>(sum);
        const int idx = lane >> (6 - kL);
        const bool writer = (lane & ((64 >> kL) - 1)) == 0 && (idx & 1) == 0;
        const int rb = idx >> 1;
        if (writer && rb < n)
          co_store<uint32_t>(a.hs + r0 + rb, tag16(epoch, f32_to_bf16(silu(round_bf16(sum)) * round_bf16(partner))));
      }
    }
    // Sigmoid of the shared-expert gate logit (one row, from L2).
    if (wave == 0) {
      RowLoad<kBF16, CH> rl;
      issue_row<kBF16, CH>(a.shared_expert_gate, nullptr, colH16, rl);
      const float g = wave_sum(dot_row<kBF16, CH>(rl, xb, colH16));
      if (lane == 0) *lsg = round_bf16(sigmoidf_(round_bf16(g)));
    }
    UQM_FUSED_TRACE(2);

    // Shared down rows and the combine with y_r.
    {
      Cols<kBF16, CISX> colIS;
      make_cols<kBF16, CISX>(Is / 8, 1, colIS);
      const int oa = uniform(static_cast<int>(static_cast<int64_t>(sw) * H / ws));
      const int ob = uniform(static_cast<int>(static_cast<int64_t>(sw + 1) * H / ws));
      RowLoad<kBF16, CISX> rs;
      if (oa < ob) issue_row<kBF16, CISX>(a.sd_w + oa * rowIS, nullptr, colIS, rs);
      UQM_FUSED_TRACE(3);
      stage_tagged16(a.hs, Is, lhs, epoch, error);
      UQM_FUSED_TRACE(4);
      const float sg = *lsg;
      for (int o = oa; o < ob; ++o) {
        if (o > oa) issue_row<kBF16, CISX>(a.sd_w + o * rowIS, nullptr, colIS, rs);
        XFrag<kBF16> fs[CISX];
        frags_from<kBF16, CISX>(lhs, colIS, fs);
        const float ys = wave_sum(dot_row<kBF16, CISX>(rs, fs, colIS));
        if (lane == 0) {
          uint64_t t = co_load(a.yr + o);
          for (uint32_t spins = 0; static_cast<uint32_t>(t >> 32) != epoch; ++spins) {
            if (spins > kSpinLimit) {
              atomicOr(error, 1u);
              break;
            }
            __builtin_amdgcn_s_sleep(8);
            t = co_load(a.yr + o);
          }
          a.out[o] = f32_to_bf16(fmaf(sg, ys, __uint_as_float(static_cast<uint32_t>(t))));
        }
      }
    }
    UQM_FUSED_TRACE(5);
  }

  // ---------------------------------------------------------------- finish
  drain();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t old = atomicAdd(sync + kSyncBlocksDone, 1u);
    if (old == static_cast<uint32_t>(nb - 1)) {
      co_store<uint32_t>(sync + kSyncEpoch, epoch);
      co_store<uint32_t>(sync + kSyncBlocksDone, 0u);
    }
  }
}

namespace {

int cpl(int64_t chunks) { return static_cast<int>((chunks + 63) / 64); }

size_t lds_bytes(const FusedArgs& a, int kmax) {
  const size_t routed = kRoutedLdsHeader + static_cast<size_t>(kmax) * a.I * 2;
  const size_t shared = ((2 * static_cast<size_t>(a.Is) + 15) & ~static_cast<size_t>(15)) + 16;
  return routed > shared ? routed : shared;
}

template <int ENC, int CH, int CHR, int CIR, int CIS, int KMAX>
hipError_t launch_cfg(const FusedArgs& args, int routed_blocks, hipStream_t stream) {
  auto kern = moe_decode_fused_kernel<ENC, CH, CHR, CIR, CIS, KMAX>;
  const size_t lds = lds_bytes(args, KMAX);
  if (lds > 64 * 1024) return hipErrorInvalidValue;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  int per_cu = 0, cus = 0;
  if ((e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kThreads, lds)) != hipSuccess) return e;
  if ((e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
  if (per_cu < 1 || cus < 2) return hipErrorInvalidConfiguration;
  FusedArgs a = args;
  const int blocks = cus;  // one workgroup per CU, all resident
  a.routed_blocks = CIS > 0 ? (routed_blocks > 0 && routed_blocks < blocks ? routed_blocks : blocks / 2) : blocks;
  hipLaunchKernelGGL(kern, dim3(blocks), dim3(kThreads), lds, stream, a);
  return hipGetLastError();
}

}  // namespace

int fused_config_id(int enc, int64_t H, int64_t I, int64_t Is, int64_t k) {
  // Per-lane chunk loops are masked, so an instantiation serves every shape
  // whose chunk counts per lane do not exceed its template arguments.
  const int el = enc == kQ4 ? 32 : enc == kQ8 ? 16 : 8;
  const int ch = cpl(H / 8), chr = cpl(H / el), cir = cpl(I / el), cis = Is > 0 ? cpl(Is / 8) : 0;
  if (k < 1 || k > 8 || ch > 4 || cis > 11) return -1;
  if (kRoutedLdsHeader + (k <= 4 ? 4 : 8) * I * 2 > 64 * 1024 || Is * 2 + 32 > 64 * 1024) return -1;
  if (enc == kQ4 && chr <= 1 && cir <= 1) return 0;
  if (enc == kQ8 && chr <= 2 && cir <= 2) return 1;
  if (enc == kBF16 && chr <= 4 && cir <= 3) return 2;
  return -1;
}

hipError_t launch_moe_decode_fused(int enc, const FusedArgs& a, int routed_blocks, hipStream_t stream) {
  if (fused_config_id(enc, a.H, a.I, a.Is, a.k) < 0) return hipErrorInvalidValue;
  const bool shared = a.Is > 0;
  const bool k4 = a.k <= 4;
#define UQM_FUSED(ENCV, CHR, CIR)                                                                 \
  if (shared) {                                                                                    \
    return k4 ? launch_cfg<ENCV, 4, CHR, CIR, 11, 4>(a, routed_blocks, stream)                     \
              : launch_cfg<ENCV, 4, CHR, CIR, 11, 8>(a, routed_blocks, stream);                    \
  }                                                                                                \
  return k4 ? launch_cfg<ENCV, 4, CHR, CIR, 0, 4>(a, routed_blocks, stream)                        \
            : launch_cfg<ENCV, 4, CHR, CIR, 0, 8>(a, routed_blocks, stream);
  if (enc == kQ4) {
    UQM_FUSED(kQ4, 1, 1)
  }
  if (enc == kQ8) {
    UQM_FUSED(kQ8, 2, 2)
  }
  UQM_FUSED(kBF16, 4, 3)
#undef UQM_FUSED
}

}  // namespace uqm
