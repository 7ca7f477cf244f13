// Fused single-token MoE block for gfx950: one persistent launch per layer.
//
// A decode step of one MoE block reads ~88 MB of weights (Qwen1.5-MoE shape:
// 4 routed Q4 experts, the BF16 shared expert, the router) and does almost no
// arithmetic on them, so its time is HBM time plus whatever part of the
// dependent chain router -> top-k -> routed gate/up -> down the streaming
// cannot hide. The reference runs this chain as ~12 launches with host syncs
// (src/uma_qmoe/native_backend.py:319-372; Transformers router and shared MLP
// around it, src/uma_qmoe/qwen_compressed_loader.py:67-86).
//
// One workgroup per CU, all resident, each with 8 streaming waves and one
// control wave. Every CU takes an equal share of every phase:
//
//   A  shared gate+up row pairs (no dependence on routing) -> SiLU products;
//   B  routed gate+up row pairs of the k selected experts -> SiLU products;
//   C  one or more output rows o: y_s[o] = shared down row o . h_s and
//      y_r[o] = sum_k w_k * (down_ek row o . h_k), summed in the same wave:
//      out[o] = bf16(sigmoid(x . w_g) * y_s[o] + y_r[o]).
//
// The routed-only ops pass their routes in (routes_in / weights_in): the
// control wave then loads the k ids and weights instead of routing.
//
// Routing runs beside phase A: the router rows (plus the shared expert's gate
// row) are spread over the workgroups, one row each, and published; the
// control wave of every workgroup polls the published logits, runs the
// softmax / top-k (ties to the lower expert id) in registers and hands the
// routes to its streaming waves through LDS. A streaming wave issues its
// phase-B loads when its phase A is done and the routes are in LDS, together
// with its phase-C shared down row, and all of its phase-C loads before it
// waits for the other CUs' SiLU products.
//
// Hand-offs between CUs (router logits, SiLU products) are epoch-tagged words
// written with agent-scope (sc1) stores, which are coherent across the eight
// XCD L2 caches. A consumer loads and validates them in one round trip and
// reloads until every tag carries this launch's epoch; there are no counter
// barriers and no store drains on the critical path. Each workgroup keeps its
// own copy of the epoch in the workspace and advances it once per launch.
// The waits need all workgroups resident at once (the grid is one workgroup
// per CU), and every wait is bounded by wall-clock time: each wave takes a
// deadline (s_memrealtime, kFusedWaitBudgetUs) at its start, shared by all
// of its waits. When one expires, the wave raises the sticky error word,
// records the launch's epoch in the expired word (the product waits of every
// other wave then give up at once) and runs to the end, so no wave can hang
// the device and a launch that lost its co-residency ends within the budget.
// Its result is poisoned, never silently wrong: routes taken from an
// incomplete logit poll make the workgroup publish NaN products, and a wave
// whose product staging expired writes NaN output rows (with routes -1 and
// weights NaN from workgroup 0 when its own poll expired). Every wave that
// gives up raises the error word; workgroup 0 removes expired markers of
// earlier launches at the end of each launch.
//
// Each lane streams fixed 16-byte column chunks of every row (non-temporal
// loads: each weight byte is read once) against activation fragments held in
// registers. Loads are issued branch-free (out-of-row lanes re-read the row's
// first chunk and are masked in the arithmetic) and all row bookkeeping is
// wave-uniform, so every load of a batch is in flight before the first wait.
#include <type_traits>

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

constexpr int kWaves = 8;                  // streaming waves per workgroup
constexpr int kThreads = (kWaves + 1) * 64;  // + the control wave
constexpr int kLdsHeader = 256;            // flags, routes, weights, shared gate (16-byte aligned)
constexpr uint16_t kBf16NaN = 0x7FC0;      // poison of products and outputs after an expired wait
// s_sleep units (64 clocks; s_sleep takes at most 127) before the first logit
// poll with a shared expert: one poll is in flight at a time and each is
// re-issued as soon as it returns incomplete (c2: 20.8-20.9 us per launch
// back to back with a first delay of 96-127, 21.1 with 160, 21.4 with 192,
// 22.1 with 40; three polls ~1 us apart from 64: 21.2-21.9)
constexpr int kPollDelay = 104;
// The same without a shared expert, where nothing streams while the routes
// are pending (c1: 15.7 us per launch back to back with a first delay of 40,
// 16.2 with 64, 16.7 with 12-24; three polls 20 apart from 24: 17.9-18.1).
constexpr int kPollDelayRoutedOnly = 40;
// Without a shared expert the routed products are staged right after a
// wave's own phase B, while other CUs are still publishing theirs: a first
// staging round that comes back incomplete costs a round trip. Waiting this
// many s_sleep units first (the routed down rows already in flight) lets it
// complete (c1 in bench.py: 14.66 vs 15.22 us per call; 8: 14.90, 16: 14.71,
// 32: 14.76, 64: 15.55).
constexpr int kProductDelayRoutedOnly = 24;
constexpr int kRouterHeadStart = 12;       // s_sleep units the streaming waves of router workgroups yield
enum { kNormNone = 0, kNormUnit = 1, kNormWeighted = 2 };  // input RMSNorm: none, weight ones, weight row
#ifndef UQM_FUSED_CTRL_PRIO
#define UQM_FUSED_CTRL_PRIO 3
#endif

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

// Constant-rate wall clock (hipDeviceAttributeWallClockRate ticks).
__device__ __forceinline__ uint64_t wall_clock() { return __builtin_amdgcn_s_memrealtime(); }

// A wait of this wave expired: raise the sticky error word and mark the
// launch (epoch) as expired, ordered before anything the workgroup publishes
// afterwards.
__device__ __forceinline__ void raise_expired(uint32_t* sync, uint32_t epoch) {
  if ((threadIdx.x & 63) == 0) {
    atomicOr(sync + kSyncError, 1u);
    co_store<uint32_t>(sync + kSyncExpired, epoch);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
}

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
// Chunk and mask are recomputed at each use (two VALU ops) rather than held
// in registers; scale offsets (a division) are kept for scaled encodings.
template <int ENC, int CPL>
struct Cols {
  int C, ln;
  bool full;  // C == 64 * CPL (wave-uniform): no chunk is clamped or masked
  int sc[Enc<ENC>::kScaled ? CPL : 1];
  __device__ __forceinline__ int c(int j) const {
    const int v = ln + 64 * j;
    return full || v < C ? v : 0;
  }
  __device__ __forceinline__ float m(int j) const { return full || ln + 64 * j < C ? 1.f : 0.f; }
  __device__ __forceinline__ int s(int j) const {
    if constexpr (Enc<ENC>::kScaled) return sc[j];
    return 0;
  }
};

// Lane id the compiler cannot merge with threadIdx-derived values: column
// offsets built from it for a rarely taken loop are recomputed there instead
// of being kept live (in registers) from the first use.
__device__ __forceinline__ int opaque_lane() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// A zero the compiler treats as per-lane: a load from `p + opaque_zero()` is
// not copied to a scalar register right after issue, so the wave waits for it
// only where the value is used.
__device__ __forceinline__ int opaque_zero() {
  int z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  return z;
}

// Returns v, but only once `dep` has been computed: keeps the compiler from
// hoisting a use of a loaded value (and the wait for its load) above `dep`.
__device__ __forceinline__ uint32_t pinned_after(uint32_t v, float dep) {
  asm volatile("" : "+v"(v) : "v"(dep));
  return v;
}

template <int ENC, int CPL>
__device__ __forceinline__ void make_cols(int C, int group, Cols<ENC, CPL>& cl, int ln = -1) {
  cl.C = C;
  cl.full = C == 64 * CPL;
  cl.ln = ln >= 0 ? ln : static_cast<int>(threadIdx.x & 63);
  if constexpr (Enc<ENC>::kScaled) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) cl.sc[j] = (cl.c(j) * Enc<ENC>::kElems) / group;
  }
}

// A BF16 activation row's raw words at this lane's chunks (global or LDS),
// and the fragments built from them. Split so that a wave can issue the raw
// loads early and build the fragments after issuing its weight loads.
template <int ENC, int CPL>
struct XRaw {
  uint32_t w[CPL][Enc<ENC>::kElems / 2];
};

template <int ENC, int CPL>
__device__ __forceinline__ void load_x(const uint16_t* row, const Cols<ENC, CPL>& cl, XRaw<ENC, CPL>& r) {
  using E = Enc<ENC>;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const uint16_t* src = row + static_cast<uint32_t>(cl.c(j) * E::kElems);
#pragma unroll
    for (int q = 0; q < E::kElems / 8; ++q) {
      const uint4 v = *reinterpret_cast<const uint4*>(src + 8 * q);
      r.w[j][4 * q] = v.x;
      r.w[j][4 * q + 1] = v.y;
      r.w[j][4 * q + 2] = v.z;
      r.w[j][4 * q + 3] = v.w;
    }
  }
}

template <int ENC, int CPL>
__device__ __forceinline__ void frags_of(const XRaw<ENC, CPL>& r, XFrag<ENC> (&f)[CPL]) {
#pragma unroll
  for (int j = 0; j < CPL; ++j) make_frag<ENC>(r.w[j], f[j]);
}

template <int ENC, int CPL>
__device__ __forceinline__ void frags_from(const uint16_t* row, const Cols<ENC, CPL>& cl, XFrag<ENC> (&f)[CPL]) {
  XRaw<ENC, CPL> r;
  load_x<ENC, CPL>(row, cl, r);
  frags_of<ENC, CPL>(r, f);
}

// Input RMSNorm folded into the activation staging (Transformers
// Qwen2MoeRMSNorm, modeling_qwen2_moe.py:65-70):
//   x' = bf16(w * bf16(x * rsqrt(mean(x^2) + eps))), w = 1 without a weight.
// The FP32 sum of squares is taken over the row in the 8-element chunk layout
// (chunk lane + 64 j) in one fixed order, so that every wave of every
// workgroup derives the same scale whatever layout it stages x in.
template <int CPL>
__device__ __forceinline__ float rms_scale(const XRaw<kBF16, CPL>& r, const Cols<kBF16, CPL>& cl, int64_t H,
                                           float eps) {
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    float sj = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float lo = __uint_as_float(r.w[j][q] << 16), hi = __uint_as_float(r.w[j][q] & 0xFFFF0000u);
      sj = fmaf(lo, lo, sj);
      sj = fmaf(hi, hi, sj);
    }
    s += cl.m(j) * sj;
  }
  return rsqrtf(wave_sum(s) / static_cast<float>(H) + eps);
}

// A staged row normalised in place: x' = bf16(x * scale), then, with a
// weight row w staged in the same layout, x' = bf16(w * x').
template <int ENC, int CPL>
__device__ __forceinline__ void rms_row(XRaw<ENC, CPL>& r, float scale) {
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
#pragma unroll
    for (int q = 0; q < Enc<ENC>::kElems / 2; ++q) {
      const uint32_t v = r.w[j][q];
      r.w[j][q] = pack_bf16x2(__uint_as_float(v << 16) * scale, __uint_as_float(v & 0xFFFF0000u) * scale);
    }
  }
}
template <int ENC, int CPL>
__device__ __forceinline__ void rms_row(XRaw<ENC, CPL>& r, float scale, const XRaw<ENC, CPL>& w) {
  rms_row<ENC, CPL>(r, scale);
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
#pragma unroll
    for (int q = 0; q < Enc<ENC>::kElems / 2; ++q) {
      const uint32_t n = r.w[j][q], m = w.w[j][q];
      r.w[j][q] = pack_bf16x2(__uint_as_float(n << 16) * __uint_as_float(m << 16),
                              __uint_as_float(n & 0xFFFF0000u) * __uint_as_float(m & 0xFFFF0000u));
    }
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
    // 32-bit lane offsets from a uniform row address (the SGPR-base form)
    r.w[j] = ld_stream(row + static_cast<uint32_t>(cl.c(j) * 16));
    if constexpr (Enc<ENC>::kScaled) r.s[j] = ld_stream(srow + static_cast<uint32_t>(cl.s(j)));
  }
}

template <int ENC, int CPL>
__device__ __forceinline__ float dot_row(const RowLoad<ENC, CPL>& r, const XFrag<ENC> (&f)[CPL],
                                         const Cols<ENC, CPL>& cl) {
  float acc = 0.f;
  if (cl.full && !Enc<ENC>::kScaled) {  // unscaled rows filling every lane: plain sum
#pragma unroll
    for (int j = 0; j < CPL; ++j) acc += dot_chunk<ENC>(r.w[j], f[j]);
    return acc;
  }
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const float d = dot_chunk<ENC>(r.w[j], f[j]);
    acc = fmaf(d, Enc<ENC>::kScaled ? r.s[j] * cl.m(j) : cl.m(j), acc);
  }
  return acc;
}

__device__ __forceinline__ int lane_value(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }
__device__ __forceinline__ float lane_value(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Bare workgroup barrier: completes this wave's LDS operations first, but
// leaves its outstanding global loads in flight (a streaming wave can hold a
// whole batch of weight rows across it).
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt, expcnt unconstrained
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// [lo, hi) of n items split evenly over `parts`.
// (part * n must fit in 32 bits: parts <= 8192 waves, n <= 2^18.)
__device__ __forceinline__ int split_at(int n, int part, int parts) {
  return uniform(static_cast<int>(static_cast<uint32_t>(part) * static_cast<uint32_t>(n) / static_cast<uint32_t>(parts)));
}

}  // namespace

// LDS of one workgroup: header | shared SiLU products [Is] bf16 | routed SiLU
// products [k, I] bf16 | routed fragments [k * CR][kXWords] u32 | their offset
// terms [k * CR] f32, where CR = I / elems is the chunk count of a routed row.
template <int ENC>
size_t fused_lds_bytes(int64_t I, int64_t Is, int64_t k) {
  const int64_t jobs = k * (I / Enc<ENC>::kElems);
  return kLdsHeader + 2 * static_cast<size_t>(Is + k * I) + static_cast<size_t>(jobs) * (4 * Enc<ENC>::kXWords + 4);
}

// Template parameters: routed encoding; 16-byte chunks per lane for a BF16
// row of H (CH), an encoded row of H (CHR), an encoded row of I (CIR) and a
// BF16 row of Is (CIS, 0 without a shared expert); KMAX >= top_k.
template <int ENC, int CH, int CHR, int CIR, int CIS, int KMAX, int NORM>
__global__ __launch_bounds__(kThreads) void moe_decode_fused_kernel(FusedArgs a) {
  using ER = Enc<ENC>;
  constexpr bool RMS = NORM != kNormNone;         // the block's input is RMSNorm(x)
  constexpr bool kWeighted = NORM == kNormWeighted;  // ... with a weight row (else ones)
  constexpr int CISX = CIS > 0 ? CIS : 1;  // array extent when there is no shared expert
  constexpr bool kShared = CIS > 0;
  // Routed gate+up row pairs per load batch (the most a wave takes at the
  // shapes served: 5632 pairs / 2048 waves with a shared expert, 8192 / 2048
  // without; BF16 rows, 4 KB each, two pairs), and their value count rounded
  // up to a power of two. Each batch is one round trip.
  constexpr int RBP = CHR == 1 ? (kShared ? 3 : 4) : (CHR == 2 ? 3 : 2);
  constexpr int VB = RBP == 3 ? 8 : 2 * RBP;
  // Routed down chunks per lane: the k rows of an output row are flattened
  // over the wave's lanes (k * CR chunks).
  constexpr int NJ = KMAX * CIR;
  // 64-bit tag loads per lane per staging round: one round covers 3072 pairs
  // (6144 products: the shared or the routed products of c2) with a shared
  // expert, 4096 pairs without (the routed products of c1).
  constexpr int SL = kShared ? 6 : 8;
  constexpr int LPL = 5;  // router logits per lane: E + 1 <= 320
  extern __shared__ __align__(16) unsigned char lds[];
  const int H = static_cast<int>(a.H), I = static_cast<int>(a.I), Is = kShared ? static_cast<int>(a.Is) : 0;
  const int E = a.E, k = a.k;
  const int CR = I / ER::kElems;  // chunks per routed down row
  const int jobs = k * CR;
  int* l_route = reinterpret_cast<int*>(lds);
  float* l_w = reinterpret_cast<float*>(lds + 32);
  float* l_sg = reinterpret_cast<float*>(lds + 64);
  int* l_bad = reinterpret_cast<int*>(lds + 96);     // routes came from an expired logit poll
  int* l_stale = reinterpret_cast<int*>(lds + 100);  // a product staging wait expired
  uint16_t* lhs = reinterpret_cast<uint16_t*>(lds + kLdsHeader);
  uint16_t* lhr = lhs + Is;
  uint32_t* lfr = reinterpret_cast<uint32_t*>(lds + kLdsHeader + 2 * (Is + k * I));
  float* loff = reinterpret_cast<float*>(lfr + jobs * ER::kXWords);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nb = static_cast<int>(gridDim.x);
  const int b = static_cast<int>(blockIdx.x);
  const int gw = b * (kWaves + 1) + wave;  // for trace hooks
  (void)gw;
  UQM_FUSED_TRACE_INIT
  UQM_FUSED_TRACE(0);
  const uint64_t deadline = wall_clock() + a.wait_ticks;
  // A zero budget (a host option for tests of the poisoning path) makes every
  // wait give up at its first check, ready or not, so that each launch takes
  // the expired path on every workgroup and still ends normally.
  const bool force_expiry = a.wait_ticks == 0;
  uint32_t* const my_epoch = a.sync + kSyncEpochBase + b;
  const int group = ER::kScaled ? a.group : 1;
  const int nrow = E + (kShared ? 1 : 0);  // router rows + the shared-expert gate row

  // Every workgroup keeps its own copy of the launch epoch and advances it
  // once per launch, so all copies agree without any cross-workgroup atomic.
  // Tag 0 never marks valid data (zero-filled workspace).
  // (Kept per lane, not made uniform: a uniform copy would make the wave
  // wait for the load at the copy.)
  auto next_epoch = [](uint32_t last) {
    const uint32_t e = (last + 1u) & 0xFFFFu;
    return e == 0 ? 1u : e;
  };

  const int64_t rowH16 = static_cast<int64_t>(H) * 2, rowHR = static_cast<int64_t>(H) * ER::kBitsPerWeight / 8,
                rowIR = static_cast<int64_t>(I) * ER::kBitsPerWeight / 8, rowIS = static_cast<int64_t>(Is) * 2;
  const int hpg = H / group, ipg = I / group;  // scale groups per row

  Cols<kBF16, CH> colH16;
  make_cols<kBF16, CH>(H / 8, 1, colH16);

  // Builds the routed fragments (once per workgroup, from the staged routed
  // products): every wave takes part, between the staging and the final
  // barrier.
  auto build_fragments = [&]() {
    for (int jb = threadIdx.x; jb < jobs; jb += kThreads) {
      const int s = jb / CR, c = jb - s * CR;
      const uint16_t* src = lhr + s * I + c * ER::kElems;
      uint32_t raw[ER::kElems / 2];
#pragma unroll
      for (int q = 0; q < ER::kElems / 8; ++q) {
        const uint4 v = *reinterpret_cast<const uint4*>(src + 8 * q);
        raw[4 * q] = v.x;
        raw[4 * q + 1] = v.y;
        raw[4 * q + 2] = v.z;
        raw[4 * q + 3] = v.w;
      }
      XFrag<ENC> f;
      make_frag<ENC>(raw, f);
#pragma unroll
      for (int q = 0; q < ER::kXWords / 4; ++q)
        *reinterpret_cast<uint4*>(lfr + jb * ER::kXWords + 4 * q) =
            make_uint4(f.w[4 * q], f.w[4 * q + 1], f.w[4 * q + 2], f.w[4 * q + 3]);
      loff[jb] = f.off;
    }
  };

  if (wave == kWaves) {
    // ========================================================= control wave
    // Routing is on every wave's critical path: its instructions go first
    // when it shares a SIMD with streaming waves.
    __builtin_amdgcn_s_setprio(UQM_FUSED_CTRL_PRIO);
    // After the routes are in LDS: the workgroup's barriers, the routed
    // fragments, and the epoch advanced for the next launch. `late` runs
    // while the streaming waves issue their phase-B loads.
    auto finish_control = [&](uint32_t epoch, auto late) {
      UQM_FUSED_TRACE(3);
      lds_barrier();  // routes ready
      late();
      lds_barrier();  // routed gate/up rows issued
      lds_barrier();  // shared products staged
      lds_barrier();  // routed products staged
      build_fragments();
      lds_barrier();  // routed fragments built
      if (lane == 0) co_store<uint32_t>(my_epoch, epoch);
      // An expired marker left by an earlier launch is taken out (it would
      // otherwise make the waits of the launch that reaches the same 16-bit
      // epoch again give up at once). The marker of this launch stays: the
      // compare-and-swap cannot remove a value stored after the load.
      if (b == 0 && lane == 0) {
        const uint32_t old = co_load(a.sync + kSyncExpired);
        if (old != 0u && old != epoch) atomicCAS(a.sync + kSyncExpired, old, 0u);
      }
    };
    if (a.routes_in != nullptr) {
      // Routes given by the caller (the routed-only ops, no shared expert):
      // no router and no logit poll. An id outside [0, E) contributes
      // nothing (weight 0, expert 0 read in its place).
      const uint32_t last_epoch = co_load(my_epoch + opaque_zero());
      if (lane < k) {
        const int64_t r = a.routes_in[lane];
        const bool ok = r >= 0 && r < E;
        l_route[lane] = ok ? static_cast<int>(r) : 0;
        l_w[lane] = ok ? bf16_to_f32(a.weights_in[lane]) : 0.f;
      }
      if (lane == 0) {
        *l_bad = 0;
        *l_stale = 0;
      }
      finish_control(next_epoch(last_epoch), [] {});
      return;
    }
    // Activation, epoch and router row loads go out together: one round trip.
    XRaw<kBF16, CH> x_raw, w_raw;
    load_x<kBF16, CH>(a.x, colH16, x_raw);
    if constexpr (kWeighted) load_x<kBF16, CH>(a.rms_w, colH16, w_raw);
    const uint32_t last_epoch = co_load(my_epoch + opaque_zero());
    bool normed = !RMS;
    for (int r = b; r < nrow; r += nb) {
      RowLoad<kBF16, CH> rl;
      issue_row<kBF16, CH>(r < E ? a.router + r * rowH16 : a.shared_expert_gate, nullptr, colH16, rl);
      if constexpr (RMS) {
        if (!normed) {  // with the first row in flight
          const float scale = rms_scale<CH>(x_raw, colH16, H, a.rms_eps);
          if constexpr (kWeighted)
            rms_row<kBF16, CH>(x_raw, scale, w_raw);
          else
            rms_row<kBF16, CH>(x_raw, scale);
          normed = true;
        }
      }
      XFrag<kBF16> xb[CH];
      frags_of<kBF16, CH>(x_raw, xb);
      const float g = wave_sum(dot_row<kBF16, CH>(rl, xb, colH16));
      if (lane == 0) co_store<uint64_t>(a.lgt + r, tag32(next_epoch(pinned_after(last_epoch, g)), round_bf16(g)));
    }
    const uint32_t epoch = next_epoch(last_epoch);
    UQM_FUSED_TRACE(1);
    // Every logit, once all its producers have published it: one poll in
    // flight, re-issued as soon as it comes back incomplete. (With several
    // polls in flight, the one that finds every logit is followed by a wait
    // for the later ones: the compiler reuses their registers for what comes
    // next, and a register with a load outstanding waits for it first, up
    // to a round trip.) Every poll issues the same loads (lanes past the end
    // re-read the last word).
    float lv[LPL];
    bool bad = false;
    if constexpr (kShared) {
      uint64_t pa[LPL];
      auto poll = [&](uint64_t (&t)[LPL]) {
#pragma unroll
        for (int j = 0; j < LPL; ++j) t[j] = co_load(a.lgt + min(lane + 64 * j, nrow - 1));
      };
      auto ready = [&](const uint64_t (&t)[LPL]) {
        bool ok = true;
#pragma unroll
        for (int j = 0; j < LPL; ++j) ok &= static_cast<uint32_t>(t[j] >> 32) == epoch || lane + 64 * j >= nrow;
        return __all(ok) != 0;
      };
      auto take = [&](const uint64_t (&t)[LPL]) {
#pragma unroll
        for (int j = 0; j < LPL; ++j) lv[j] = __uint_as_float(static_cast<uint32_t>(t[j]));
      };
      __builtin_amdgcn_s_sleep(kPollDelay);
      poll(pa);
      for (;;) {
        if (!force_expiry && ready(pa)) {
          take(pa);
          break;
        }
        if (wall_clock() > deadline) {
          raise_expired(a.sync, epoch);
          bad = true;
          take(pa);
          break;
        }
        poll(pa);
      }
    } else {
      // Without a shared expert: one load per lane when the rows fit in one
      // (E <= 64), else LPL. (Written separately from the shared-expert case
      // above: folding both into one routine changed the c2 kernel's code and
      // cost it 0.4 us per call.)
      auto poll_logits = [&](auto loads) {
        constexpr int L = decltype(loads)::value;
        uint64_t pa[L];
        auto poll = [&](uint64_t (&t)[L]) {
#pragma unroll
          for (int j = 0; j < L; ++j) t[j] = co_load(a.lgt + min(lane + 64 * j, nrow - 1));
        };
        auto ready = [&](const uint64_t (&t)[L]) {
          bool ok = true;
#pragma unroll
          for (int j = 0; j < L; ++j) ok &= static_cast<uint32_t>(t[j] >> 32) == epoch || lane + 64 * j >= nrow;
          return __all(ok) != 0;
        };
        auto take = [&](const uint64_t (&t)[L]) {
#pragma unroll
          for (int j = 0; j < LPL; ++j) lv[j] = j < L ? __uint_as_float(static_cast<uint32_t>(t[j < L ? j : 0])) : 0.f;
        };
        __builtin_amdgcn_s_sleep(kPollDelayRoutedOnly);
        poll(pa);
        for (;;) {
          if (!force_expiry && ready(pa)) {
            take(pa);
            break;
          }
          if (wall_clock() > deadline) {
            raise_expired(a.sync, epoch);
            bad = true;
            take(pa);
            break;
          }
          poll(pa);
        }
      };
      if (nrow <= 64)
        poll_logits(std::integral_constant<int, 1>{});
      else
        poll_logits(std::integral_constant<int, LPL>{});
    }
    UQM_FUSED_TRACE(2);
    // Top-k by k rounds of a wave max over (value key, 0xFFFF - id): the
    // largest logit wins, equal logits go to the lower expert id, NaN first
    // (as in a descending sort). The logits are bf16 values, so a key comes
    // straight from their upper 16 bits, without branches.
    uint32_t key[LPL];
#pragma unroll
    for (int j = 0; j < LPL; ++j) {
      const int e = lane + 64 * j;
      const uint32_t kv = (bf16_key_select(__float_as_uint(lv[j]) >> 16) << 16) | static_cast<uint32_t>(0xFFFF - e);
      key[j] = e < E ? kv : 0u;
    }
    int route_e = 0;
    float route_l = 0.f;
    for (int s = 0; s < k; ++s) {
      uint32_t m = key[0];
#pragma unroll
      for (int j = 1; j < LPL; ++j) m = max(m, key[j]);
      m = wave_max_u32(m);
#pragma unroll
      for (int j = 0; j < LPL; ++j)
        if (key[j] == m) key[j] = 0u;
      if (lane == s) {
        route_e = 0xFFFF - static_cast<int>(m & 0xFFFFu);
        route_l = bf16_of_key(m >> 16);
      }
    }
    if (lane < k) l_route[lane] = route_e;
    if (lane == 0) {
      *l_bad = bad ? 1 : 0;
      *l_stale = 0;
    }
    // FP32 softmax over the E expert logits at the k selected ones, the
    // shared gate, and workgroup 0's outputs: only phase C reads them.
    // Without a shared expert they are computed while the streaming waves
    // issue their phase-B loads (c1 15.2 vs 15.5 us per call); with one,
    // before the routes go out (there the later placement measured slower,
    // 20.41 vs 20.28 us).
    auto weights = [&]() {
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < LPL; ++j)
        if (lane + 64 * j < E) mx = fmaxf(mx, lv[j]);
      mx = wave_max(mx);
      float se = 0.f;
#pragma unroll
      for (int j = 0; j < LPL; ++j)
        if (lane + 64 * j < E) se += __expf(lv[j] - mx);
      se = wave_sum(se);
      float p = lane < k ? __expf(route_l - mx) / se : 0.f;
      if (a.norm) p = p / wave_sum(p);
      const uint16_t wb = bad ? kBf16NaN : f32_to_bf16(p);
      if (lane < k) l_w[lane] = bf16_to_f32(wb);
      if constexpr (kShared) {
        float le = 0.f;
#pragma unroll
        for (int j = 0; j < LPL; ++j)
          if (j == (E >> 6)) le = lv[j];
        const float gl = lane_value(le, E & 63);
        if (lane == 0) *l_sg = round_bf16(sigmoidf_(gl));
      }
      if (b == 0) {
        if (lane < k) {
          if (a.weights_out != nullptr) a.weights_out[lane] = wb;
          if (a.indices_out != nullptr) a.indices_out[lane] = bad ? -1 : route_e;
        }
        if (a.logits_out != nullptr) {
#pragma unroll
          for (int j = 0; j < LPL; ++j)
            if (lane + 64 * j < E) a.logits_out[lane + 64 * j] = f32_to_bf16(lv[j]);
        }
      }
    };
    if constexpr (kShared) {
      weights();
      finish_control(epoch, [] {});
    } else {
      finish_control(epoch, weights);
    }
    return;
  }

  // ======================================================= streaming waves
  // In the workgroups that compute a router row, the streaming waves let the
  // control wave's loads go first, so that routing is not queued behind them.
  if (a.routes_in == nullptr && b < nrow) __builtin_amdgcn_s_sleep(kRouterHeadStart);
  const int sw = b * kWaves + wave, nsw = nb * kWaves;
  Cols<ENC, CHR> colHR;
  make_cols<ENC, CHR>(H / ER::kElems, group, colHR);
  const int64_t spe = static_cast<int64_t>(I) * hpg;  // gate/up scales per expert
  const int64_t spd = static_cast<int64_t>(H) * ipg;  // down scales per expert

  // Activation words and the epoch first: waits for them then never wait for
  // weight rows issued later.
  XRaw<kBF16, CH> xb_raw, wb_raw;
  if constexpr (kShared || RMS) load_x<kBF16, CH>(a.x, colH16, xb_raw);
  XRaw<ENC, CHR> xr_raw, wr_raw;
  load_x<ENC, CHR>(a.x, colHR, xr_raw);
  if constexpr (kWeighted) {  // the norm's weight row in both layouts
    if constexpr (kShared) load_x<kBF16, CH>(a.rms_w, colH16, wb_raw);
    load_x<ENC, CHR>(a.rms_w, colHR, wr_raw);
  }
  const uint32_t last_epoch = co_load(my_epoch + opaque_zero());
  // Normalises the staged activations (the sum of squares is taken over the
  // BF16 layout): done once the first weight rows are in flight, so that the
  // arithmetic overlaps their loads.
  auto normalise = [&]() {
    if constexpr (RMS) {
      const float scale = rms_scale<CH>(xb_raw, colH16, H, a.rms_eps);
      if constexpr (kWeighted) {
        if constexpr (kShared) rms_row<kBF16, CH>(xb_raw, scale, wb_raw);
        rms_row<ENC, CHR>(xr_raw, scale, wr_raw);
      } else {
        if constexpr (kShared) rms_row<kBF16, CH>(xb_raw, scale);
        rms_row<ENC, CHR>(xr_raw, scale);
      }
    }
  };
  // The epoch is derived from last_epoch where each product is stored, after
  // that product's dot (see pinned_after).
  auto epoch_after = [&](float dep) { return next_epoch(pinned_after(last_epoch, dep)); };

  // Phase A: shared gate+up row pairs, one pair in flight per wave (64 KB per
  // CU: enough to keep HBM busy, shallow enough that the control wave's
  // routing loads are not held up long behind it).
  if constexpr (kShared) {
    const int pa = split_at(Is, sw, nsw), pb = split_at(Is, sw + 1, nsw);
    XFrag<kBF16> xb[CH];
    if constexpr (!RMS) frags_of<kBF16, CH>(xb_raw, xb);
    auto pair = [&](int p, bool first) {
      RowLoad<kBF16, CH> rg, ru;
      issue_row<kBF16, CH>(a.sg_w + p * rowH16, nullptr, colH16, rg);
      issue_row<kBF16, CH>(a.su_w + p * rowH16, nullptr, colH16, ru);
      if constexpr (RMS) {
        if (first) {
          normalise();
          frags_of<kBF16, CH>(xb_raw, xb);
        }
      }
      float v[2] = {dot_row<kBF16, CH>(rg, xb, colH16), dot_row<kBF16, CH>(ru, xb, colH16)};
      const float sum = wave_multi_sum<2>(v);  // lanes 0-31: gate, 32-63: up
      const float up = xor_partner<32>(sum);
      if (lane == 0)
        co_store<uint32_t>(a.hs + p, tag16(epoch_after(sum), f32_to_bf16(silu(round_bf16(sum)) * round_bf16(up))));
    };
    if constexpr (RMS) {
      // The first pair is peeled off, so that the norm's weight rows are dead
      // in the loop.
      if (pa < pb) {
        pair(pa, true);
        for (int p = pa + 1; p < pb; ++p) pair(p, false);
      } else {
        normalise();
      }
    } else {
      for (int p = pa; p < pb; ++p) pair(p, false);
    }
  } else {
    normalise();
  }
  XFrag<ENC> xr[CHR];
  frags_of<ENC, CHR>(xr_raw, xr);
  UQM_FUSED_TRACE(4);
  // All waves move to phase B together (one workgroup barrier; letting each
  // wave start phase B on its own, through an LDS flag, measured slower).
  lds_barrier();  // routes ready
  const int route_e = lane < k ? l_route[lane] : 0;
  const bool routes_bad = *l_bad != 0;
  UQM_FUSED_TRACE(5);

  // Phase B: routed gate+up row pairs q = slot * I + i, RBP pairs per batch.
  const int nq = k * I;
  const int qa = split_at(nq, sw, nsw), qb = split_at(nq, sw + 1, nsw);
  RowLoad<ENC, CHR> rb[RBP][2];
  // Always issues RBP pairs (pairs past n re-read pair n - 1, which is then
  // still in flight, so the repeat costs no HBM traffic): a fixed count keeps
  // the compiler's waits for each pair exact, so computing the pairs never
  // waits for loads issued after them.
  auto issue_b = [&](int q0, int n) {
    int slot = q0 / I, i = q0 - slot * I;
#pragma unroll
    for (int t = 0; t < RBP; ++t) {
      const int64_t e = lane_value(route_e, slot);
      const int64_t grow = e * I + i;
      const int64_t srow = e * spe + static_cast<int64_t>(i) * hpg;
      issue_row<ENC, CHR>(a.eg + grow * rowHR, a.egs + srow, colHR, rb[t][0]);
      issue_row<ENC, CHR>(a.eu + grow * rowHR, a.eus + srow, colHR, rb[t][1]);
      if (t + 1 < n && ++i == I) {
        i = 0;
        ++slot;
      }
    }
  };
  // Every issued pair is reduced (only the stores depend on n): a load whose
  // value were used under a branch could be sunk into it by the compiler,
  // behind loads issued later.
  auto compute_b = [&](int q0, int n) {
    float v[VB];
#pragma unroll
    for (int t = 0; t < RBP; ++t) {
      v[2 * t] = dot_row<ENC, CHR>(rb[t][0], xr, colHR);
      v[2 * t + 1] = dot_row<ENC, CHR>(rb[t][1], xr, colHR);
    }
#pragma unroll
    for (int t = 2 * RBP; t < VB; ++t) v[t] = 0.f;
    const float sum = wave_multi_sum<VB>(v);  // value lane >> (6 - log2 VB): gate t, up t, ...
    const float up = xor_partner<64 / VB>(sum);
    constexpr int kL = log2_of<VB>();
    const int idx = lane >> (6 - kL);
    const int t = idx >> 1;
    if ((lane & ((64 >> kL) - 1)) == 0 && (idx & 1) == 0 && t < n) {
      const uint16_t h = routes_bad ? kBf16NaN : f32_to_bf16(silu(round_bf16(sum)) * round_bf16(up));
      co_store<uint32_t>(a.hr + q0 + t, tag16(epoch_after(sum), h));
    }
  };

  // Phase C: output rows o in [oa, ob): the shared down row (CISX chunks per
  // lane) and the k routed down rows flattened into k * CR chunk jobs, job
  // lane + 64 t of this lane.
  const int oa = split_at(H, sw, nsw), ob = split_at(H, sw + 1, nsw);
  Cols<kBF16, CISX> colIS;
  make_cols<kBF16, CISX>(kShared ? Is / 8 : 0, 1, colIS);
  const int njw = uniform((jobs + 63) >> 6);  // job rounds of this wave (<= NJ)
  // Job lane + 64 t: (index clamped to 0 past the end, slot, chunk). The slot
  // comes from a float reciprocal: exact here (jobs < 2^13, and the quotient
  // is never within 1/(2 CR) of an integer boundary).
  const float rcp_cr = 1.0f / static_cast<float>(CR);
  struct Job {
    int jj, s, c;
    bool ok;
  };
  // Up to 4 jobs per lane their index and slot are kept in registers; with
  // more (Q8/BF16 rows) they are recomputed at each use (a few VALU ops).
  constexpr bool kJobRegs = NJ <= 4;
  int jjs_[kJobRegs ? NJ : 1], js_[kJobRegs ? NJ : 1];  // job index (0 past the end); slot, -1 past the end
  auto job_slot = [&](int t, int& jj, int& sl) {
    const int j = lane + 64 * t;
    jj = j < jobs ? j : 0;
    sl = j < jobs ? static_cast<int>((static_cast<float>(jj) + 0.5f) * rcp_cr) : -1;
  };
  if constexpr (kJobRegs) {
#pragma unroll
    for (int t = 0; t < NJ; ++t) job_slot(t, jjs_[t], js_[t]);
  }
  auto job = [&](int t) {
    int jj, sl;
    if constexpr (kJobRegs) {
      jj = jjs_[t];
      sl = js_[t];
    } else {
      job_slot(t, jj, sl);
    }
    Job r;
    r.ok = sl >= 0;
    r.jj = jj;
    r.s = r.ok ? sl : 0;
    r.c = r.jj - r.s * CR;
    return r;
  };
  RowLoad<kBF16, CISX> rs;
  uint4 rw[NJ];
  float rsc[NJ];
  auto issue_cs = [&](int o, const Cols<kBF16, CISX>& cis) {
    if constexpr (kShared) issue_row<kBF16, CISX>(a.sd_w + static_cast<int64_t>(o) * rowIS, nullptr, cis, rs);
  };
  auto issue_cr = [&](int o) {
#pragma unroll
    for (int t = 0; t < NJ; ++t) {
      if (t < njw) {
        const Job jt = job(t);
        const int64_t e = l_route[jt.s];
        rw[t] = ld_stream(a.ed + (e * H + o) * rowIR + static_cast<uint32_t>(jt.c * 16));
        if constexpr (ER::kScaled)
          rsc[t] = ld_stream(a.eds + e * spd + static_cast<int64_t>(o) * ipg +
                             static_cast<uint32_t>((jt.c * ER::kElems) / group));
      }
    }
  };

  int q0 = qa;
  for (; qb - q0 > RBP; q0 += RBP) {
    issue_b(q0, RBP);
    compute_b(q0, RBP);
  }
  // Issued unconditionally (a wave without pairs or rows re-reads a valid
  // one) so that the waits stay exact, as above.
  // The routed products are what every CU waits for, and scattered 1 KB rows
  // lose out at the memory controllers to long sequential streams. So every
  // wave issues its routed gate/up rows, and computes and publishes its routed
  // products, before it issues its routed down rows and its 11 KB shared down
  // row (measured: issuing the shared down row with the routed rows, or at
  // kernel start, is 2-4 us slower per call).
  const int n = qb - q0;
  issue_b(n > 0 ? q0 : nq - 1, n > 0 ? n : 1);
  lds_barrier();  // routed gate/up rows issued
  compute_b(q0, n);
  UQM_FUSED_TRACE(6);

  // Staging of SiLU products into LDS: each wave takes 64-bit tag pairs
  // r0 + lane + 512 t (t < SL) of a round, reloads until all carry this
  // launch's epoch, and stores the bf16 pairs. The shared products (published
  // since phase A) are loaded before the phase-C rows, so they are in LDS by
  // the time the shared down row arrives; the routed products are loaded
  // after the routed down rows (and, with Q4 rows, after the first part of
  // the shared down row), so that they are ready when they arrive.
  const uint32_t epoch = next_epoch(last_epoch);
  constexpr int kRound = SL * kWaves * 64;
  auto load_round = [&](const uint64_t* src, int n2, int base, uint64_t (&v)[SL]) {
#pragma unroll
    for (int t = 0; t < SL; ++t) v[t] = co_load(src + min(base + t * kWaves * 64, n2 - 1));
  };
  auto round_ok = [&](int n2, int base, const uint64_t (&v)[SL]) {
    bool ok = true;
#pragma unroll
    for (int t = 0; t < SL; ++t) {
      const bool tagged = static_cast<uint32_t>(v[t] >> 48) == epoch && (static_cast<uint32_t>(v[t]) >> 16) == epoch;
      ok &= tagged | (base + t * kWaves * 64 >= n2);
    }
    return __all(ok) != 0;
  };
  // Retries give up at this wave's deadline, or at once when another wave
  // has marked this launch as expired; the workgroup's outputs are then
  // poisoned (l_stale).
  auto finish_round = [&](const uint64_t* src, int n2, int base, uint32_t* dst, uint64_t (&v)[SL]) {
    // The first check is outside the retry loop, so the compiler waits for
    // exactly these loads (not for the rows issued after them).
    if (force_expiry || !round_ok(n2, base, v)) {
      for (;;) {
        if (wall_clock() > deadline) {
          raise_expired(a.sync, epoch);
          if (lane == 0) *l_stale = 1;
          break;
        }
        if (co_load(a.sync + kSyncExpired) == epoch) {
          raise_expired(a.sync, epoch);  // the error word is raised by every wave that gives up
          if (lane == 0) *l_stale = 1;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
        load_round(src, n2, base, v);
        if (round_ok(n2, base, v)) break;
      }
    }
#pragma unroll
    for (int t = 0; t < SL; ++t) {
      const int j = base + t * kWaves * 64;
      if (j < n2) dst[j] = (static_cast<uint32_t>(v[t]) & 0xFFFFu) | (static_cast<uint32_t>(v[t] >> 32) << 16);
    }
  };
  const uint64_t* hs64 = reinterpret_cast<const uint64_t*>(a.hs);
  const uint64_t* hr64 = reinterpret_cast<const uint64_t*>(a.hr);
  const int n2s = Is / 2, n2r = k * I / 2;
  const int base0 = wave * 64 + lane;
  // Rows wider than Q4 (Q8/BF16 routed down rows) do not fit in registers
  // beside the shared down row: there the routed down rows are issued once
  // the shared part is reduced.
  auto stage_hs = [&](uint64_t (&vs)[SL]) {
    finish_round(hs64, n2s, base0, reinterpret_cast<uint32_t*>(lhs), vs);
    for (int b2 = base0 + kRound; b2 - lane < n2s; b2 += kRound) {
      load_round(hs64, n2s, b2, vs);
      finish_round(hs64, n2s, b2, reinterpret_cast<uint32_t*>(lhs), vs);
    }
  };
  // With Q4 routed rows (job ids in registers) the shared down row goes out
  // in two parts around the routed-product loads: its first CSA chunks per
  // lane, the product loads, the rest. The products then arrive while the
  // rest of the row streams, so their staging and the routed fragments are
  // built before the row is complete, and only the dot products remain once
  // it is. A product wait that has to retry re-issues its loads behind the
  // whole row, which is where the loads sat before (CSA = 3 of 11 chunks:
  // 22.4-22.8 vs 22.8-23.8 us per launch in the timeline harness; 5: 22.9,
  // 7: 23.1, 0: 22.9).
  constexpr bool kSplit = kJobRegs && kShared;
  constexpr int CSA = kSplit ? 3 : CISX;
  auto issue_cs_range = [&](int o, auto lo_tag, auto hi_tag) {
    constexpr int J0 = decltype(lo_tag)::value, J1 = decltype(hi_tag)::value;
#pragma unroll
    for (int j = J0; j < J1; ++j)
      rs.w[j] = ld_stream(a.sd_w + static_cast<int64_t>(o) * rowIS + static_cast<uint32_t>(colIS.c(j) * 16));
  };
  uint64_t vr[SL];
  {
    uint64_t vs[SL];
    if constexpr (kShared) load_round(hs64, n2s, base0, vs);
    if constexpr (kJobRegs || !kShared) issue_cr(oa < ob ? oa : H - 1);
    if constexpr (kSplit)
      issue_cs_range(oa < ob ? oa : H - 1, std::integral_constant<int, 0>{}, std::integral_constant<int, CSA>{});
    else
      issue_cs(oa < ob ? oa : H - 1, colIS);
    if constexpr (kShared) stage_hs(vs);
  }
  if constexpr (!kShared) __builtin_amdgcn_s_sleep(kProductDelayRoutedOnly);
  load_round(hr64, n2r, base0, vr);
  if constexpr (kSplit)
    issue_cs_range(oa < ob ? oa : H - 1, std::integral_constant<int, CSA>{}, std::integral_constant<int, CISX>{});
  UQM_FUSED_TRACE(7);
  lds_barrier();  // shared products staged

  float sg = 0.f;
  if constexpr (kShared) sg = *l_sg;
  // Shared part of out[o] (per lane): sg * (shared down row o . h_s).
  auto shared_part = [&](const Cols<kBF16, CISX>& cis) {
    float acc = 0.f;
    if constexpr (kShared) {
      XFrag<kBF16> fs[CISX];
      frags_from<kBF16, CISX>(lhs, cis, fs);
      acc = sg * dot_row<kBF16, CISX>(rs, fs, cis);
    }
    return acc;
  };
  // Routed part of out[o] (per lane): sum over this lane's jobs of
  // w_slot * scale * (down chunk . h_slot chunk).
  auto routed_part = [&]() {
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < NJ; ++t) {
      if (t < njw) {
        const Job jt = job(t);
        XFrag<ENC> f;
#pragma unroll
        for (int q = 0; q < ER::kXWords / 4; ++q) {
          const uint4 u = *reinterpret_cast<const uint4*>(lfr + jt.jj * ER::kXWords + 4 * q);
          f.w[4 * q] = u.x;
          f.w[4 * q + 1] = u.y;
          f.w[4 * q + 2] = u.z;
          f.w[4 * q + 3] = u.w;
        }
        f.off = loff[jt.jj];
        const float w = jt.ok ? l_w[jt.s] : 0.f;
        const float d = dot_chunk<ENC>(rw[t], f);
        acc = fmaf(d, ER::kScaled ? rsc[t] * w : w, acc);
      }
    }
    return acc;
  };
  float acc_s = 0.f;
  if constexpr (!kSplit) acc_s = shared_part(colIS);
  if constexpr (!kJobRegs && kShared) issue_cr(oa < ob ? oa : H - 1);
  finish_round(hr64, n2r, base0, reinterpret_cast<uint32_t*>(lhr), vr);
  for (int b2 = base0 + kRound; b2 - lane < n2r; b2 += kRound) {
    load_round(hr64, n2r, b2, vr);
    finish_round(hr64, n2r, b2, reinterpret_cast<uint32_t*>(lhr), vr);
  }
  lds_barrier();  // routed products staged
  build_fragments();
  lds_barrier();  // routed fragments built
  UQM_FUSED_TRACE(8);
  if constexpr (kSplit) acc_s = shared_part(colIS);  // waits for the rest of the shared down row
  const bool stale = *l_stale != 0;
  // out[o] = bf16(sum over lanes of (shared part + routed part)).
  {
    const float y = wave_sum(acc_s + routed_part());
    if (lane == 0 && oa < ob) a.out[oa] = stale ? kBf16NaN : f32_to_bf16(y);
  }
  for (int o = oa + 1; o < ob; ++o) {  // more rows than streaming waves (small grids only)
    Cols<kBF16, CISX> cis;
    make_cols<kBF16, CISX>(kShared ? Is / 8 : 0, 1, cis, opaque_lane());
    issue_cs(o, cis);
    issue_cr(o);
    const float y = wave_sum(shared_part(cis) + routed_part());
    if (lane == 0) a.out[o] = stale ? kBf16NaN : f32_to_bf16(y);
  }
  UQM_FUSED_TRACE(9);
}

namespace {

int cpl(int64_t chunks) { return static_cast<int>((chunks + 63) / 64); }

template <int ENC, int CH, int CHR, int CIR, int CIS, int KMAX, int NORM>
hipError_t launch_kernel(const FusedArgs& args, hipStream_t stream) {
  auto kern = moe_decode_fused_kernel<ENC, CH, CHR, CIR, CIS, KMAX, NORM>;
  const size_t lds = fused_lds_bytes<ENC>(args.I, args.Is, args.k);
  if (lds > 64 * 1024) return hipErrorInvalidValue;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  int per_cu = 0, cus = 0;
  if ((e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kThreads, lds)) != hipSuccess) return e;
  if ((e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
  if (per_cu < 1 || cus < 1 || cus > kMaxFusedBlocks) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(kern, dim3(cus), dim3(kThreads), lds, stream, args);  // one workgroup per CU, all resident
  return hipGetLastError();
}

}  // namespace

int fused_config_id(int enc, int64_t H, int64_t I, int64_t Is, int64_t k, int64_t E) {
  // Per-lane chunk loops are masked, so an instantiation serves every shape
  // whose chunk counts per lane do not exceed its template arguments.
  const int el = enc == kQ4 ? 32 : enc == kQ8 ? 16 : 8;
  const int ch = cpl(H / 8), chr = cpl(H / el), cir = cpl(I / el), cis = Is > 0 ? cpl(Is / 8) : 0;
  if (k < 1 || k > 8 || k > E || E < 1 || E + 1 > 320 || ch > 4 || cis > 11) return -1;
  // Instantiations (others run the multi-kernel path): Q4 with a shared
  // expert and k <= 4 or without one and k <= 8; Q8 and BF16 with k <= 4.
  if (k > (enc == kQ4 && Is == 0 ? 8 : 4)) return -1;
  if (H % 8 != 0 || I % 8 != 0 || Is % 8 != 0) return -1;
  const size_t lds = enc == kQ4 ? fused_lds_bytes<kQ4>(I, Is, k)
                                 : enc == kQ8 ? fused_lds_bytes<kQ8>(I, Is, k) : fused_lds_bytes<kBF16>(I, Is, k);
  if (lds > 64 * 1024) return -1;
  if (enc == kQ4 && chr <= 1 && cir <= 1) return 0;
  if (enc == kQ8 && chr <= 2 && cir <= 2) return 1;
  if (enc == kBF16 && chr <= 4 && cir <= 3) return 2;
  return -1;
}

namespace {

// The input norm is a template parameter: the kernels without it (or
// without its weight row, which costs registers) are not perturbed by its
// code (register allocation, scheduling).
template <int ENC, int CH, int CHR, int CIR, int CIS, int KMAX>
hipError_t launch_cfg(const FusedArgs& args, hipStream_t stream) {
  if (!args.rms) return launch_kernel<ENC, CH, CHR, CIR, CIS, KMAX, kNormNone>(args, stream);
  return args.rms_w != nullptr ? launch_kernel<ENC, CH, CHR, CIR, CIS, KMAX, kNormWeighted>(args, stream)
                               : launch_kernel<ENC, CH, CHR, CIR, CIS, KMAX, kNormUnit>(args, stream);
}

}  // namespace

hipError_t launch_moe_decode_fused(int enc, const FusedArgs& a, hipStream_t stream) {
  if (fused_config_id(enc, a.H, a.I, a.Is, a.k, a.E) < 0) return hipErrorInvalidValue;
  const bool k4 = a.k <= 4;
  if (enc == kQ4) {
    if (a.Is > 0) return launch_cfg<kQ4, 4, 1, 1, 11, 4>(a, stream);
    return k4 ? launch_cfg<kQ4, 4, 1, 1, 0, 4>(a, stream) : launch_cfg<kQ4, 4, 1, 1, 0, 8>(a, stream);
  }
  const bool shared = a.Is > 0;
  if (enc == kQ8) return shared ? launch_cfg<kQ8, 4, 2, 2, 11, 4>(a, stream) : launch_cfg<kQ8, 4, 2, 2, 0, 4>(a, stream);
  return shared ? launch_cfg<kBF16, 4, 4, 3, 11, 4>(a, stream) : launch_cfg<kBF16, 4, 4, 3, 0, 4>(a, stream);
}

}  // namespace uqm
