// extern "C" entry points of libuma_qmoe_hip.so (declared in
// include/uma_qmoe_hip.h). Each validates its arguments on the host, carves
// the caller's workspace and enqueues kernels on the caller's stream.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <string>
#include <unordered_map>

#include "../../include/uma_qmoe_hip.h"
#include "uqm_dense.h"
#include "uqm_internal.h"
#include "uqm_route.h"

namespace {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(UQM_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return UQM_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int elems_per_chunk(int enc) { return enc == UQM_Q4 ? 32 : enc == UQM_Q8 ? 16 : 8; }

size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

// Workspace carve-up shared by the size query and the entry points.
// FP32 partial outputs a K-split MFMA down projection may write.
constexpr int kMaxSplit = 4;

struct Layout {
  size_t fused_sync, fused_hs, fused_hr, fused_lgt, normed, counters, route_expert, route_order, expert_offsets, active_experts,
      tiles, logits, weights, indices, sg, router_part, h_routed, y_routed, h_shared, y_shared, total;
};

Layout layout(int64_t T, int64_t H, int64_t I, int64_t Is, int64_t E, int64_t k) {
  Layout L{};
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += align256(bytes);
    return at;
  };
  const size_t R = static_cast<size_t>(T * k);
  L.fused_sync = take(4 * uqm::kSyncWords);
  L.fused_hs = take(4 * static_cast<size_t>(Is));
  L.fused_hr = take(4 * static_cast<size_t>(k) * I);
  L.fused_lgt = take(8 * static_cast<size_t>(E + 1));
  L.normed = take(2 * static_cast<size_t>(T) * H);  // RMSNorm(hidden) of a pre-normalised block
  L.counters = take(256);
  L.route_expert = take(4 * R);
  L.route_order = take(4 * R);
  L.expert_offsets = take(4 * (E + 1));
  L.active_experts = take(4 * E);
  L.tiles = take(8 * (E + R));
  L.logits = take(2 * static_cast<size_t>(T) * (E + 1));
  L.weights = take(2 * R);
  L.indices = take(8 * R);
  L.sg = take(4 * static_cast<size_t>(T));
  L.router_part = take(T > 1 ? 4 * static_cast<size_t>(kMaxSplit) * T * ((E + 1 + 15) / 16 * 16) : 0);
  L.h_routed = take(2 * R * I);
  L.y_routed = take(4 * R * H * (T > 1 ? kMaxSplit : 1));
  L.h_shared = take(2 * static_cast<size_t>(T) * Is);
  L.y_shared = take(4 * static_cast<size_t>(T) * H * (T > 1 && Is > 0 ? kMaxSplit : 1));
  L.total = off;
  return L;
}

template <typename P>
P* at(void* ws, size_t off) {
  return reinterpret_cast<P*>(static_cast<unsigned char*>(ws) + off);
}

// Process-wide options (uqm_set_option).
std::atomic<int64_t> g_opt_fused{1};
std::atomic<int64_t> g_opt_fused_wait_us{uqm::kFusedWaitBudgetUs};
std::atomic<int64_t> g_opt_mfma_min_tokens{2};
std::atomic<int64_t> g_opt_overlap_shared{1};
std::atomic<int64_t> g_opt_stream_max_routes{32};

// Token counts served by one fused single-token launch per token.
constexpr int64_t kFusedMaxTokens = 2;

// Compute units of the current device (cached per device id).
std::atomic<int> g_cus[64];

int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev >= 0 && dev < 64) {
    const int v = g_cus[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  if (dev >= 0 && dev < 64) g_cus[dev].store(n, std::memory_order_relaxed);
  return n;
}

// The fused kernel's wait budget in s_memrealtime ticks of the current device
// (UQM_OPT_FUSED_WAIT_US; the clock runs at hipDeviceAttributeWallClockRate
// kHz, cached per device id). A zero budget stays zero: every wait of the
// launch then gives up at its first check.
std::atomic<int> g_clock_khz[64];

uint64_t fused_wait_ticks() {
  const int64_t us = g_opt_fused_wait_us.load(std::memory_order_relaxed);
  if (us <= 0) return 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  int khz = dev >= 0 && dev < 64 ? g_clock_khz[dev].load(std::memory_order_relaxed) : 0;
  if (khz <= 0) {
    if (dev < 0 || hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || khz <= 0)
      khz = 100000;  // the 100 MHz reference clock of CDNA parts
    if (dev >= 0 && dev < 64) g_clock_khz[dev].store(khz, std::memory_order_relaxed);
  }
  return static_cast<uint64_t>(khz) * static_cast<uint64_t>(us) / 1000u;
}

// Layout of the fused kernel's hand-off words (shared SiLU products, routed
// SiLU products, router logits) in a workspace: their offsets and extent
// depend on these four sizes only. Every entry point that writes into a
// workspace records the layout it used; a fused launch whose layout differs
// from the last one recorded for its workspace (or on a workspace not seen
// before) first zeroes its hand-off region. Words another layout left there
// (tagged words at other offsets, route tables, partial sums) could otherwise
// carry the new launch's epoch in both halves of a pair by chance and be
// taken as this launch's products. Within one layout every fused launch
// rewrites every hand-off word it reads, so its words always carry the
// previous launch's epoch and the 16-bit epoch can wrap safely.
struct HandoffLayout {
  int64_t E, k, I, Is;
  bool operator==(const HandoffLayout& o) const { return E == o.E && k == o.k && I == o.I && Is == o.Is; }
};
std::mutex g_layout_mu;
std::unordered_map<uintptr_t, HandoffLayout> g_layouts;  // workspace address -> last layout
constexpr size_t kMaxTrackedWorkspaces = 4096;           // beyond: forget all (each is cleared once more)

// Records `lay` for `workspace`; for a fused launch, zeroes the hand-off
// region on `s` first when the layout changed.
int note_layout(void* workspace, const Layout& L, HandoffLayout lay, bool fused, hipStream_t s) {
  bool clear = false;
  {
    std::lock_guard<std::mutex> lock(g_layout_mu);
    const uintptr_t key = reinterpret_cast<uintptr_t>(workspace);
    auto it = g_layouts.find(key);
    clear = fused && (it == g_layouts.end() || !(it->second == lay));
    if (it != g_layouts.end()) {
      it->second = lay;
    } else {
      if (g_layouts.size() >= kMaxTrackedWorkspaces) g_layouts.clear();
      g_layouts.emplace(key, lay);
    }
  }
  if (!clear) return UQM_OK;
  return hip_check(uqm::launch_zero_fill(at<unsigned char>(workspace, L.fused_hs), L.normed - L.fused_hs, s),
                   "hand-off region clear");
}

// Launch shape of one MFMA grouped GEMM (see launch_expert_mfma).
struct MfmaPlan {
  int nb = 1, kw = 1, mw = 4, ksplit = 1;
};

// 16-route tiles per workgroup from the mean routes per expert.
int nb_for(int enc, double mean_routes) {
  if (mean_routes <= 16) return 1;
  if (mean_routes <= 32) return 2;
  if (mean_routes <= 64 || enc != UQM_BF16) return 4;
  return 8;
}

// Enough work items (row block x route tile) for the persistent grid: 8 MMA
// waves (128 rows per item) when there is plenty of work, 4 (64 rows), then
// waves and workgroups along K when there is little. Every K range keeps
// >= 3 steps of 128 per wave.
MfmaPlan plan_mfma(int enc, int nmat, int64_t rows, int64_t K, int nb, int64_t tiles, int cus, int max_split) {
  MfmaPlan p;
  p.nb = nb;
  if (nb <= 3 && (nmat == 1 || enc == UQM_Q4) && rows % 128 == 0 && rows / 128 * tiles >= cus) {
    p.mw = 8;
    return p;
  }
  const int64_t items64 = rows / 64 * tiles;
  if (items64 >= cus) return p;
  if (nb == 1 && K / 128 >= 12) p.kw = 4;
  if (nmat == 2) return p;
  const int64_t items = rows / (p.kw == 4 ? 16 : 64) * tiles;
  int64_t ks = (cus + items - 1) / items;
  const int64_t max_by_k = (K / 128) / (3 * p.kw);
  if (ks > max_split) ks = max_split;
  if (ks > max_by_k) ks = max_by_k;
  p.ksplit = ks < 1 ? 1 : static_cast<int>(ks);
  return p;
}

bool routed_uses_mfma(const uqm_expert_weights* w, int64_t T) {
  const int64_t min_t = g_opt_mfma_min_tokens.load(std::memory_order_relaxed);
  return min_t > 0 && T >= min_t && uqm::mfma_supported(w->encoding, w->intermediate_size, w->hidden_size, w->group_size) &&
         uqm::mfma_supported(w->encoding, w->hidden_size, w->intermediate_size, w->group_size);
}

bool shared_uses_mfma(int64_t H, int64_t Is, int64_t T) {
  const int64_t min_t = g_opt_mfma_min_tokens.load(std::memory_order_relaxed);
  return min_t > 0 && T >= min_t && uqm::mfma_supported(UQM_BF16, Is, H, 0) && uqm::mfma_supported(UQM_BF16, H, Is, 0);
}

// The shared expert of calls with many tokens takes the dense kernel.
bool shared_uses_dense(int64_t H, int64_t Is, int64_t T) {
  return g_opt_mfma_min_tokens.load(std::memory_order_relaxed) > 0 && uqm::dense_supported(Is, H, T) &&
         uqm::dense_supported(H, Is, T);
}

// Whether the GEMV path of the routed experts streams (uqm_stream.hip) rather
// than staging activations per workgroup (uqm_gemv.hip).
bool routed_uses_stream(const uqm_expert_weights* w) {
  return g_opt_stream_max_routes.load(std::memory_order_relaxed) > 0 &&
         uqm::stream_supported(w->encoding, w->hidden_size, w->group_size) &&
         uqm::stream_supported(w->encoding, w->intermediate_size, w->group_size);
}

// Route tile size the routed MFMA path uses (0 = GEMV path). From 16 routes
// per expert on average, 32-route tiles: measured faster than 16 (c5: 80 vs
// 105 us) and than 64 (c4: 247 vs 271 us), whose 4-wave items take longer per
// weight byte.
int routed_tile_tokens(const uqm_expert_weights* w, int64_t T, int64_t k) {
  if (!routed_uses_mfma(w, T)) return 0;
  const int64_t R = T * k;
  const int64_t active = R < w->num_experts ? R : w->num_experts;
  const double mean = static_cast<double>(R) / static_cast<double>(active);
  if (routed_uses_stream(w) && R <= g_opt_stream_max_routes.load(std::memory_order_relaxed)) return 0;
  // 48-route tiles when most experts would otherwise take a second, nearly
  // empty 32-route tile (every tile costs a full pass over the expert's rows)
  // and both Q4 projections run 128-row items (the only kernels built for them)
  const int cus = device_cus();
  if (mean > 32 && mean <= 48 && w->encoding == UQM_Q4 && w->intermediate_size % 128 == 0 &&
      w->hidden_size % 128 == 0 && active * (w->intermediate_size / 128) >= cus &&
      active * (w->hidden_size / 128) >= cus)
    return 48;
  return 16 * (mean >= 16 ? 2 : nb_for(w->encoding, mean));
}

// Per-device side stream and fork/join events: a multi-token block runs the
// shared expert (which reads only the input) on the side stream, beside the
// router -> top-k -> permute -> routed chain on the caller's stream, and the
// combine waits for both. The mutex is held from the fork to the join so that
// two host threads never interleave records of the same events. The stream is
// non-blocking (no implicit sync with the legacy default stream) and keeps the
// default priority.
struct SideStream {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
std::mutex g_side_mu;
SideStream g_side[64];

// Side stream of the current device, created on first use; nullptr when it
// does not exist yet and `caller` is being captured into a graph (creation
// is not a capturable call), or when creation fails: the caller then runs the
// shared expert in order on its own stream.
SideStream* side_stream(hipStream_t caller) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  SideStream& ss = g_side[dev];
  if (ss.stream != nullptr) return &ss;
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(caller, &st) != hipSuccess || st != hipStreamCaptureStatusNone) return nullptr;
  hipStream_t s = nullptr;
  hipEvent_t f = nullptr, j = nullptr;
  if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) return nullptr;
  if (hipEventCreateWithFlags(&f, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&j, hipEventDisableTiming) != hipSuccess) {
    if (f != nullptr) (void)hipEventDestroy(f);
    (void)hipStreamDestroy(s);
    return nullptr;
  }
  ss.fork = f;
  ss.join = j;
  ss.stream = s;
  return &ss;
}

// Per-device verdict of the gfx950 check: 0 unknown, 1 gfx950, 2 other.
std::atomic<int> g_device_ok[64];

int check_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(UQM_ERR_HIP, "hipGetDevice failed");
  if (dev >= 0 && dev < 64) {
    const int v = g_device_ok[dev].load(std::memory_order_relaxed);
    if (v == 1) return UQM_OK;
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return fail(UQM_ERR_HIP, "hipGetDeviceProperties failed");
  const bool ok = strncmp(prop.gcnArchName, "gfx950", 6) == 0;
  if (dev >= 0 && dev < 64) g_device_ok[dev].store(ok ? 1 : 2, std::memory_order_relaxed);
  if (!ok) return fail(UQM_ERR_DEVICE, "libuma_qmoe_hip requires gfx950, current device is %s", prop.gcnArchName);
  return UQM_OK;
}

int check_matrix(int enc, int64_t K, int64_t group, const void* w, const float* s, const char* name) {
  if (w == nullptr) return fail(UQM_ERR_ARGUMENT, "%s weights are NULL", name);
  if (!aligned16(w)) return fail(UQM_ERR_ARGUMENT, "%s weights must be 16-byte aligned", name);
  const int el = elems_per_chunk(enc);
  if (K <= 0 || K % el != 0) return fail(UQM_ERR_ARGUMENT, "%s input features %lld must be a multiple of %d", name, (long long)K, el);
  if (K % 8 != 0) return fail(UQM_ERR_ARGUMENT, "%s input features must be a multiple of 8", name);
  if (enc != UQM_BF16) {
    if (s == nullptr) return fail(UQM_ERR_ARGUMENT, "%s scales are NULL", name);
    if (group <= 0 || group % el != 0)
      return fail(UQM_ERR_ARGUMENT, "%s group size %lld must be a positive multiple of %d", name, (long long)group, el);
  }
  return UQM_OK;
}

int check_experts(const uqm_expert_weights* w) {
  if (w == nullptr) return fail(UQM_ERR_ARGUMENT, "expert weights descriptor is NULL");
  if (w->encoding != UQM_Q4 && w->encoding != UQM_Q8 && w->encoding != UQM_BF16)
    return fail(UQM_ERR_ARGUMENT, "unsupported expert encoding %d", w->encoding);
  if (w->num_experts <= 0 || w->num_experts > 256) return fail(UQM_ERR_ARGUMENT, "num_experts must be in [1, 256]");
  if (w->hidden_size <= 0 || w->intermediate_size <= 0) return fail(UQM_ERR_ARGUMENT, "hidden and intermediate sizes must be positive");
  int rc;
  if ((rc = check_matrix(w->encoding, w->hidden_size, w->group_size, w->gate, w->gate_scales, "gate"))) return rc;
  if ((rc = check_matrix(w->encoding, w->hidden_size, w->group_size, w->up, w->up_scales, "up"))) return rc;
  if ((rc = check_matrix(w->encoding, w->intermediate_size, w->group_size, w->down, w->down_scales, "down"))) return rc;
  return UQM_OK;
}

int check_lds(int enc, int64_t K, int nt) {
  if (uqm::gemv_lds_bytes(enc, K, nt) > 64 * 1024)
    return fail(UQM_ERR_ARGUMENT, "input features %lld exceed the decode kernel's LDS staging limit", (long long)K);
  return UQM_OK;
}

bool router_uses_mfma(int64_t H, int64_t T) {
  const int64_t min_t = g_opt_mfma_min_tokens.load(std::memory_order_relaxed);
  return min_t > 0 && T >= min_t && T > 1 && uqm::mfma_supported(UQM_BF16, 64, H, 0);
}

// Router on T > 1 tokens as an MFMA GEMM over the router rows (plus the shared
// expert's gate row, appended as row E): FP32 partial logits in the
// workspace, then top-k, which rounds their sum to bf16 like the router's
// bf16 linear. logits (optional) receives the bf16 logits [T, E].
int run_router_mfma(const void* router, const void* gate_row, int64_t E, const uint16_t* x, int64_t T, int64_t H,
                    int64_t k, int norm, const Layout& L, void* ws, uint16_t* wout, int64_t* iout,
                    int32_t* route_expert, float* sg, uint16_t* logits, const uqm::RouteTables* perm,
                    int tile_tokens, uint32_t* counter, hipStream_t stream) {
  using namespace uqm;
  const int64_t rows = E + (gate_row != nullptr ? 1 : 0);
  const int64_t rp = (rows + 15) / 16 * 16;
  const int64_t tiles = (T + 15) / 16;
  const int cus = device_cus();
  MfmaArgs r{};
  r.w[0] = static_cast<const uint8_t*>(router);
  r.w_tail = static_cast<const uint8_t*>(gate_row);
  r.tail_from = E;
  r.rows = rp;
  r.rows_valid = rows;
  r.K = H;
  r.x = x;
  r.ldx = H;
  r.x_div = 1;
  r.tile_bound = static_cast<int32_t>(tiles);
  r.n_routes = static_cast<int32_t>(T);
  r.out = at<float>(ws, L.router_part);
  r.ldo = rp;
  r.part_stride = T * rp;
  const int64_t items = rp / 16 * tiles;
  int64_t ks = (cus + items - 1) / items;
  const int64_t max_by_k = (H / 64) / (3 * 4);  // >= 3 steps of 64 per wave
  if (ks > kMaxSplit) ks = kMaxSplit;
  if (ks > max_by_k) ks = max_by_k;
  r.ksplit = ks < 1 ? 1 : static_cast<int>(ks);
  int rc = hip_check(launch_expert_mfma(UQM_BF16, 1, r, 1, 4, 4, cus, stream), "router MFMA launch");
  if (rc) return rc;
  if (perm != nullptr)
    return hip_check(launch_route_topk_permute(nullptr, at<float>(ws, L.router_part), r.ksplit, T * rp, rp, T, E, k,
                                               norm, wout, iout, sg, logits, *perm, tile_tokens, counter, stream),
                     "top-k + permute launch");
  return hip_check(launch_route_topk_partials(at<float>(ws, L.router_part), r.ksplit, T * rp, rp, T, E, k, norm, wout,
                                              iout, route_expert, sg, logits, stream),
                   "top-k launch");
}

// Routed experts, given device route tables already built in the workspace
// (with route tiles of `tile_tokens` when the MFMA path is used). Returns the
// number of FP32 partials written to y_routed through *parts.
int run_routed(const uqm_expert_weights* w, const uint16_t* hidden, int64_t T, int64_t k, const Layout& L,
               void* ws, int tile_tokens, int* parts, hipStream_t stream) {
  using namespace uqm;
  const int64_t E = w->num_experts, H = w->hidden_size, I = w->intermediate_size;
  const int64_t R = T * k;
  *parts = 1;
  if (tile_tokens > 0) {
    const int nb = tile_tokens / 16;
    const int64_t active = R < E ? R : E;
    const int cus = device_cus();
    MfmaArgs g{};
    g.w[0] = static_cast<const uint8_t*>(w->gate);
    g.w[1] = static_cast<const uint8_t*>(w->up);
    g.s[0] = w->gate_scales;
    g.s[1] = w->up_scales;
    g.rows = I;
    g.K = H;
    g.group = w->group_size;
    g.x = hidden;
    g.ldx = H;
    g.x_div = static_cast<int32_t>(k);
    g.route_order = at<int32_t>(ws, L.route_order);
    g.expert_offsets = at<int32_t>(ws, L.expert_offsets);
    g.tiles = at<int32_t>(ws, L.tiles);
    g.tile_count = at<int32_t>(ws, L.counters) + 1;
    g.tile_bound = static_cast<int32_t>(active + R / tile_tokens);
    g.out = at<uint16_t>(ws, L.h_routed);
    g.ldo = I;
    g.ksplit = 1;
    // gate/up: row blocks fastest when most experts have one tile (c4 gate/up
    // 194 vs 229 MB fetched per call for 184 MB of weights); hot experts with
    // many tiles (c5) share their rows with tiles fastest (53 vs 60 MB for 40)
    g.order = kOrderAuto;
    g.active_count = at<int32_t>(ws, L.counters);
    const MfmaPlan pg = plan_mfma(w->encoding, 2, I, H, nb, active, cus, 1);
    int rc = hip_check(launch_expert_mfma(w->encoding, 2, g, pg.nb, pg.kw, pg.mw, cus, stream), "gate/up MFMA launch");
    if (rc) return rc;
    MfmaArgs d = g;
    d.w[0] = static_cast<const uint8_t*>(w->down);
    d.w[1] = nullptr;
    d.s[0] = w->down_scales;
    d.s[1] = nullptr;
    d.rows = H;
    d.K = I;
    d.x = at<uint16_t>(ws, L.h_routed);
    d.ldx = I;
    d.x_div = 1;
    d.out = at<float>(ws, L.y_routed);
    d.ldo = H;
    d.part_stride = R * H;
    d.order = kOrderRowFastest;
    const MfmaPlan pd = plan_mfma(w->encoding, 1, H, I, nb, active, cus, T > 1 ? kMaxSplit : 1);
    d.ksplit = pd.ksplit;
    *parts = pd.ksplit;
    return hip_check(launch_expert_mfma(w->encoding, 1, d, pd.nb, pd.kw, pd.mw, cus, stream), "down MFMA launch");
  }
  const int grid_y = static_cast<int>(E < R ? E : R);
  const bool stream_path = routed_uses_stream(w);
  // Streaming GEMV: routes per expert held in registers, from the mean routes
  // per active expert (experts with more take further passes).
  const int64_t mean_routes = (R + grid_y - 1) / grid_y;
  const int nt = stream_path ? static_cast<int>(mean_routes <= 1 ? 1 : mean_routes <= 2 ? 2 : 4)
                             : static_cast<int>(T < 4 ? T : 4);
  GemvArgs g{};
  g.w[0] = static_cast<const uint8_t*>(w->gate);
  g.w[1] = static_cast<const uint8_t*>(w->up);
  g.s[0] = w->gate_scales;
  g.s[1] = w->up_scales;
  g.rows = I;
  g.K = H;
  g.group = w->group_size;
  g.x = hidden;
  g.ldx = H;
  g.x_div = static_cast<int32_t>(k);
  g.route_order = at<int32_t>(ws, L.route_order);
  g.expert_offsets = at<int32_t>(ws, L.expert_offsets);
  g.active_experts = at<int32_t>(ws, L.active_experts);
  g.active_count = at<int32_t>(ws, L.counters);
  g.out = at<uint16_t>(ws, L.h_routed);
  g.ldo = I;
  const int cus = device_cus();
  int rc = hip_check(stream_path ? launch_routed_stream(w->encoding, 2, kModeSilu, g, nt, grid_y, cus, stream)
                                 : launch_expert_gemv(w->encoding, 2, kModeSilu, g, grid_y, nt, stream),
                     "gate/up launch");
  if (rc) return rc;
  GemvArgs d = g;
  d.w[0] = static_cast<const uint8_t*>(w->down);
  d.w[1] = nullptr;
  d.s[0] = w->down_scales;
  d.s[1] = nullptr;
  d.rows = H;
  d.K = I;
  d.x = at<uint16_t>(ws, L.h_routed);
  d.ldx = I;
  d.x_div = 1;
  d.out = at<float>(ws, L.y_routed);
  d.ldo = H;
  return hip_check(stream_path ? launch_routed_stream(w->encoding, 1, kModeF32, d, nt, grid_y, cus, stream)
                               : launch_expert_gemv(w->encoding, 1, kModeF32, d, grid_y, nt, stream),
                   "down launch");
}

// Shared expert on T tokens: h_shared = silu(x Wg^T) * (x Wu^T), y_shared =
// h_shared Wd^T (FP32, *parts K-split partials).
int run_shared(const uqm_layer_weights* layer, const uint16_t* x, int64_t T, int64_t H, const Layout& L, void* ws,
               int* parts, bool beside, hipStream_t stream) {
  using namespace uqm;
  const int64_t Is = layer->shared_intermediate_size;
  *parts = 1;
  if (shared_uses_dense(H, Is, T)) {
    // Dense square tiles (uqm_dense.hip); beside the routing chain at 3/4 of
    // the CUs, as the grouped kernel below.
    const int cus = beside ? device_cus() * 3 / 4 : device_cus();
    DenseArgs g{};
    g.w[0] = static_cast<const uint16_t*>(layer->shared_gate);
    g.w[1] = static_cast<const uint16_t*>(layer->shared_up);
    g.x = x;
    g.ldx = H;
    g.rows = Is;
    g.K = H;
    g.T = T;
    g.out = at<uint16_t>(ws, L.h_shared);
    g.ldo = Is;
    g.ksplit = 1;
    const DensePlan pg = plan_dense(2, Is, H, T, cus, 1);
    int rc = hip_check(launch_dense_mfma(2, g, pg.waves, cus, stream), "shared gate/up dense launch");
    if (rc) return rc;
    DenseArgs d{};
    d.w[0] = static_cast<const uint16_t*>(layer->shared_down);
    d.x = at<uint16_t>(ws, L.h_shared);
    d.ldx = Is;
    d.rows = H;
    d.K = Is;
    d.T = T;
    d.out = at<float>(ws, L.y_shared);
    d.ldo = H;
    d.part_stride = T * H;
    const DensePlan pd = plan_dense(1, H, Is, T, cus, kMaxSplit);
    d.ksplit = pd.ksplit;
    *parts = d.ksplit;
    return hip_check(launch_dense_mfma(1, d, pd.waves, cus, stream), "shared down dense launch");
  }
  if (shared_uses_mfma(H, Is, T)) {
    // Up to 32 tokens: 16-token tiles, so that the plan can split K over
    // waves (16-row items) and fill the grid; the second tile of a row block
    // runs right after the first on the same workgroup and reads the rows
    // from L2.
    const int nb = T <= 32 ? 1 : nb_for(UQM_BF16, static_cast<double>(T));
    const int ntok = 16 * nb;
    const int64_t tiles = (T + ntok - 1) / ntok;
    // Beside the routing chain, the persistent grids take 3/4 of the CUs'
    // slots, so that the router and top-k launches find room at once (batch
    // 32: 113.6 vs 122.0 us per call; 1/2: 118.0, 5/8: 117.9, 7/8: 120.9).
    const int cus = beside ? device_cus() * 3 / 4 : device_cus();
    MfmaArgs g{};
    g.w[0] = static_cast<const uint8_t*>(layer->shared_gate);
    g.w[1] = static_cast<const uint8_t*>(layer->shared_up);
    g.rows = Is;
    g.K = H;
    g.x = x;
    g.ldx = H;
    g.x_div = 1;
    g.tile_bound = static_cast<int32_t>(tiles);
    g.n_routes = static_cast<int32_t>(T);
    g.out = at<uint16_t>(ws, L.h_shared);
    g.ldo = Is;
    g.ksplit = 1;
    const MfmaPlan pg = plan_mfma(UQM_BF16, 2, Is, H, nb, tiles, cus, 1);
    int rc = hip_check(launch_expert_mfma(UQM_BF16, 2, g, pg.nb, pg.kw, pg.mw, cus, stream), "shared gate/up MFMA launch");
    if (rc) return rc;
    MfmaArgs d = g;
    d.w[0] = static_cast<const uint8_t*>(layer->shared_down);
    d.w[1] = nullptr;
    d.rows = H;
    d.K = Is;
    d.x = at<uint16_t>(ws, L.h_shared);
    d.ldx = Is;
    d.out = at<float>(ws, L.y_shared);
    d.ldo = H;
    d.part_stride = T * H;
    const MfmaPlan pd = plan_mfma(UQM_BF16, 1, H, Is, nb, tiles, cus, T > 1 ? kMaxSplit : 1);
    d.ksplit = pd.ksplit;
    *parts = pd.ksplit;
    return hip_check(launch_expert_mfma(UQM_BF16, 1, d, pd.nb, pd.kw, pd.mw, cus, stream), "shared down MFMA launch");
  }
  const int nt = static_cast<int>(T < 4 ? T : 4);
  GemvArgs g{};
  g.w[0] = static_cast<const uint8_t*>(layer->shared_gate);
  g.w[1] = static_cast<const uint8_t*>(layer->shared_up);
  g.rows = Is;
  g.K = H;
  g.x = x;
  g.ldx = H;
  g.x_div = 1;
  g.n_routes = static_cast<int32_t>(T);
  g.out = at<uint16_t>(ws, L.h_shared);
  g.ldo = Is;
  int rc = hip_check(launch_expert_gemv(UQM_BF16, 2, kModeSilu, g, 1, nt, stream), "shared gate/up launch");
  if (rc) return rc;
  GemvArgs d{};
  d.w[0] = static_cast<const uint8_t*>(layer->shared_down);
  d.rows = H;
  d.K = Is;
  d.x = at<uint16_t>(ws, L.h_shared);
  d.ldx = Is;
  d.x_div = 1;
  d.n_routes = static_cast<int32_t>(T);
  d.out = at<float>(ws, L.y_shared);
  d.ldo = H;
  return hip_check(launch_expert_gemv(UQM_BF16, 1, kModeF32, d, 1, nt, stream), "shared down launch");
}

}  // namespace

extern "C" {

int uqm_abi_version(void) { return UQM_ABI_VERSION; }

const char* uqm_last_error(void) { return g_error.c_str(); }

int uqm_device_arch(int device, char* buf, int buf_len) {
  if (buf == nullptr || buf_len <= 0) return fail(UQM_ERR_ARGUMENT, "buffer is NULL");
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return fail(UQM_ERR_HIP, "hipGetDeviceProperties(%d): %s", device, hipGetErrorString(e));
  snprintf(buf, static_cast<size_t>(buf_len), "%s", prop.gcnArchName);
  return UQM_OK;
}

size_t uqm_moe_workspace_bytes(int64_t tokens, int64_t hidden_size, int64_t intermediate_size,
                               int64_t shared_intermediate_size, int64_t num_experts, int64_t top_k) {
  if (tokens < 0 || hidden_size <= 0 || intermediate_size <= 0 || shared_intermediate_size < 0 || num_experts <= 0 ||
      top_k <= 0)
    return 0;
  return layout(tokens, hidden_size, intermediate_size, shared_intermediate_size, num_experts, top_k).total;
}

static int linear_impl(int enc, const void* input, int64_t rows, const void* w, const float* s, int64_t out_features,
                       int64_t in_features, int64_t group_size, void* output, void* stream) {
  using namespace uqm;
  int rc = check_device();
  if (rc) return rc;
  if (rows < 0 || out_features <= 0) return fail(UQM_ERR_ARGUMENT, "rows must be >= 0 and out_features > 0");
  if ((rc = check_matrix(enc, in_features, group_size, w, s, "linear"))) return rc;
  if (rows == 0) return UQM_OK;
  if (input == nullptr || output == nullptr || !aligned16(input)) return fail(UQM_ERR_ARGUMENT, "input must be a 16-byte aligned device pointer and output non-NULL");
  if ((rc = check_lds(enc, in_features, 4))) return rc;
  GemvArgs a{};
  a.w[0] = static_cast<const uint8_t*>(w);
  a.s[0] = s;
  a.rows = out_features;
  a.K = in_features;
  a.group = group_size;
  a.x = static_cast<const uint16_t*>(input);
  a.ldx = in_features;
  a.x_div = 1;
  a.n_routes = static_cast<int32_t>(rows);
  a.out = output;
  a.ldo = out_features;
  const int nt = static_cast<int>(rows < 4 ? rows : 4);
  return hip_check(launch_expert_gemv(enc, 1, kModeBF16, a, 1, nt, static_cast<hipStream_t>(stream)), "linear launch");
}

int uqm_q4_linear(const void* input, int64_t rows, const void* packed, const float* scales, int64_t out_features,
                  int64_t in_features, int64_t group_size, void* output, void* stream) {
  return linear_impl(UQM_Q4, input, rows, packed, scales, out_features, in_features, group_size, output, stream);
}

int uqm_q8_linear(const void* input, int64_t rows, const void* quantized, const float* scales, int64_t out_features,
                  int64_t in_features, int64_t group_size, void* output, void* stream) {
  return linear_impl(UQM_Q8, input, rows, quantized, scales, out_features, in_features, group_size, output, stream);
}

int uqm_bf16_linear(const void* input, int64_t rows, const void* weight, int64_t out_features, int64_t in_features,
                    void* output, void* stream) {
  return linear_impl(UQM_BF16, input, rows, weight, nullptr, out_features, in_features, 0, output, stream);
}

int uqm_route_permute(const int64_t* expert_indices, int64_t tokens, int64_t top_k, int64_t num_experts,
                      int64_t* route_order, int64_t* expert_offsets, void* workspace, size_t workspace_bytes,
                      void* stream) {
  using namespace uqm;
  int rc = check_device();
  if (rc) return rc;
  if (tokens < 0 || top_k <= 0 || num_experts <= 0 || num_experts > 256)
    return fail(UQM_ERR_ARGUMENT, "tokens >= 0, top_k > 0 and num_experts in [1, 256] are required");
  if (route_order == nullptr || expert_offsets == nullptr || (tokens > 0 && expert_indices == nullptr))
    return fail(UQM_ERR_ARGUMENT, "route tensors must be non-NULL");
  const Layout L = layout(tokens, 8, 8, 0, num_experts, top_k);
  if (workspace == nullptr || workspace_bytes < L.total)
    return fail(UQM_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu required", workspace_bytes, L.total);
  if ((rc = note_layout(workspace, L, {num_experts, top_k, 8, 0}, false, static_cast<hipStream_t>(stream)))) return rc;
  RouteTables rt{at<int32_t>(workspace, L.route_expert), at<int32_t>(workspace, L.route_order),
                 at<int32_t>(workspace, L.expert_offsets), at<int32_t>(workspace, L.active_experts),
                 at<int32_t>(workspace, L.counters), at<int32_t>(workspace, L.tiles),
                 at<int32_t>(workspace, L.counters) + 1};
  return hip_check(launch_route_permute(nullptr, expert_indices, tokens * top_k, num_experts, rt, route_order,
                                        expert_offsets, 0, static_cast<hipStream_t>(stream)),
                   "permute launch");
}

int uqm_router_topk(const void* hidden, int64_t tokens, int64_t hidden_size, const void* router, int64_t num_experts,
                    int64_t top_k, int32_t norm_topk_prob, void* logits, void* routing_weights,
                    int64_t* expert_indices, void* workspace, size_t workspace_bytes, void* stream) {
  using namespace uqm;
  int rc = check_device();
  if (rc) return rc;
  if (tokens < 0 || num_experts <= 0 || num_experts > 256 || top_k <= 0 || top_k > 64 || top_k > num_experts)
    return fail(UQM_ERR_ARGUMENT, "need tokens >= 0, 1 <= top_k <= min(64, E), E <= 256");
  if ((rc = check_matrix(UQM_BF16, hidden_size, 0, router, nullptr, "router"))) return rc;
  if (tokens == 0) return UQM_OK;
  if (hidden == nullptr || !aligned16(hidden) || routing_weights == nullptr || expert_indices == nullptr)
    return fail(UQM_ERR_ARGUMENT, "hidden (16-byte aligned), routing_weights and expert_indices are required");
  if ((rc = check_lds(UQM_BF16, hidden_size, 4))) return rc;
  const Layout L = layout(tokens, hidden_size, 8, 0, num_experts, top_k);
  if (workspace == nullptr || workspace_bytes < L.total)
    return fail(UQM_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu required", workspace_bytes, L.total);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if ((rc = note_layout(workspace, L, {num_experts, top_k, 8, 0}, false, s))) return rc;
  if (router_uses_mfma(hidden_size, tokens))
    return run_router_mfma(router, nullptr, num_experts, static_cast<const uint16_t*>(hidden), tokens, hidden_size,
                           top_k, norm_topk_prob, L, workspace, static_cast<uint16_t*>(routing_weights),
                           expert_indices, nullptr, nullptr, static_cast<uint16_t*>(logits), nullptr, 0, nullptr, s);
  uint16_t* lg = logits != nullptr ? static_cast<uint16_t*>(logits) : at<uint16_t>(workspace, L.logits);
  GemvArgs a{};
  a.w[0] = static_cast<const uint8_t*>(router);
  a.rows = num_experts;
  a.K = hidden_size;
  a.x = static_cast<const uint16_t*>(hidden);
  a.ldx = hidden_size;
  a.x_div = 1;
  a.n_routes = static_cast<int32_t>(tokens);
  a.out = lg;
  a.ldo = num_experts;
  if ((rc = hip_check(launch_expert_gemv(UQM_BF16, 1, kModeBF16, a, 1, static_cast<int>(tokens < 4 ? tokens : 4), s),
                      "router launch")))
    return rc;
  return hip_check(launch_route_topk(lg, num_experts, tokens, num_experts, top_k, norm_topk_prob,
                                     static_cast<uint16_t*>(routing_weights), expert_indices, nullptr, nullptr, s),
                   "top-k launch");
}

int uqm_moe_forward(const uqm_expert_weights* weights, const void* hidden, int64_t tokens,
                    const int64_t* expert_indices, const void* routing_weights, int64_t top_k, void* output,
                    void* workspace, size_t workspace_bytes, void* stream) {
  using namespace uqm;
  int rc = check_device();
  if (rc) return rc;
  if ((rc = check_experts(weights))) return rc;
  if (tokens < 0 || top_k <= 0 || top_k > 64) return fail(UQM_ERR_ARGUMENT, "need tokens >= 0 and 1 <= top_k <= 64");
  if (tokens == 0) return UQM_OK;
  if (hidden == nullptr || !aligned16(hidden) || expert_indices == nullptr || routing_weights == nullptr ||
      output == nullptr || !aligned16(output))
    return fail(UQM_ERR_ARGUMENT, "hidden/output (16-byte aligned), expert_indices and routing_weights are required");
  if (weights->hidden_size % 4 != 0) return fail(UQM_ERR_ARGUMENT, "hidden size must be a multiple of 4");
  if ((rc = check_lds(weights->encoding, weights->hidden_size, 4))) return rc;
  if ((rc = check_lds(weights->encoding, weights->intermediate_size, 4))) return rc;
  const Layout L = layout(tokens, weights->hidden_size, weights->intermediate_size, 0, weights->num_experts, top_k);
  if (workspace == nullptr || workspace_bytes < L.total || !aligned16(workspace))
    return fail(UQM_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu required (or misaligned)",
                workspace_bytes, L.total);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t H = weights->hidden_size, I = weights->intermediate_size, E = weights->num_experts;
  // One or two tokens: the fused single-token kernel with the caller's routes
  // (no router), one launch per token.
  const bool fused = tokens <= kFusedMaxTokens && g_opt_fused.load(std::memory_order_relaxed) != 0 &&
                     fused_config_id(weights->encoding, H, I, 0, top_k, E) >= 0 &&
                     (weights->encoding == UQM_BF16 || (H % weights->group_size == 0 && I % weights->group_size == 0));
  if ((rc = note_layout(workspace, L, {E, top_k, I, 0}, fused, s))) return rc;
  if (fused) {
    FusedArgs fa{};
    fa.eg = static_cast<const uint8_t*>(weights->gate);
    fa.eu = static_cast<const uint8_t*>(weights->up);
    fa.ed = static_cast<const uint8_t*>(weights->down);
    fa.egs = weights->gate_scales;
    fa.eus = weights->up_scales;
    fa.eds = weights->down_scales;
    fa.H = H;
    fa.I = I;
    fa.Is = 0;
    fa.E = static_cast<int>(E);
    fa.k = static_cast<int>(top_k);
    fa.group = weights->encoding == UQM_BF16 ? 1 : weights->group_size;
    fa.wait_ticks = fused_wait_ticks();
    fa.sync = at<uint32_t>(workspace, L.fused_sync);
    fa.hs = at<uint32_t>(workspace, L.fused_hs);
    fa.hr = at<uint32_t>(workspace, L.fused_hr);
    fa.lgt = at<uint64_t>(workspace, L.fused_lgt);
    for (int64_t t = 0; t < tokens; ++t) {
      fa.x = static_cast<const uint16_t*>(hidden) + t * H;
      fa.out = static_cast<uint16_t*>(output) + t * H;
      fa.routes_in = expert_indices + t * top_k;
      fa.weights_in = static_cast<const uint16_t*>(routing_weights) + t * top_k;
      if ((rc = hip_check(launch_moe_decode_fused(weights->encoding, fa, s), "fused routed launch"))) return rc;
    }
    return UQM_OK;
  }
  RouteTables rt{at<int32_t>(workspace, L.route_expert), at<int32_t>(workspace, L.route_order),
                 at<int32_t>(workspace, L.expert_offsets), at<int32_t>(workspace, L.active_experts),
                 at<int32_t>(workspace, L.counters), at<int32_t>(workspace, L.tiles),
                 at<int32_t>(workspace, L.counters) + 1};
  const int tile_tokens = routed_tile_tokens(weights, tokens, top_k);
  if ((rc = hip_check(launch_route_permute(nullptr, expert_indices, tokens * top_k, weights->num_experts, rt, nullptr,
                                           nullptr, tile_tokens, s),
                      "permute launch")))
    return rc;
  int parts = 1;
  if ((rc = run_routed(weights, static_cast<const uint16_t*>(hidden), tokens, top_k, L, workspace, tile_tokens, &parts,
                       s)))
    return rc;
  return hip_check(launch_combine(at<float>(workspace, L.y_routed), parts, tokens * top_k * weights->hidden_size,
                                  static_cast<const uint16_t*>(routing_weights), expert_indices, tokens, top_k,
                                  weights->num_experts, weights->hidden_size, nullptr, 1, 0, nullptr,
                                  static_cast<uint16_t*>(output), s),
                   "combine launch");
}

namespace {

// RMSNorm applied to the block's input (rms == false: none).
struct InputNorm {
  bool rms;
  const void* weight;
  float eps;
};

int moe_layer_impl(const uqm_layer_weights* layer, const void* hidden, int64_t tokens, InputNorm norm, void* output,
                   void* logits, void* routing_weights, int64_t* expert_indices, void* workspace,
                   size_t workspace_bytes, void* stream, bool allow_side_stream = true) {
  using namespace uqm;
  int rc = check_device();
  if (rc) return rc;
  if (layer == nullptr) return fail(UQM_ERR_ARGUMENT, "layer descriptor is NULL");
  const uqm_expert_weights* w = &layer->experts;
  if ((rc = check_experts(w))) return rc;
  const int64_t E = w->num_experts, H = w->hidden_size, k = layer->top_k;
  if (tokens < 0 || k <= 0 || k > 64 || k > E) return fail(UQM_ERR_ARGUMENT, "need tokens >= 0 and 1 <= top_k <= min(64, E)");
  if ((rc = check_matrix(UQM_BF16, H, 0, layer->router, nullptr, "router"))) return rc;
  const int64_t Is = layer->has_shared ? layer->shared_intermediate_size : 0;
  if (layer->has_shared) {
    if (Is <= 0) return fail(UQM_ERR_ARGUMENT, "shared_intermediate_size must be positive");
    if ((rc = check_matrix(UQM_BF16, H, 0, layer->shared_gate, nullptr, "shared gate"))) return rc;
    if ((rc = check_matrix(UQM_BF16, H, 0, layer->shared_up, nullptr, "shared up"))) return rc;
    if ((rc = check_matrix(UQM_BF16, Is, 0, layer->shared_down, nullptr, "shared down"))) return rc;
    if ((rc = check_matrix(UQM_BF16, H, 0, layer->shared_expert_gate, nullptr, "shared expert gate"))) return rc;
    if ((rc = check_lds(UQM_BF16, Is, 4))) return rc;
  }
  if (tokens == 0) return UQM_OK;
  if (hidden == nullptr || !aligned16(hidden) || output == nullptr || !aligned16(output))
    return fail(UQM_ERR_ARGUMENT, "hidden and output must be 16-byte aligned device pointers");
  if (H % 4 != 0) return fail(UQM_ERR_ARGUMENT, "hidden size must be a multiple of 4");
  if ((rc = check_lds(w->encoding, H, 4))) return rc;
  if ((rc = check_lds(w->encoding, w->intermediate_size, 4))) return rc;
  const Layout L = layout(tokens, H, w->intermediate_size, Is, E, k);
  if (workspace == nullptr || workspace_bytes < L.total || !aligned16(workspace))
    return fail(UQM_ERR_WORKSPACE, "workspace of %zu bytes is smaller than the %zu required (or misaligned)",
                workspace_bytes, L.total);
  if (norm.rms && !(norm.eps >= 0.f)) return fail(UQM_ERR_ARGUMENT, "RMSNorm eps must be >= 0");
  if (norm.rms && norm.weight != nullptr && !aligned16(norm.weight))
    return fail(UQM_ERR_ARGUMENT, "RMSNorm weight must be a 16-byte aligned device pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* x = static_cast<const uint16_t*>(hidden);
  const int nt = static_cast<int>(tokens < 4 ? tokens : 4);
  const int64_t rows_router = E + (layer->has_shared ? 1 : 0);

  // One or two tokens: one persistent launch per token for the whole block
  // (two tokens: 2 x 20.7 us against 57.9 us on the multi-launch path for c2
  // shapes; three: 62.1 against 63.1).
  const bool fused = tokens <= kFusedMaxTokens && g_opt_fused.load(std::memory_order_relaxed) != 0 &&
                     fused_config_id(w->encoding, H, w->intermediate_size, Is, k, E) >= 0 &&
                     (w->encoding == UQM_BF16 || (H % w->group_size == 0 && w->intermediate_size % w->group_size == 0));
  if ((rc = note_layout(workspace, L, {E, k, w->intermediate_size, Is}, fused, s))) return rc;
  if (fused) {
    FusedArgs fa{};
    fa.x = x;
    fa.rms = norm.rms ? 1 : 0;
    fa.rms_w = static_cast<const uint16_t*>(norm.weight);
    fa.rms_eps = norm.eps;
    fa.router = static_cast<const uint8_t*>(layer->router);
    fa.shared_expert_gate = static_cast<const uint8_t*>(layer->shared_expert_gate);
    fa.sg_w = static_cast<const uint8_t*>(layer->shared_gate);
    fa.su_w = static_cast<const uint8_t*>(layer->shared_up);
    fa.sd_w = static_cast<const uint8_t*>(layer->shared_down);
    fa.eg = static_cast<const uint8_t*>(w->gate);
    fa.eu = static_cast<const uint8_t*>(w->up);
    fa.ed = static_cast<const uint8_t*>(w->down);
    fa.egs = w->gate_scales;
    fa.eus = w->up_scales;
    fa.eds = w->down_scales;
    fa.H = H;
    fa.I = w->intermediate_size;
    fa.Is = Is;
    fa.E = static_cast<int>(E);
    fa.k = static_cast<int>(k);
    fa.group = w->encoding == UQM_BF16 ? 1 : w->group_size;
    fa.norm = layer->norm_topk_prob;
    fa.wait_ticks = fused_wait_ticks();
    fa.sync = at<uint32_t>(workspace, L.fused_sync);
    fa.hs = at<uint32_t>(workspace, L.fused_hs);
    fa.hr = at<uint32_t>(workspace, L.fused_hr);
    fa.lgt = at<uint64_t>(workspace, L.fused_lgt);
    for (int64_t t = 0; t < tokens; ++t) {
      fa.x = x + t * H;
      fa.out = static_cast<uint16_t*>(output) + t * H;
      fa.logits_out = logits != nullptr ? static_cast<uint16_t*>(logits) + t * E : nullptr;
      fa.weights_out = routing_weights != nullptr ? static_cast<uint16_t*>(routing_weights) + t * k : nullptr;
      fa.indices_out = expert_indices != nullptr ? expert_indices + t * k : nullptr;
      if ((rc = hip_check(launch_moe_decode_fused(w->encoding, fa, s), "fused block launch"))) return rc;
    }
    return UQM_OK;
  }

  // 0. input RMSNorm into the workspace
  if (norm.rms) {
    uint16_t* xn = at<uint16_t>(workspace, L.normed);
    if ((rc = hip_check(launch_rmsnorm(x, tokens, H, static_cast<const uint16_t*>(norm.weight), norm.eps, xn, s),
                        "rmsnorm launch")))
      return rc;
    x = xn;
  }
  // 4 (forked). shared expert on the side stream, beside steps 1-3
  int ys_parts = 1;
  std::unique_lock<std::mutex> side_lock;
  SideStream* side = nullptr;
  // Once forked, the side stream is joined back into the caller's stream on
  // every return path (an error return included), so that a graph capture of
  // the caller's stream never ends with an unjoined branch.
  struct JoinOnExit {
    hipStream_t caller;
    SideStream* side = nullptr;
    ~JoinOnExit() {
      if (side == nullptr) return;
      (void)hipEventRecord(side->join, side->stream);
      (void)hipStreamWaitEvent(caller, side->join, 0);
    }
  } join_on_exit{s};
  if (layer->has_shared) {
    if (allow_side_stream && g_opt_overlap_shared.load(std::memory_order_relaxed) != 0) {
      side_lock = std::unique_lock<std::mutex>(g_side_mu);
      side = side_stream(s);
    }
    // the fork point: the shared expert reads only the input, so it waits for
    // nothing the routing chain does; its launches follow the routing chain's
    // (below)
    if (side != nullptr && (rc = hip_check(hipEventRecord(side->fork, s), "fork record"))) return rc;
  }
  // 1-2. router logits (+ shared-gate logit in column E), top-k
  uint16_t* wout = routing_weights != nullptr ? static_cast<uint16_t*>(routing_weights) : at<uint16_t>(workspace, L.weights);
  int64_t* iout = expert_indices != nullptr ? expert_indices : at<int64_t>(workspace, L.indices);
  float* sg = layer->has_shared ? at<float>(workspace, L.sg) : nullptr;
  RouteTables rt{at<int32_t>(workspace, L.route_expert), at<int32_t>(workspace, L.route_order),
                 at<int32_t>(workspace, L.expert_offsets), at<int32_t>(workspace, L.active_experts),
                 at<int32_t>(workspace, L.counters), at<int32_t>(workspace, L.tiles),
                 at<int32_t>(workspace, L.counters) + 1};
  // top-k and the permutation in one launch when the routes fit one workgroup
  const int tile_tokens = routed_tile_tokens(w, tokens, k);
  const bool fuse_permute = route_topk_permute_fits(tokens, k);
  uint32_t* permute_counter = at<uint32_t>(workspace, L.fused_sync) + kSyncPermuteDone;
  if (router_uses_mfma(H, tokens)) {
    if ((rc = run_router_mfma(layer->router, layer->has_shared ? layer->shared_expert_gate : nullptr, E, x, tokens, H,
                              k, layer->norm_topk_prob, L, workspace, wout, iout, rt.route_expert, sg,
                              static_cast<uint16_t*>(logits), fuse_permute ? &rt : nullptr, tile_tokens,
                              permute_counter, s)))
      return rc;
  } else {
    uint16_t* lg = at<uint16_t>(workspace, L.logits);
    GemvArgs r{};
    r.w[0] = static_cast<const uint8_t*>(layer->router);
    if (layer->has_shared) {
      r.w_tail = static_cast<const uint8_t*>(layer->shared_expert_gate);
      r.tail_from = E;
    }
    r.rows = rows_router;
    r.K = H;
    r.x = x;
    r.ldx = H;
    r.x_div = 1;
    r.n_routes = static_cast<int32_t>(tokens);
    r.out = lg;
    r.ldo = rows_router;
    if ((rc = hip_check(launch_expert_gemv(UQM_BF16, 1, kModeBF16, r, 1, nt, s), "router launch"))) return rc;
    if (fuse_permute) {
      if ((rc = hip_check(launch_route_topk_permute(lg, nullptr, 1, 0, rows_router, tokens, E, k,
                                                    layer->norm_topk_prob, wout, iout, sg, nullptr, rt, tile_tokens,
                                                    permute_counter, s),
                          "top-k + permute launch")))
        return rc;
    } else if ((rc = hip_check(launch_route_topk(lg, rows_router, tokens, E, k, layer->norm_topk_prob, wout, iout,
                                                 rt.route_expert, sg, s),
                               "top-k launch"))) {
      return rc;
    }
    if (logits != nullptr) {
      if ((rc = hip_check(hipMemcpy2DAsync(logits, 2 * E, lg, 2 * rows_router, 2 * E, tokens, hipMemcpyDeviceToDevice,
                                           s),
                          "logits copy")))
        return rc;
    }
  }
  if (!fuse_permute &&
      (rc = hip_check(launch_route_permute(rt.route_expert, nullptr, tokens * k, E, rt, nullptr, nullptr, tile_tokens, s),
                      "permute launch")))
    return rc;
  // The shared expert on the side stream, launched after the router and the
  // top-k but dependent only on the fork: a HIP graph replay dispatches the
  // nodes in this order, so the router's small grid goes out before the shared
  // expert's persistent grids instead of ~5.6 us behind them (graph replay:
  // batch 32 101.9-102.1 vs 102.9-103.2 us per call, T = 16 82.0-82.1 vs
  // 88.6-88.7, c4 164.4-164.6 vs 167.6-167.7).
  if (side != nullptr) {
    if ((rc = hip_check(hipStreamWaitEvent(side->stream, side->fork, 0), "fork wait"))) return rc;
    join_on_exit.side = side;
    if ((rc = run_shared(layer, x, tokens, H, L, workspace, &ys_parts, true, side->stream))) return rc;
  }
  // 3. routed experts
  int yr_parts = 1;
  if ((rc = run_routed(w, x, tokens, k, L, workspace, tile_tokens, &yr_parts, s))) return rc;
  // 4. shared expert (joined, or in order on the caller's stream)
  if (side != nullptr) {
    join_on_exit.side = nullptr;
    if ((rc = hip_check(hipEventRecord(side->join, side->stream), "join record")) ||
        (rc = hip_check(hipStreamWaitEvent(s, side->join, 0), "join wait")))
      return rc;
  } else if (layer->has_shared && (rc = run_shared(layer, x, tokens, H, L, workspace, &ys_parts, false, s))) {
    return rc;
  }
  // 5. combine
  return hip_check(launch_combine(at<float>(workspace, L.y_routed), yr_parts, tokens * k * H, wout, iout, tokens, k, E,
                                  H, layer->has_shared ? at<float>(workspace, L.y_shared) : nullptr, ys_parts,
                                  tokens * H, sg, static_cast<uint16_t*>(output), s),
                   "combine launch");
}

}  // namespace

}  // extern "C"

namespace uqm {

int api_fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int moe_layer_on_workspace(const uqm_layer_weights* layer, const void* hidden, int64_t tokens, void* output,
                           void* logits, void* routing_weights, int64_t* expert_indices, void* workspace,
                           size_t workspace_bytes, bool side_stream, void* stream) {
  return moe_layer_impl(layer, hidden, tokens, InputNorm{false, nullptr, 0.f}, output, logits, routing_weights,
                        expert_indices, workspace, workspace_bytes, stream, side_stream);
}

}  // namespace uqm

extern "C" {

int uqm_moe_layer(const uqm_layer_weights* layer, const void* hidden, int64_t tokens, void* output, void* logits,
                  void* routing_weights, int64_t* expert_indices, void* workspace, size_t workspace_bytes,
                  void* stream) {
  return moe_layer_impl(layer, hidden, tokens, InputNorm{false, nullptr, 0.f}, output, logits, routing_weights,
                        expert_indices, workspace, workspace_bytes, stream);
}

int uqm_norm_moe_layer(const uqm_layer_weights* layer, const void* hidden, int64_t tokens, const void* norm_weight,
                       float eps, void* output, void* logits, void* routing_weights, int64_t* expert_indices,
                       void* workspace, size_t workspace_bytes, void* stream) {
  return moe_layer_impl(layer, hidden, tokens, InputNorm{true, norm_weight, eps}, output, logits, routing_weights,
                        expert_indices, workspace, workspace_bytes, stream);
}

int uqm_set_option(int option, int64_t value) {
  switch (option) {
    case UQM_OPT_FUSED_DECODE:
      g_opt_fused.store(value != 0 ? 1 : 0);
      return UQM_OK;
    case UQM_OPT_MFMA_MIN_TOKENS:
      if (value < 0) return fail(UQM_ERR_ARGUMENT, "token threshold must be >= 0");
      g_opt_mfma_min_tokens.store(value);
      return UQM_OK;
    case UQM_OPT_OVERLAP_SHARED:
      g_opt_overlap_shared.store(value != 0 ? 1 : 0);
      return UQM_OK;
    case UQM_OPT_STREAM_MAX_ROUTES:
      if (value < 0) return fail(UQM_ERR_ARGUMENT, "routes threshold must be >= 0");
      g_opt_stream_max_routes.store(value);
      return UQM_OK;
    case UQM_OPT_FUSED_WAIT_US:
      if (value < 0 || value > 10000000) return fail(UQM_ERR_ARGUMENT, "wait budget must be in [0, 10^7] us");
      g_opt_fused_wait_us.store(value);
      return UQM_OK;
    default:
      return fail(UQM_ERR_ARGUMENT, "unknown option %d", option);
  }
}

int uqm_workspace_status(void* workspace, size_t workspace_bytes, void* stream) {
  if (workspace == nullptr || workspace_bytes < 4 * uqm::kSyncWords)
    return fail(UQM_ERR_WORKSPACE, "workspace is NULL or too small");
  static_assert(uqm::kSyncExpired == uqm::kSyncError + 1, "error and expired words are adjacent");
  uint32_t words[2] = {0, 0};  // error word, expired-launch word
  uint32_t* dev = static_cast<uint32_t*>(workspace) + uqm::kSyncError;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc;
  if ((rc = hip_check(hipMemcpyAsync(words, dev, 8, hipMemcpyDeviceToHost, s), "status read"))) return rc;
  if ((rc = hip_check(hipStreamSynchronize(s), "status sync"))) return rc;
  if (words[0] == 0 && words[1] == 0) return UQM_OK;
  const uint32_t zero[2] = {0, 0};
  if ((rc = hip_check(hipMemcpyAsync(dev, zero, 8, hipMemcpyHostToDevice, s), "status clear"))) return rc;
  if ((rc = hip_check(hipStreamSynchronize(s), "status sync"))) return rc;
  if (words[0] == 0) return UQM_OK;  // only a stale expired marker: cleared
  return fail(UQM_ERR_HIP,
              "a fused launch on this workspace hit its wait bound (error word %u, launch tag %u): its output is "
              "invalid",
              words[0], words[1]);
}

int uqm_rmsnorm(const void* input, int64_t rows, int64_t hidden_size, const void* weight, float eps, void* output,
                void* stream) {
  using namespace uqm;
  int rc = check_device();
  if (rc) return rc;
  if (rows < 0 || hidden_size <= 0) return fail(UQM_ERR_ARGUMENT, "rows >= 0 and hidden_size > 0 required");
  if (rows == 0) return UQM_OK;
  if (input == nullptr || output == nullptr) return fail(UQM_ERR_ARGUMENT, "input and output are required");
  return hip_check(launch_rmsnorm(static_cast<const uint16_t*>(input), rows, hidden_size,
                                  static_cast<const uint16_t*>(weight), eps, static_cast<uint16_t*>(output),
                                  static_cast<hipStream_t>(stream)),
                   "rmsnorm launch");
}

int uqm_dequantize(int32_t encoding, const void* data, const float* scales, int64_t elements, int64_t group_size,
                   void* output, void* stream) {
  using namespace uqm;
  int rc = check_device();
  if (rc) return rc;
  if (encoding != UQM_Q4 && encoding != UQM_Q8)
    return fail(UQM_ERR_ARGUMENT, "dequantize takes a Q4 or Q8 tensor, not encoding %d", encoding);
  if (elements < 0 || elements % 8 != 0) return fail(UQM_ERR_ARGUMENT, "element count must be a multiple of 8");
  if (group_size <= 0 || group_size % 8 != 0)
    return fail(UQM_ERR_ARGUMENT, "group size %lld must be a positive multiple of 8", (long long)group_size);
  if (elements == 0) return UQM_OK;
  if (data == nullptr || scales == nullptr || output == nullptr)
    return fail(UQM_ERR_ARGUMENT, "data, scales and output are required");
  if (!aligned16(data) || !aligned16(output) || reinterpret_cast<uintptr_t>(scales) % 4 != 0)
    return fail(UQM_ERR_ARGUMENT, "data and output must be 16-byte aligned, scales 4-byte aligned");
  return hip_check(launch_dequantize(encoding == UQM_Q4, data, scales, elements, group_size, output,
                                     static_cast<hipStream_t>(stream)),
                   "dequantize launch");
}

}  // extern "C"
