// Internal (C++) interfaces between the kernel translation units and the
// extern "C" entry points in uqm_api.hip. Nothing here is exported.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "uqm_device.h"

struct uqm_layer_weights;  // include/uma_qmoe_hip.h

namespace uqm {

enum GemvMode : int { kModeSilu = 0, kModeF32 = 1, kModeBF16 = 2 };

// One expert-grouped GEMV launch. Matrix m of expert e, row r starts at
// w[m] + (e * rows + r) * row_bytes; its scale for chunk c is
// s[m][e * scales_per_expert + (r * K + c * elems) / group]: groups run over
// each expert's flattened tensor, scales_per_expert = ceil(rows * K / group).
struct GemvArgs {
  const uint8_t* w[2];
  // Optional separate storage for rows >= tail_from of matrix 0 (expert 0
  // only): lets the router GEMV append the shared-expert gate row.
  const uint8_t* w_tail;
  int64_t tail_from;
  const float* s[2];
  int64_t rows;   // output rows per expert
  int64_t K;      // input features
  int64_t group;  // scale group size in elements (Q4/Q8)
  int64_t scales_per_expert;
  const uint16_t* x;  // bf16 activations
  int64_t ldx;        // elements between activation rows
  int32_t x_div;      // activation row of route r is r / x_div
  const int32_t* route_order;     // routes sorted by expert; null = identity
  const int32_t* expert_offsets;  // [E+1] into route_order; null = one group
  const int32_t* active_experts;  // compact list of experts with routes; null = blockIdx.y
  const int32_t* active_count;    // device count of active experts; null = gridDim.y
  int32_t n_routes;               // route count when expert_offsets is null
  void* out;                      // output row = route id
  int64_t ldo;
};

hipError_t launch_expert_gemv(int enc, int nmat, int mode, const GemvArgs& a, int grid_y, int nt,
                              hipStream_t stream);
size_t gemv_lds_bytes(int enc, int64_t K, int nt);

// Expert-grouped streaming GEMV (uqm_stream.hip): a persistent grid splits
// the (active expert, row) pairs evenly over its waves; activations of up to
// nt routes of an expert live in registers. Needs route_order,
// expert_offsets, active_experts and active_count; max_active bounds
// *active_count (grid sizing only). Writes out[route * ldo + row].
bool stream_supported(int enc, int64_t K, int64_t group);
hipError_t launch_routed_stream(int enc, int nmat, int mode, const GemvArgs& a, int nt, int64_t max_active, int cus,
                                hipStream_t stream);

// Expert-grouped GEMM on the MFMA cores (uqm_mfma.hip). Output block =
// rows of one expert x one tile of up to 16*nb routes. Matrix m of expert e,
// row r starts at w[m] + (e * rows + r) * row_bytes; scales as GemvArgs.
struct MfmaArgs {
  const uint8_t* w[2];
  const float* s[2];
  // Optional (single row group per work item only, i.e. kw 4 with mw 4): rows
  // >= rows_valid read row rows_valid - 1 (their outputs are padding), and rows
  // >= tail_from of matrix 0 come from w_tail (the router's appended
  // shared-expert gate row).
  const uint8_t* w_tail;
  int64_t tail_from;
  int64_t rows_valid;  // 0 = rows
  int64_t rows;  // output rows per expert (multiple of the workgroup's row block)
  int64_t K;     // input features (multiple of 128)
  int64_t group;
  int64_t scales_per_expert;  // set by the launcher
  const uint16_t* x;          // bf16 activations
  int64_t ldx;
  int32_t x_div;                  // activation row of route r is r / x_div
  const int32_t* route_order;     // routes sorted by expert; null = identity
  const int32_t* expert_offsets;  // [E+1] into route_order (with tiles)
  const int32_t* tiles;           // [tile][2] = (expert, first index into route_order); null = one expert
  const int32_t* tile_count;      // device count of tiles (with tiles)
  int32_t tile_bound;             // tiles the grid covers (>= the device count)
  int32_t n_routes;               // routes when tiles is null
  void* out;                      // kModeSilu: bf16 [route, ldo]; kModeF32: fp32 [split][route, ldo]
  int64_t ldo;
  int64_t part_stride;  // elements between K-split partial outputs
  int32_t ksplit;       // workgroups along K (kModeF32 only)
  int32_t row_blocks;   // set by the launcher
  // Order of the (row block, route tile) work items: kOrderTileFastest shares
  // an expert's rows between its tiles, kOrderRowFastest shares a tile's
  // activations between the row blocks, kOrderAuto takes row blocks fastest
  // when the device tile list has fewer than 1.5 tiles per active expert.
  int32_t order;
  const int32_t* active_count;  // device count of active experts (kOrderAuto)
};
constexpr int kOrderTileFastest = 0, kOrderRowFastest = 1, kOrderAuto = 2;

bool mfma_supported(int enc, int64_t rows, int64_t K, int64_t group);
// nmat 2 = gate/up with the SiLU epilogue (bf16 out), 1 = FP32 rows. nb: 16-route
// tiles per work item (1, 2; 4 and (BF16) 8 with mw 4); kw: waves along K (1, or
// 4 with nb 1 and mw 4); mw: MMA waves per workgroup (4 or 8; a work item covers
// 16 * mw / kw rows); cus: compute units (the grid is persistent).
hipError_t launch_expert_mfma(int enc, int nmat, const MfmaArgs& a, int nb, int kw, int mw, int cus,
                              hipStream_t stream);

// Route tables produced on the device by the top-k / permutation kernels.
struct RouteTables {
  int32_t* route_expert;    // [T*k] expert id per route (route = t*k + slot)
  int32_t* route_order;     // [T*k] routes stably sorted by expert
  int32_t* expert_offsets;  // [E+1]
  int32_t* active_experts;  // [min(E, T*k)]
  int32_t* active_count;    // [1]
  int32_t* tiles;           // [min(E, T*k) + T*k / tile_tokens][2] (optional)
  int32_t* tile_count;      // [1]
};

// Top-k over bf16 logits [T, ldl] (columns 0..E-1), softmax in FP32, ties to
// the lower expert id. Writes bf16 weights / int64 indices [T, k], the route
// expert table, and (if shared_gate != null) sigmoid of column E.
// launch_route_topk_partials takes the logits as `parts` FP32 partial sums
// [parts][T][ldl] (pstride elements apart), rounds their sum to bf16 (the
// router's bf16 output) and, if logits_out != null, stores it [T, E].
hipError_t launch_route_topk_partials(const float* plog, int parts, int64_t pstride, int64_t ldl, int64_t T,
                                      int64_t E, int64_t k, int norm, uint16_t* weights_out, int64_t* indices_out,
                                      int32_t* route_expert, float* shared_gate, uint16_t* logits_out,
                                      hipStream_t stream);
hipError_t launch_route_topk(const uint16_t* logits, int64_t ldl, int64_t T, int64_t E, int64_t k, int norm,
                             uint16_t* weights_out, int64_t* indices_out, int32_t* route_expert,
                             float* shared_gate, hipStream_t stream);
// Stable counting sort of the route expert table (invalid ids are dropped).
// If order64/offsets64 are non-null, int64 copies are written too. With
// tile_tokens > 0 it also lists, per expert in ascending id, its route tiles
// of at most tile_tokens routes (rt.tiles, rt.tile_count).
hipError_t launch_route_permute(const int32_t* route_expert, const int64_t* indices64, int64_t n_routes,
                                int64_t E, const RouteTables& rt, int64_t* order64, int64_t* offsets64,
                                int tile_tokens, hipStream_t stream);

// out[t, o] = bf16( sum_s w[t,s] * y[t*k+s, o] + sg[t] * ys[t, o] ), where y and
// ys are the sums of y_parts / ys_parts FP32 partials spaced by *_stride elements.
hipError_t launch_combine(const float* y, int y_parts, int64_t y_stride, const uint16_t* weights,
                          const int64_t* indices, int64_t T, int64_t k, int64_t E, int64_t H, const float* ys,
                          int ys_parts, int64_t ys_stride, const float* sg, uint16_t* out, hipStream_t stream);
// Single-token fused MoE block (uqm_fused.hip). Sync words live in `sync`
// (zero before the first launch): a sticky error word the kernel raises when
// one of its bounded waits expires (cleared only by uqm_workspace_status), the
// epoch of the last launch in which a wait expired (the other waits of that
// launch then give up at once), and one launch epoch per workgroup that the
// workgroup advances on every launch.
enum : int { kSyncError = 4, kSyncExpired = 5, kSyncEpochBase = 64 };
// Wall-clock budget of one fused launch's waits, counted by every wave from
// its own start (~20 us is a normal launch).
constexpr int64_t kFusedWaitBudgetUs = 2000;
constexpr int kMaxFusedBlocks = 1024;  // workgroups (one per CU)
constexpr int kSyncWords = kSyncEpochBase + kMaxFusedBlocks;

struct FusedArgs {
  const uint16_t* x;                   // [H] bf16, 16-byte aligned
  const uint16_t* rms_w;               // [H] bf16 RMSNorm weight applied to x (NULL: ones)
  float rms_eps;
  int rms;                             // 1: the block's input is RMSNorm(x)
  const uint8_t* router;               // [E, H] bf16
  const uint8_t* shared_expert_gate;   // [H] bf16 (shared expert only)
  const uint8_t* sg_w;                 // shared gate [Is, H] bf16
  const uint8_t* su_w;                 // shared up   [Is, H] bf16
  const uint8_t* sd_w;                 // shared down [H, Is] bf16
  const uint8_t* eg;                   // routed gate [E, I, H] encoded
  const uint8_t* eu;                   // routed up   [E, I, H]
  const uint8_t* ed;                   // routed down [E, H, I]
  const float* egs;                    // scales (Q4/Q8), group along the row
  const float* eus;
  const float* eds;
  int64_t H, I, Is;
  int E, k, group, norm;
  uint64_t wait_ticks;                 // wait budget in s_memrealtime ticks (kFusedWaitBudgetUs)
  uint32_t* sync;                      // kSyncWords words
  uint32_t* hs;                        // [Is] epoch-tagged shared SiLU products (8-byte aligned)
  uint32_t* hr;                        // [k, I] epoch-tagged routed SiLU products (8-byte aligned)
  uint64_t* lgt;                       // [E + 1] epoch-tagged router logits (fp32), shared gate last
  uint16_t* out;                       // [H]
  uint16_t* logits_out;                // optional [E]
  uint16_t* weights_out;               // optional [k]
  int64_t* indices_out;                // optional [k]
  // Routes given by the caller (routed-only ops, no shared expert): expert
  // ids [k] and bf16 routing weights [k]; NULL: the kernel routes itself.
  const int64_t* routes_in;
  const uint16_t* weights_in;
  // Per-wave phase stamps of a timing harness that defines the kernel's trace
  // hooks (csrc/timeline/fused_timeline.hip); NULL and unused in the library.
  unsigned long long* trace;
};

// Returns >= 0 when a compiled instantiation covers (encoding, H, I, Is, k, E).
int fused_config_id(int enc, int64_t H, int64_t I, int64_t Is, int64_t k, int64_t E);
// One workgroup per CU; needs every workgroup resident at once.
hipError_t launch_moe_decode_fused(int enc, const FusedArgs& a, hipStream_t stream);

hipError_t launch_rmsnorm(const uint16_t* x, int64_t rows, int64_t H, const uint16_t* weight, float eps,
                          uint16_t* out, hipStream_t stream);
// Zeroes `bytes` (a multiple of 16) at the 16-byte aligned device address p,
// with a kernel (no hipMemsetAsync, so that it can be captured into a graph).
hipError_t launch_zero_fill(void* p, size_t bytes, hipStream_t stream);
// out[i] = bf16(q_i * scales[i / group]) over `elements` (a multiple of 8)
// values of a Q4 (q4 = true) or Q8 tensor; group a multiple of 8.
hipError_t launch_dequantize(bool q4, const void* data, const float* scales, int64_t elements, int64_t group,
                             void* out, hipStream_t stream);

// Entry-point plumbing shared by the translation units that export C-ABI
// functions (uqm_api.hip): sets the thread's uqm_last_error message and
// returns `code`; runs uqm_moe_layer on a given workspace, with or without
// the shared-expert side stream.
int api_fail(int code, const char* fmt, ...);
int moe_layer_on_workspace(const uqm_layer_weights* layer, const void* hidden, int64_t tokens, void* output,
                           void* logits, void* routing_weights, int64_t* expert_indices, void* workspace,
                           size_t workspace_bytes, bool side_stream, void* stream);

}  // namespace uqm
