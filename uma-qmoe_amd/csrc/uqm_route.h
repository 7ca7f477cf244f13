// Top-k + permutation in one launch (uqm_route.hip), for the multi-token
// block path (uqm_api.hip).
#pragma once

#include "uqm_internal.h"

namespace uqm {

// Workspace sync word (among the first kSyncEpochBase words, which the
// single-token fused kernel leaves unused apart from kSyncError) holding the
// completion counter of route_topk_permute_kernel: zero before every launch
// and put back to zero by the launch's last workgroup. Its offset does not
// depend on the token count, so a workspace reused across token counts keeps it.
constexpr int kSyncPermuteDone = 8;
static_assert(kSyncPermuteDone != kSyncError && kSyncPermuteDone != kSyncExpired && kSyncPermuteDone < kSyncEpochBase,
              "sync word taken");

// Top-k (over bf16 logits, or over `parts` FP32 partials when plog is set)
// and the permutation of its routes into rt, in one launch.
bool route_topk_permute_fits(int64_t T, int64_t k);
hipError_t launch_route_topk_permute(const uint16_t* logits, const float* plog, int parts, int64_t pstride,
                                     int64_t ldl, int64_t T, int64_t E, int64_t k, int norm, uint16_t* weights_out,
                                     int64_t* indices_out, float* shared_gate, uint16_t* logits_out,
                                     const RouteTables& rt, int tile_tokens, uint32_t* counter, hipStream_t stream);

}  // namespace uqm
