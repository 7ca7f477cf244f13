// uqm_moe_layer_noalloc: uqm_moe_layer without a caller workspace and without
// any allocation, for callers that cannot allocate device memory (code under
// HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// The workspace of uqm_moe_layer (synchronisation words, the fused kernel's
// tagged hand-off words, route tables, partial sums) lives here in a
// file-scope device array of kScratchBytes. Each GPU holds its own copy of
// the array, at its own address, for the life of the process; host code
// never passes the array's name to a kernel (in host code the name is only a
// stand-in), only the device address hipGetSymbolAddress returns for the
// current device, looked up once per device on that device's first call.
// That first call also zero-fills the array on the caller's stream (the sync
// words must start at zero); it must therefore not be under graph capture.
// Later calls reuse the array as they find it: every kernel leaves its sync
// words ready for the next call, whatever its token count. Calls that
// overlap in time on one GPU share the array and race; calls in order on one
// stream are safe. The shared expert runs in order on the caller's stream
// (no side stream is created).
#include <mutex>

#include "../../include/uma_qmoe_hip.h"
#include "uqm_internal.h"

constexpr size_t kScratchBytes = UQM_NOALLOC_SCRATCH_BYTES;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
void* g_scratch[kMaxDevices];  // device address of `scratch` per device, set once
std::mutex g_scratch_mu;

// Device address of this device's scratch array; the first call on a device
// looks it up and zero-fills it on `s`.
int device_scratch(hipStream_t s, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return uqm::api_fail(UQM_ERR_HIP, "no current device (or device id >= %d)", kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(s, &capture);
    if (e != hipSuccess) return uqm::api_fail(UQM_ERR_HIP, "hipStreamIsCapturing: %s", hipGetErrorString(e));
    if (capture != hipStreamCaptureStatusNone)
      return uqm::api_fail(UQM_ERR_ARGUMENT,
                           "the first uqm_moe_layer_noalloc call on a device zero-fills its scratch array and must "
                           "run outside graph capture");
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return uqm::api_fail(UQM_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    e = uqm::launch_zero_fill(p, kScratchBytes, s);
    if (e != hipSuccess) return uqm::api_fail(UQM_ERR_HIP, "scratch fill launch: %s", hipGetErrorString(e));
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return UQM_OK;
}

}  // namespace

extern "C" int uqm_moe_layer_noalloc(const uqm_layer_weights* layer, const void* hidden, int64_t tokens,
                                     void* output, void* logits, void* routing_weights, int64_t* expert_indices,
                                     void* stream) {
  if (layer == nullptr) return uqm::api_fail(UQM_ERR_ARGUMENT, "layer descriptor is NULL");
  const uqm_expert_weights* w = &layer->experts;
  const size_t need = uqm_moe_workspace_bytes(tokens, w->hidden_size, w->intermediate_size,
                                              layer->has_shared ? layer->shared_intermediate_size : 0,
                                              w->num_experts, layer->top_k);
  if (need == 0 && tokens > 0) return uqm::api_fail(UQM_ERR_ARGUMENT, "invalid layer shape or token count");
  if (need > kScratchBytes)
    return uqm::api_fail(UQM_ERR_WORKSPACE,
                         "%lld tokens need %zu bytes of scratch, more than the %zu bytes uqm_moe_layer_noalloc "
                         "holds per device; call uqm_moe_layer with a workspace",
                         static_cast<long long>(tokens), need, kScratchBytes);
  void* ws = nullptr;
  if (tokens > 0) {
    const int rc = device_scratch(static_cast<hipStream_t>(stream), &ws);
    if (rc != UQM_OK) return rc;
  }
  return uqm::moe_layer_on_workspace(layer, hidden, tokens, output, logits, routing_weights, expert_indices, ws,
                                     kScratchBytes, /*side_stream=*/false, stream);
}

extern "C" int uqm_noalloc_status(void* stream) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return uqm::api_fail(UQM_ERR_HIP, "no current device (or device id >= %d)", kMaxDevices);
  void* ws = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ws = g_scratch[dev];
  }
  if (ws == nullptr) return UQM_OK;  // nothing has run on this device's scratch
  return uqm_workspace_status(ws, kScratchBytes, stream);
}
