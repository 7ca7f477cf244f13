/*
 * uma_qmoe_hip.h — C ABI of the MI355X (gfx950) UMA-QMoE MoE-operator library
 * (libuma_qmoe_hip.so).
 *
 * Conventions
 *   - Every pointer argument is a device pointer unless noted; sizes are in
 *     elements. BF16 tensors are passed as `const void*` holding little-endian
 *     bf16 words. Matrices are row-major [out, in] with `in` contiguous.
 *   - Expert weights are expert-major, projection by projection, exactly as the
 *     reference stages them on the device (src/uma_qmoe/native_backend.py:374-455):
 *       gate, up: [E, I, H]   down: [E, H, I]
 *     Q4: packed two's-complement nibbles, low nibble = even element, H*I/2
 *         bytes per expert, FP32 scale per `group_size` elements of the
 *         flattened tensor (src/uma_qmoe/q4.py:96-179).
 *     Q8: int8 codes + FP32 scales (src/uma_qmoe/target_pack.py:92-112).
 *     BF16: raw bf16 (src/uma_qmoe/target_pack.py:78-89).
 *     Nothing is ever dequantized to memory.
 *   - Kernels run on `stream` (pass torch's current stream); multi-token
 *     blocks with a shared expert fork it onto a library-owned side stream
 *     and join it back with events (UQM_OPT_OVERLAP_SHARED). No entry point
 *     allocates device memory or synchronises (except uqm_workspace_status;
 *     the side stream and its two events are created once per device);
 *     temporaries live in the caller's `workspace`, sized by
 *     uqm_moe_workspace_bytes(). The workspace must be zero-filled before its
 *     first use: its first 4352 bytes hold synchronisation words (the
 *     single-token fused kernel's error word and one launch epoch per
 *     workgroup, advanced by every launch, and a completion counter that
 *     multi-token calls leave at zero). Calls in order on one stream may
 *     reuse a workspace, also with different token counts and shapes (a
 *     fused launch whose shape differs from the last call's on the same
 *     workspace first zeroes its hand-off words with a small kernel); calls
 *     that overlap in time must not share one. The library tracks that last
 *     shape on the host: a captured graph replays its launches as captured,
 *     so calls of another shape on the same workspace between replays of a
 *     graph that holds fused launches need a workspace of their own.
 *   - Return 0 on success, nonzero UQM_ERR_* otherwise; the message is in
 *     uqm_last_error() (thread-local). Invalid arguments are rejected before
 *     any launch.
 */
#ifndef UMA_QMOE_HIP_H
#define UMA_QMOE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define UQM_ABI_VERSION 1

enum {
  UQM_OK = 0,
  UQM_ERR_ARGUMENT = 1,  /* shape / pointer / alignment / range error      */
  UQM_ERR_HIP = 2,       /* a HIP runtime call or kernel launch failed       */
  UQM_ERR_DEVICE = 3,    /* current device is not gfx950                     */
  UQM_ERR_WORKSPACE = 4, /* workspace missing or smaller than required       */
  UQM_ERR_PACK = 5       /* pack file unreadable or violating its contract   */
};

enum { UQM_Q4 = 0, UQM_Q8 = 1, UQM_BF16 = 2 };

/* Options for uqm_set_option (process-wide). */
enum {
  UQM_OPT_FUSED_DECODE = 1,   /* 1 (default): blocks of one or two tokens use the fused persistent
                                  kernel, one launch per token */
  UQM_OPT_MFMA_MIN_TOKENS = 3,     /* token count from which multi-token calls run the expert projections
                                      as MFMA grouped GEMMs (default 2; 0 = never, batched GEMV instead) */
  UQM_OPT_OVERLAP_SHARED = 4,      /* 1 (default): multi-token blocks run the shared expert on a
                                      library-owned side stream (one per device, default priority),
                                      forked from and joined back into the caller's stream with
                                      events; 0: everything in order on the caller's stream */
  UQM_OPT_STREAM_MAX_ROUTES = 5,   /* multi-token calls with at most this many routes (tokens x top_k;
                                      default 32, 0 = never) run the routed projections as
                                      expert-grouped streaming GEMVs instead of MFMA grouped GEMMs */
  UQM_OPT_FUSED_WAIT_US = 6        /* wall-clock budget of the fused kernel's inter-workgroup waits in
                                      microseconds (default 2000). 0 makes every wait give up at its
                                      first check, ready or not: each fused launch then takes its
                                      expired path (poisoned outputs, error word raised) and ends
                                      normally; for tests of that path */
};

/* Routed-expert weights of one MoE layer (device pointers). */
typedef struct uqm_expert_weights {
  int32_t encoding;          /* UQM_Q4 / UQM_Q8 / UQM_BF16                         */
  int32_t group_size;        /* scale group in elements (Q4/Q8); ignored for BF16  */
  int64_t num_experts;       /* E  (<= 256)                                        */
  int64_t hidden_size;       /* H                                                  */
  int64_t intermediate_size; /* I                                                  */
  const void* gate;          /* [E, I, H] encoded                                  */
  const float* gate_scales;  /* [E*I*H/group] or NULL for BF16                     */
  const void* up;
  const float* up_scales;
  const void* down;          /* [E, H, I] encoded                                  */
  const float* down_scales;
} uqm_expert_weights;

/* One full MoE block: router + routed experts (+ Qwen shared expert). */
typedef struct uqm_layer_weights {
  uqm_expert_weights experts;
  const void* router;        /* bf16 [E, H] router weight (mlp.gate.weight)          */
  int64_t top_k;             /* k (<= 64, <= E)                                     */
  int32_t norm_topk_prob;    /* renormalise the top-k probabilities (Qwen/OLMoE: 0) */
  int32_t has_shared;        /* 1 = Qwen shared expert present                      */
  int64_t shared_intermediate_size; /* Is                                            */
  const void* shared_gate;   /* bf16 [Is, H]                                        */
  const void* shared_up;     /* bf16 [Is, H]                                        */
  const void* shared_down;   /* bf16 [H, Is]                                        */
  const void* shared_expert_gate; /* bf16 [1, H] (mlp.shared_expert_gate.weight)     */
} uqm_layer_weights;

/* ABI version of the loaded library (UQM_ABI_VERSION). */
int uqm_abi_version(void);

/* Thread-local message of the last failing call on this thread. */
const char* uqm_last_error(void);

/* Writes the gcnArchName of `device` into buf (host memory). Replaces the
 * platform probe observed_native_platform, src/uma_qmoe/native_backend.py:52-68. */
int uqm_device_arch(int device, char* buf, int buf_len);

/* Bytes of workspace uqm_moe_forward / uqm_moe_layer need for `tokens` tokens. */
size_t uqm_moe_workspace_bytes(int64_t tokens, int64_t hidden_size, int64_t intermediate_size,
                               int64_t shared_intermediate_size, int64_t num_experts, int64_t top_k);

/* output[rows, out] = bf16(input[rows, in] @ dequant(W)^T), FP32 accumulation.
 * Replaces q4_linear: src/uma_qmoe/native/packed_q4_binding.cpp:130-163
 * (kernel packed_q4_kernel.cu:72-113, launcher :1430-1456). */
int uqm_q4_linear(const void* input, int64_t rows, const void* packed, const float* scales,
                  int64_t out_features, int64_t in_features, int64_t group_size, void* output,
                  void* stream);

/* Replaces q8_linear: src/uma_qmoe/native/packed_q4_binding.cpp:165-195
 * (kernel packed_q4_kernel.cu:115-152, launcher :1458-1484). */
int uqm_q8_linear(const void* input, int64_t rows, const void* quantized, const float* scales,
                  int64_t out_features, int64_t in_features, int64_t group_size, void* output,
                  void* stream);

/* BF16 linear for the mixed backend's bf16_linear (src/uma_qmoe/native_backend.py:636-668,
 * there torch F.linear). */
int uqm_bf16_linear(const void* input, int64_t rows, const void* weight, int64_t out_features,
                    int64_t in_features, void* output, void* stream);

/* Stable token->expert permutation of expert_indices [tokens, top_k] (int64):
 * route_order [tokens*top_k] (int64) lists route ids t*k+slot grouped by ascending
 * expert, ties in route order; expert_offsets [E+1] (int64). Routes with an id
 * outside [0, E) are dropped. Replaces argsort(stable)/bincount/cumsum at
 * src/uma_qmoe/native_backend.py:530-543 and :1007-1020. */
int uqm_route_permute(const int64_t* expert_indices, int64_t tokens, int64_t top_k, int64_t num_experts,
                      int64_t* route_order, int64_t* expert_offsets, void* workspace, size_t workspace_bytes,
                      void* stream);

/* Router: logits = bf16(hidden @ router^T) [tokens, E]; FP32 softmax; top-k with
 * ties to the lower expert id; routing_weights bf16 [tokens, k]; expert_indices
 * int64 [tokens, k]. logits may be NULL. Replaces Transformers'
 * Qwen2MoeTopKRouter.forward (modeling_qwen2_moe.py:330-336), called by the
 * reference host at src/uma_qmoe/qwen_compressed_loader.py:73. */
int uqm_router_topk(const void* hidden, int64_t tokens, int64_t hidden_size, const void* router,
                    int64_t num_experts, int64_t top_k, int32_t norm_topk_prob, void* logits,
                    void* routing_weights, int64_t* expert_indices, void* workspace, size_t workspace_bytes,
                    void* stream);

/* Routed experts only: output[t] = bf16(sum_slot w[t,slot] * FFN_e(hidden[t])),
 * FFN_e(x) = down_e(silu(gate_e x) * up_e x). hidden bf16 [tokens, H];
 * expert_indices int64 [tokens, k]; routing_weights bf16 [tokens, k].
 * Replaces q4_moe_forward / q4_moe_prefill / q8_moe_forward / q8_moe_prefill
 * (src/uma_qmoe/native/packed_q4_binding.cpp:197-488, 490-515) and the Python
 * per-expert Qwen loops (src/uma_qmoe/native_backend.py:319-372, 722-753) and
 * the BF16 grouped_mm path (:958-1005). Any E, k, H, I; any token count. One
 * or two tokens of a shape the fused kernel covers (see uqm_moe_layer) run as
 * one persistent launch per token with these routes; expert ids outside
 * [0, E) contribute nothing on every path. */
int uqm_moe_forward(const uqm_expert_weights* weights, const void* hidden, int64_t tokens,
                    const int64_t* expert_indices, const void* routing_weights, int64_t top_k, void* output,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Whole MoE block: router + routed experts (+ sigmoid-gated shared expert):
 *   out = routed(hidden) + sigmoid(hidden . w_g) * shared(hidden)
 * Replaces the host block QuantizedQwenMoEBlock.forward
 * (src/uma_qmoe/qwen_compressed_loader.py:67-86) and QuantizedMoEBlock.forward
 * (src/uma_qmoe/compressed_loader.py:58-67). logits [tokens, E] bf16,
 * routing_weights [tokens, k] bf16 and expert_indices [tokens, k] int64 are
 * optional outputs (NULL to skip). With tokens <= 2 and a supported shape
 * (H = 2048, I/Is giving 1-3 / 11 chunks per lane, top_k <= 8, Q4/Q8/BF16)
 * the whole block is one persistent launch per token (see uqm_set_option). */
int uqm_moe_layer(const uqm_layer_weights* layer, const void* hidden, int64_t tokens, void* output, void* logits,
                  void* routing_weights, int64_t* expert_indices, void* workspace, size_t workspace_bytes,
                  void* stream);

/* Pre-normalised block, as a decoder layer calls it:
 *   out = MoE(RMSNorm(hidden)),  RMSNorm(x) = bf16(w * bf16(x * rsqrt(mean(x^2) + eps)))
 * (Transformers Qwen2MoeRMSNorm, modeling_qwen2_moe.py:65-70, the
 * post_attention_layernorm that Qwen2MoeDecoderLayer applies before the block
 * the reference replaces, src/uma_qmoe/qwen_compressed_loader.py:67-86).
 * norm_weight bf16 [H] or NULL for ones; eps >= 0; output must not overlap
 * hidden. Otherwise as uqm_moe_layer;
 * on the single-token fused path the norm is folded into the kernel's
 * activation staging (no extra launch), elsewhere it is one launch into the
 * workspace. */
int uqm_norm_moe_layer(const uqm_layer_weights* layer, const void* hidden, int64_t tokens, const void* norm_weight,
                       float eps, void* output, void* logits, void* routing_weights, int64_t* expert_indices,
                       void* workspace, size_t workspace_bytes, void* stream);

/* Sets a process-wide option (UQM_OPT_*). No counterpart in the reference:
 * it selects between this library's own single-token code paths. */
int uqm_set_option(int option, int64_t value);

/* Synchronously reads (and clears) the sticky error word that the fused
 * single-token kernel raises when one of its inter-workgroup waits runs past
 * its wall-clock budget (UQM_OPT_FUSED_WAIT_US, 2 ms from the start of each
 * wave by default; a launch takes ~20 us), together with the word that marks
 * the launch in which that happened. That can only happen when its grid is
 * not fully resident, e.g. while another kernel holds CUs. Such a launch
 * still ends within the budget, and its output is poisoned rather than
 * silently wrong: NaN output rows, and routes -1 / weights NaN when the
 * routing itself expired. Returns UQM_OK when clean. No counterpart in the
 * reference. */
int uqm_workspace_status(void* workspace, size_t workspace_bytes, void* stream);

/* Scratch bytes uqm_moe_layer_noalloc holds per device (16 MiB: c2 shapes up
 * to ~80 tokens; uqm_moe_workspace_bytes gives what a call needs). */
#define UQM_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)

/* uqm_moe_layer without a workspace argument and without any allocation: the
 * temporaries live in a library-owned device array of
 * UQM_NOALLOC_SCRATCH_BYTES per device, held until the process ends. No
 * counterpart in the reference; it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Calls needing more than the array hold
 * fail with UQM_ERR_WORKSPACE. The first call on a device zero-fills the
 * array on `stream` and must not be under graph capture. Every call on one
 * GPU shares that GPU's array (it keeps the last call's contents), so calls
 * that overlap in time on one GPU race; calls in order on one stream are
 * safe. The shared expert runs on `stream` (no side stream). Otherwise as
 * uqm_moe_layer, with the same kernels and results. */
int uqm_moe_layer_noalloc(const uqm_layer_weights* layer, const void* hidden, int64_t tokens, void* output,
                          void* logits, void* routing_weights, int64_t* expert_indices, void* stream);

/* uqm_workspace_status for the scratch array of uqm_moe_layer_noalloc on the
 * current device: reads and clears its error word (and expired-launch word)
 * on `stream`, synchronously. UQM_OK when clean or when no no-allocation
 * call has run on this device yet. No counterpart in the reference; it lets
 * callers of uqm_moe_layer_noalloc, who have no workspace pointer, learn that
 * a fused launch's output was poisoned. */
int uqm_noalloc_status(void* stream);

/* RMSNorm (Transformers Qwen2MoeRMSNorm, modeling_qwen2_moe.py:65-70): bf16 in/out,
 * FP32 variance; weight bf16 [H] or NULL for ones. Used by the 24-layer stack driver. */
int uqm_rmsnorm(const void* input, int64_t rows, int64_t hidden_size, const void* weight, float eps,
                void* output, void* stream);

/* output[i] = bf16(q_i * scales[i / group_size]) (FP32 product, rounded to
 * nearest even) for the `elements` values of an encoded Q4 or Q8 tensor
 * (flattened; a multiple of 8; group_size a multiple of 8): the transient
 * dequantisation of the reference's correctness path, dequantize_q4 /
 * decode_target_tensor then .to(bfloat16) (src/uma_qmoe/q4.py:168-179,
 * src/uma_qmoe/target_pack.py:144-176, src/uma_qmoe/custom_op.py:416-431).
 * The library's performance_mode=False path runs the routed experts on
 * BF16 copies made with it; nothing keeps them after the call. */
int uqm_dequantize(int32_t encoding, const void* data, const float* scales, int64_t elements,
                   int64_t group_size, void* output, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* UMA_QMOE_HIP_H */
