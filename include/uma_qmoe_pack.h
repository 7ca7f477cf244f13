/*
 * uma_qmoe_pack.h — C ABI of the pack-file reader and device staging in
 * libuma_qmoe_hip.so (host code; only the staging call touches the GPU).
 *
 * A pack file is an ExpertPack ("UQMOEPK1", every tensor Q4) or a TargetPack
 * ("UQMOTPK1", one encoding per layer): a 96-byte little-endian prefix
 * (magic, version 1, header length, payload offset, payload length, SHA-256
 * of the header, SHA-256 of the payload), a canonical-JSON header listing
 * every tensor, zero padding to the payload offset (a multiple of 4096), and
 * the payload: each tensor at a multiple of the tensor alignment, its data,
 * zero bytes to a multiple of 4, its float32 scales, zero bytes to the next
 * alignment boundary.
 *
 * uqm_pack_open maps the file once and validates all of it before returning:
 * prefix, both hashes, canonical JSON, model and policy identities, the layout
 * and zero padding of every tensor, every tensor's SHA-256 and its payload
 * semantics (no reserved Q4 code, zero Q4 odd-tail nibble, finite positive
 * scales). Failures return UQM_ERR_PACK with the reference reader's message
 * in uqm_last_error(). Tensor pointers handed out point into the mapping and
 * stay valid until uqm_pack_close.
 */
#ifndef UMA_QMOE_PACK_H
#define UMA_QMOE_PACK_H

#include <stddef.h>
#include <stdint.h>

#include "uma_qmoe_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct uqm_pack uqm_pack;

enum { UQM_PACK_ANY = -1, UQM_PACK_EXPERT = 0, UQM_PACK_TARGET = 1 };
enum { UQM_PROJ_GATE = 0, UQM_PROJ_UP = 1, UQM_PROJ_DOWN = 2 };

/* One stored tensor: host pointers into the mapping. */
typedef struct uqm_pack_tensor {
  const uint8_t* data;   /* encoded elements (Q4 nibbles, int8 codes or bf16 words) */
  uint64_t data_bytes;
  const uint8_t* scales; /* float32 group scales; NULL for BF16                   */
  uint64_t scale_bytes;
  int64_t element_count;
  int64_t shape[4];      /* the first `ndim` entries                               */
  int32_t ndim;          /* 1..4 (tensors of higher rank are refused by this call) */
  int32_t encoding;      /* UQM_Q4 / UQM_Q8 / UQM_BF16                             */
  int32_t group_size;    /* scale group in elements; 0 for BF16                    */
  int32_t reserved;
} uqm_pack_tensor;

/* Opens and validates a pack file. expected_kind is UQM_PACK_ANY or the kind
 * the caller requires; the expected_* strings are NULL or the value the
 * header must carry (expected_policy_id applies to TargetPacks only).
 * Replaces ExpertPackReader.__init__ (src/uma_qmoe/expert_pack.py:317-556)
 * and TargetPackReader.__init__ (src/uma_qmoe/target_pack.py:493-812). */
int uqm_pack_open(const char* path, int32_t expected_kind, const char* expected_model_id,
                  const char* expected_model_revision, const char* expected_model_manifest_sha256,
                  const char* expected_policy_id, uqm_pack** pack);

/* Unmaps the file and frees the pack (and its pinned staging buffers). */
int uqm_pack_close(uqm_pack* pack);

/* Kind, payload offset and length, ExpertPack group size (128 for TargetPacks). */
int uqm_pack_info(const uqm_pack* pack, int32_t* kind, uint64_t* payload_offset, uint64_t* payload_length,
                  int32_t* group_size);

/* The header's canonical JSON bytes (inside the mapping, not NUL-terminated). */
int uqm_pack_header(const uqm_pack* pack, const char** json, size_t* length);

/* Looks a tensor up by name: its views into the mapping and its metadata.
 * Replaces tensor_views (src/uma_qmoe/expert_pack.py:529, target_pack.py:771). */
int uqm_pack_lookup(const uqm_pack* pack, const char* name, uqm_pack_tensor* tensor);

/* Encoding of one layer: UQM_Q4 for every layer of an ExpertPack, the policy's
 * for a TargetPack (layer index checked against the fixed model's layers).
 * Replaces TargetPackReader.layer_encoding (src/uma_qmoe/target_pack.py:695). */
int uqm_pack_layer_encoding(const uqm_pack* pack, int64_t layer, int32_t* encoding);

/* Copies one projection of experts 0..num_experts-1 of `layer` to the device,
 * expert-major: data_dst gets expert e's data at e * data_bytes, scales_dst
 * (NULL for BF16) its scales at e * scale_bytes. Every expert must be present
 * with the layer's encoding and expert 0's shape. The bytes go from the
 * mapping through pinned host buffers (the pack's, reused across calls) to
 * the device on `stream`; returns when the copies have completed. Replaces
 * _host_projection / _device_layer (src/uma_qmoe/native_backend.py:374-455),
 * which clone every tensor view in Python first. */
int uqm_pack_stage_projection(uqm_pack* pack, int64_t layer, int32_t projection, int64_t num_experts,
                              void* data_dst, void* scales_dst, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* UMA_QMOE_PACK_H */
