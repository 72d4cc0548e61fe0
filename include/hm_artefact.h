/*
 * hm_artefact.h -- C ABI of the packed-artefact loader (libhm_host.so).
 *
 * The C++ API is include/hm_artefact.hpp (hm::PackedModel,
 * hm::storage::ExpertIndex, hm::models::PackedManifest); these functions
 * expose it to C and to the Python binding.  Every pointer is a HOST
 * pointer.  Functions return an hm_status; HM_ERR_STORAGE is the
 * reference's storage::StorageError (malformed index, missing payload,
 * checksum mismatch), HM_ERR_INVALID its std::invalid_argument (manifest
 * validation).  hm_artefact_last_error() gives the message of the last
 * failure on this thread.
 */
#ifndef HM_ARTEFACT_H
#define HM_ARTEFACT_H

#include <stddef.h>
#include <stdint.h>

#include "hm_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

#define HM_ERR_STORAGE 5

/* src/storage/ExpertIndex.hpp:15-24 (32 bytes serialised). */
typedef struct hm_index_record {
    uint32_t layer_id;
    uint32_t expert_id;
    uint64_t offset;
    uint64_t size;
    uint32_t quantization_type;
    uint32_t checksum;
} hm_index_record;

/* src/storage/ExpertIndex.hpp:28-41 (80 bytes serialised). */
typedef struct hm_projection_record {
    uint32_t layer_id;
    uint32_t expert_id;
    uint32_t projection_type; /* 0 gate, 1 up, 2 down */
    uint32_t dtype;           /* FP32 0, FP16 1, BF16 2, INT8 3 */
    uint32_t rank;
    uint32_t reserved;
    uint64_t offset;
    uint64_t size;
    uint64_t shape[4];
    uint32_t checksum;
    uint32_t trailing_reserved;
} hm_projection_record;

typedef struct hm_packed_model hm_packed_model;

typedef struct hm_packed_model_info {
    uint32_t layers;
    uint32_t experts;
    uint64_t hidden;
    uint64_t intermediate;
    uint32_t dtype;       /* of the expert tables handed out (FP16/BF16 are widened to FP32) */
    uint32_t top_k;
    uint32_t route_flags; /* HM_ROUTE_SOFTMAX | HM_ROUTE_RENORM */
} hm_packed_model_info;

const char* hm_artefact_last_error(void);

/* CRC-32 of experts.index (reflected 0xEDB88320, ExpertStore.cpp:183-192). */
uint32_t hm_crc32(const void* data, size_t bytes);

/* ExpertIndex::load / save (ExpertIndex.cpp:59-206) with the reference's
 * validation.  hm_index_read stores up to the capacities and reports the
 * full counts. */
int hm_index_read(const char* path, hm_index_record* records, size_t record_capacity,
                  hm_projection_record* projections, size_t projection_capacity,
                  size_t* record_count, size_t* projection_count);
int hm_index_write(const char* path, const hm_index_record* records, size_t record_count,
                   const hm_projection_record* projections, size_t projection_count);

/* A packed model directory (experts.bin, experts.index, manifest.json). */
int hm_packed_open(const char* directory, int verify_checksums, hm_packed_model** out);
void hm_packed_close(hm_packed_model* model);
int hm_packed_info(const hm_packed_model* model, hm_packed_model_info* info);
/* One layer's experts, ascending id, each gate [H x I] | up [H x I] |
 * down [I x H] row-major (hm_pack_layer's input): payload_bytes must be
 * E*3*H*I*sizeof(dtype); INT8 also fills scale / zero_point [E][3]. */
int hm_packed_read_layer(const hm_packed_model* model, uint32_t layer, void* payload,
                         size_t payload_bytes, float* scale, int32_t* zero_point);
/* The layer's router matrix [H x E] FP32; count must be H*E. */
int hm_packed_read_router(const hm_packed_model* model, uint32_t layer, float* w, size_t count);

#ifdef __cplusplus
}
#endif

#endif /* HM_ARTEFACT_H */
