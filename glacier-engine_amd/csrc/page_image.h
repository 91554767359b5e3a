// page_image.h — portable paged-KV checkpoint page images
// (src/continuation_paged_kv_restore.zig PageImageV1): the byte codec and the
// source-chain check of a restore. Host only; the session reads the device
// pages back for encode and writes them for restore.
#pragma once
#include <stddef.h>
#include <stdint.h>

#include "glacier_hip.h"

namespace gpi {

constexpr uint64_t kPageImageAbi = 0x47434b5000000001ull;       // :19
constexpr uint64_t kCheckpointRestoreAbi = 0x4750435200000001ull;  // paged_kv_cache.zig:24
constexpr size_t kHeaderBytes = 208, kFooterBytes = 32;

// encodedPageImageBytesV1; 0 when the geometry is invalid
uint64_t encoded_bytes(uint64_t num_layers, uint64_t dim, uint64_t committed_rows);
uint64_t expected_rows(const glacier_hip_page_map_root_t &root, uint64_t logical_page);

// encodeCanonicalPageImageV1: returns a glacier_hip_page_image_error
uint32_t encode(const glacier_hip_page_map_root_t &root, uint64_t num_layers, uint64_t dim,
                uint64_t max_seq, const glacier_hip_page_ref_t &ref, uint64_t committed_rows,
                const uint8_t *payload, uint64_t payload_len, const uint8_t challenge[32],
                uint8_t *out, uint64_t out_capacity, uint64_t *out_len);
// decodePageImageV1: returns a glacier_hip_page_image_error and fills *info
uint32_t decode(const uint8_t *data, uint64_t len, const uint8_t challenge[32],
                glacier_hip_page_image_v1_t *info);

}  // namespace gpi
