// page_image.cpp — PageImageV1 codec (continuation_paged_kv_restore.zig).
//
// encode follows encodeCanonicalPageImageV1 (:101-170) and decode follows
// decodePageImageV1 (:263-360) check for check, so a broken image fails with
// the reason the reference gives. Fields are written and read explicitly
// little-endian; the footer is pageImageRootV1 (:488-495).
#include "page_image.h"

#include <string.h>

#include "host_util.h"
#include "paged_kv.h"

namespace gpi {

namespace {

const uint8_t kMagic[8] = {'G', 'C', 'K', 'V', 'P', 'G', '0', '1'};
const char kDomain[] = "glacier-continuation-paged-kv-page-image-v1";  // + its NUL

void image_root(const uint8_t *body, size_t n, uint8_t out[32]) {
  gh::Sha256 h;
  h.update(kDomain, sizeof(kDomain));  // the domain string ends in \0
  h.update(body, n);
  h.final(out);
}

bool zero32(const uint8_t *d) {
  for (int i = 0; i < 32; ++i)
    if (d[i]) return false;
  return true;
}

struct W {
  uint8_t *p;
  size_t at = 0;
  void u32(uint32_t v) {
    for (int i = 0; i < 4; ++i) p[at++] = (uint8_t)(v >> (8 * i));
  }
  void u64(uint64_t v) {
    for (int i = 0; i < 8; ++i) p[at++] = (uint8_t)(v >> (8 * i));
  }
  void bytes(const void *b, size_t n) {
    memcpy(p + at, b, n);
    at += n;
  }
  void root(const glacier_hip_page_map_root_t &r) {
    u64(r.abi_version);
    u64(r.cache_instance);
    u64(r.generation);
    u64(r.committed_len);
    u64(r.committed_pages);
    bytes(r.ownership_sha256, 32);
  }
  void ref(const glacier_hip_page_ref_t &r) {
    u64(r.abi_version);
    u64(r.cache_instance);
    u64(r.logical_page);
    u64(r.ownership_generation);
  }
};

struct R {
  const uint8_t *p;
  size_t at = 0;
  uint32_t u32() {
    uint32_t v = 0;
    for (int i = 0; i < 4; ++i) v |= (uint32_t)p[at++] << (8 * i);
    return v;
  }
  uint64_t u64() {
    uint64_t v = 0;
    for (int i = 0; i < 8; ++i) v |= (uint64_t)p[at++] << (8 * i);
    return v;
  }
  void bytes(void *b, size_t n) {
    memcpy(b, p + at, n);
    at += n;
  }
  void root(glacier_hip_page_map_root_t &r) {
    r.abi_version = u64();
    r.cache_instance = u64();
    r.generation = u64();
    r.committed_len = u64();
    r.committed_pages = u64();
    bytes(r.ownership_sha256, 32);
  }
  void ref(glacier_hip_page_ref_t &r) {
    r.abi_version = u64();
    r.cache_instance = u64();
    r.logical_page = u64();
    r.ownership_generation = u64();
  }
};

uint64_t ceil_pages(uint64_t len) {
  return len / gpk::kPagePositions + (len % gpk::kPagePositions != 0);
}

}  // namespace

// usize arithmetic of the reference: each step checked for overflow
static bool mul_ok(uint64_t a, uint64_t b, uint64_t *out) {
  return !__builtin_mul_overflow(a, b, out);
}

static uint32_t encoded_bytes_checked(uint64_t L, uint64_t dim, uint64_t rows, uint64_t *out) {
  if (L == 0 || dim == 0 || rows == 0 || rows > gpk::kPagePositions)
    return GLACIER_HIP_PAGE_IMAGE_INVALID_PAGE_IMAGE;
  uint64_t a, b, e, bytes;
  if (!mul_ok(L, 2, &a) || !mul_ok(a, rows, &b) || !mul_ok(b, dim, &e) || !mul_ok(e, 4, &bytes) ||
      bytes > UINT64_MAX - kHeaderBytes - kFooterBytes)
    return GLACIER_HIP_PAGE_IMAGE_ARITHMETIC_OVERFLOW;
  *out = bytes + kHeaderBytes + kFooterBytes;
  return GLACIER_HIP_PAGE_IMAGE_OK;
}

uint64_t encoded_bytes(uint64_t L, uint64_t dim, uint64_t rows) {
  uint64_t n = 0;
  return encoded_bytes_checked(L, dim, rows, &n) ? 0 : n;
}

uint64_t expected_rows(const glacier_hip_page_map_root_t &root, uint64_t logical_page) {
  const uint64_t start = logical_page * gpk::kPagePositions;
  const uint64_t remaining = root.committed_len - start;
  return remaining < gpk::kPagePositions ? remaining : gpk::kPagePositions;
}

uint32_t encode(const glacier_hip_page_map_root_t &r, uint64_t L, uint64_t dim, uint64_t max_seq,
                const glacier_hip_page_ref_t &ref, uint64_t rows, const uint8_t *payload,
                uint64_t payload_len, const uint8_t challenge[32], uint8_t *out,
                uint64_t out_capacity, uint64_t *out_len) {
  uint64_t need = 0;
  const uint32_t ge = encoded_bytes_checked(L, dim, rows, &need);
  if (ge) return ge;
  if (out_capacity < need) return GLACIER_HIP_PAGE_IMAGE_CAPACITY_EXCEEDED;
  const uint64_t count = (need - kHeaderBytes - kFooterBytes) / 4;
  if (payload_len != count * 4 || r.abi_version != gpk::kPageMapRootAbi || r.cache_instance == 0 ||
      r.generation == 0 || r.committed_len == 0 || r.committed_len > max_seq ||
      r.committed_pages == 0 || ref.abi_version != gpk::kPageRefAbi ||
      ref.cache_instance != r.cache_instance || ref.logical_page >= r.committed_pages ||
      ref.ownership_generation == 0 || rows != expected_rows(r, ref.logical_page) ||
      zero32(r.ownership_sha256) || zero32(challenge))
    return GLACIER_HIP_PAGE_IMAGE_INVALID_PAGE_IMAGE;
  if (r.committed_pages != ceil_pages(r.committed_len)) return GLACIER_HIP_PAGE_IMAGE_INVALID_PAGE_IMAGE;
  // the destination may not overlap the canonical rows it is built from
  if (out < payload + payload_len && payload < out + need)
    return GLACIER_HIP_PAGE_IMAGE_UNSAFE_DESTINATION;
  W w{out};
  w.bytes(kMagic, 8);
  w.u64(kPageImageAbi);
  w.u64(need);
  w.u32(0);  // flags
  w.u32(0);
  w.root(r);
  w.u64(L);
  w.u64(dim);
  w.u64(max_seq);
  w.ref(ref);
  w.u64(rows);
  w.u64(count);
  w.bytes(challenge, 32);
  w.bytes(payload, payload_len);
  image_root(out, w.at, out + w.at);
  *out_len = need;
  return GLACIER_HIP_PAGE_IMAGE_OK;
}

uint32_t decode(const uint8_t *data, uint64_t len, const uint8_t challenge[32],
                glacier_hip_page_image_v1_t *info) {
  memset(info, 0, sizeof *info);
  if (len < kHeaderBytes + kFooterBytes) return GLACIER_HIP_PAGE_IMAGE_INVALID_LENGTH;
  R rd{data};
  if (memcmp(data, kMagic, 8) != 0) return GLACIER_HIP_PAGE_IMAGE_INVALID_MAGIC;
  rd.at = 8;
  if (rd.u64() != kPageImageAbi) return GLACIER_HIP_PAGE_IMAGE_INVALID_ABI;
  if (rd.u64() != len) return GLACIER_HIP_PAGE_IMAGE_INVALID_LENGTH;
  const uint32_t flags = rd.u32(), reserved = rd.u32();
  if (flags != 0 || reserved != 0) return GLACIER_HIP_PAGE_IMAGE_INVALID_FLAGS;
  rd.root(info->source_root);
  info->num_layers = rd.u64();
  info->dim = rd.u64();
  info->max_seq = rd.u64();
  rd.ref(info->source_ref);
  info->committed_rows = rd.u64();
  info->payload_element_count = rd.u64();
  rd.bytes(info->challenge_sha256, 32);
  info->payload_offset = kHeaderBytes;
  uint64_t need = 0;
  const uint32_t ge = encoded_bytes_checked(info->num_layers, info->dim, info->committed_rows, &need);
  if (ge) return ge;
  if (len != need) return GLACIER_HIP_PAGE_IMAGE_INVALID_LENGTH;
  uint64_t payload_bytes;
  if (!mul_ok(info->payload_element_count, 4, &payload_bytes))
    return GLACIER_HIP_PAGE_IMAGE_ARITHMETIC_OVERFLOW;
  if (payload_bytes != len - kHeaderBytes - kFooterBytes)
    return GLACIER_HIP_PAGE_IMAGE_INVALID_PAGE_IMAGE;
  memcpy(info->image_sha256, data + len - kFooterBytes, 32);
  uint8_t want[32];
  image_root(data, (size_t)(len - kFooterBytes), want);
  if (memcmp(want, info->image_sha256, 32) != 0) return GLACIER_HIP_PAGE_IMAGE_INVALID_PAGE_IMAGE;
  const glacier_hip_page_map_root_t &r = info->source_root;
  const glacier_hip_page_ref_t &f = info->source_ref;
  if (r.abi_version != gpk::kPageMapRootAbi || r.cache_instance == 0 || r.generation == 0 ||
      r.committed_len == 0 || r.committed_len > info->max_seq || r.committed_pages == 0 ||
      r.committed_pages != ceil_pages(r.committed_len) || zero32(r.ownership_sha256) ||
      f.abi_version != gpk::kPageRefAbi || f.cache_instance != r.cache_instance ||
      f.logical_page >= r.committed_pages || f.ownership_generation == 0 ||
      info->num_layers == 0 || info->dim == 0 || info->max_seq == 0 ||
      info->committed_rows != expected_rows(r, f.logical_page) || zero32(challenge) ||
      memcmp(info->challenge_sha256, challenge, 32) != 0)
    return GLACIER_HIP_PAGE_IMAGE_INVALID_PAGE_IMAGE;
  uint64_t a, b, e;
  if (!mul_ok(info->num_layers, 2, &a) || !mul_ok(a, info->committed_rows, &b) ||
      !mul_ok(b, info->dim, &e))
    return GLACIER_HIP_PAGE_IMAGE_ARITHMETIC_OVERFLOW;
  if (info->payload_element_count != e) return GLACIER_HIP_PAGE_IMAGE_INVALID_PAGE_IMAGE;
  return GLACIER_HIP_PAGE_IMAGE_OK;
}

}  // namespace gpi

extern "C" {

uint64_t glacier_hip_page_image_bytes(uint64_t num_layers, uint64_t dim, uint64_t committed_rows) {
  return gpi::encoded_bytes(num_layers, dim, committed_rows);
}

int glacier_hip_page_image_encode_canonical(const glacier_hip_page_map_root_t *source_root,
                                            uint64_t num_layers, uint64_t dim, uint64_t max_seq,
                                            const glacier_hip_page_ref_t *source_ref,
                                            uint64_t committed_rows,
                                            const uint8_t *canonical_f32_le, uint64_t canonical_len,
                                            const uint8_t challenge_sha256[32], uint8_t *out,
                                            uint64_t out_capacity, uint64_t *out_len,
                                            glacier_hip_page_image_v1_t *info) {
  if (!source_root || !source_ref || (!canonical_f32_le && canonical_len) || !challenge_sha256 ||
      !out || !out_len)
    return GLACIER_HIP_INVALID_ARGUMENT;
  const uint32_t e = gpi::encode(*source_root, num_layers, dim, max_seq, *source_ref,
                                 committed_rows, canonical_f32_le, canonical_len, challenge_sha256,
                                 out, out_capacity, out_len);
  if (info) {
    if (e) {
      memset(info, 0, sizeof *info);
      info->error = e;
    } else {
      gpi::decode(out, *out_len, challenge_sha256, info);
    }
  }
  return e ? GLACIER_HIP_INVALID_CHECKPOINT : GLACIER_HIP_OK;
}

int glacier_hip_page_image_decode(const uint8_t *image, uint64_t len,
                                  const uint8_t expected_challenge_sha256[32],
                                  glacier_hip_page_image_v1_t *out) {
  if (!image || !expected_challenge_sha256 || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  const uint32_t e = gpi::decode(image, len, expected_challenge_sha256, out);
  out->error = e;
  return e ? GLACIER_HIP_INVALID_CHECKPOINT : GLACIER_HIP_OK;
}

}  // extern "C"
