// runtime_image.cpp — GLRT prepared runtime image reader.
//
// Follows src/model/runtime_image.zig: Header.decode (:232-276), Record.decode
// (:375-433), Record.validateDescriptor / validateBoundsForVersion
// (:435-573), validateHeaderBytes (:1335-1372) and
// MappedImage.validateIndexAndRecords / verifyRecord (:990-1049), in that
// order, so an image fails with the reason the reference would give. Every
// field is read explicitly little-endian from the mapping (no struct
// overlays), as the reference's codec does.
#include "runtime_image.h"

#include <fcntl.h>
#include <math.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "host_util.h"

namespace gri {

namespace {

constexpr size_t kHeaderSize = 512, kV1RecordSize = 128, kRecordSize = 160;
constexpr uint64_t kAlign = 64;
constexpr size_t kHeaderCrcOffset = 156, kRoleOffset = 120, kPairOffset = 122, kDigestOffset = 128;

// ABI fingerprints of the portable (row-major INT4, f32 scales) execution
// layout: SHA-256 of "GLRT v1 header512 record128 row-major-f32-v1" and of
// "GLRT v2 header512 record160 roles pair-nibble descriptor-payload-sha256
// row-major-f32-v2" (runtime_image.zig:55-82); computed, not tabled.
void abi_fingerprint(int version, uint8_t out[32]) {
  const char *s = version == 1
                      ? "GLRT v1 header512 record128 row-major-f32-v1"
                      : "GLRT v2 header512 record160 roles pair-nibble "
                        "descriptor-payload-sha256 row-major-f32-v2";
  gh::Sha256 h;
  h.update(s, strlen(s));
  h.final(out);
}

uint16_t g16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
uint32_t g32(const uint8_t *p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
uint64_t g64(const uint8_t *p) { return (uint64_t)g32(p) | ((uint64_t)g32(p + 4) << 32); }
bool all_zero(const uint8_t *p, size_t n) {
  for (size_t i = 0; i < n; ++i)
    if (p[i]) return false;
  return true;
}
bool valid_kind(uint32_t k) { return k <= 15 || k == 255; }

// Canonical v2 descriptor bytes 0..128 of a record (Record.encode, :345-373)
void encode_descriptor(const glacier_hip_glrt_record_t &r, uint8_t out[128]) {
  memset(out, 0, 128);
  auto p16 = [&](size_t o, uint16_t v) { out[o] = (uint8_t)v; out[o + 1] = (uint8_t)(v >> 8); };
  auto p32 = [&](size_t o, uint32_t v) { for (int i = 0; i < 4; ++i) out[o + i] = (uint8_t)(v >> (8 * i)); };
  auto p64 = [&](size_t o, uint64_t v) { for (int i = 0; i < 8; ++i) out[o + i] = (uint8_t)(v >> (8 * i)); };
  p32(0, r.layer_idx);
  p32(4, r.kind);
  p16(8, r.encoding);
  p16(10, r.packed_layout);
  p32(12, r.group_size);
  p32(16, r.out_f);
  p32(20, r.in_f);
  p32(24, r.flags);
  p32(28, r.payload_crc32);
  p64(32, r.num_elements);
  for (int s = 0; s < kStreams; ++s) {
    p64(40 + 16 * s, r.offset[s]);
    p64(48 + 16 * s, r.length[s]);
  }
  p16(kRoleOffset, r.role);
  p16(kPairOffset, r.pair_nibble_layout);
}

uint32_t decode_record(const uint8_t *b, int version, glacier_hip_glrt_record_t &r) {
  if (version == 1 ? !all_zero(b + 120, 8) : !all_zero(b + 124, 4))
    return GLACIER_HIP_GLRT_BAD_RESERVED_FIELD;
  memset(&r, 0, sizeof r);
  r.layer_idx = g32(b);
  r.kind = g32(b + 4);
  if (!valid_kind(r.kind)) return GLACIER_HIP_GLRT_BAD_TENSOR_KIND;
  r.encoding = g16(b + 8);
  if (r.encoding > kPairNibble) return GLACIER_HIP_GLRT_BAD_ENCODING;
  r.packed_layout = g16(b + 10);
  if (r.packed_layout != kRowMajor && r.packed_layout != kRows4K16 &&
      r.packed_layout != kLayoutNone)
    return GLACIER_HIP_GLRT_BAD_PACKED_LAYOUT;
  if (version == 1) {
    r.role = kTensor;
    r.pair_nibble_layout = 0xFFFF;
  } else {
    r.role = g16(b + kRoleOffset);
    if (r.role != kTensor && r.role != kMlpGateUpPair) return GLACIER_HIP_GLRT_BAD_ROLE;
    r.pair_nibble_layout = g16(b + kPairOffset);
    if (r.pair_nibble_layout != 0 && r.pair_nibble_layout != 0xFFFF)
      return GLACIER_HIP_GLRT_BAD_PAIR_NIBBLE_LAYOUT;
    memcpy(r.payload_digest, b + kDigestOffset, 32);
  }
  r.group_size = g32(b + 12);
  r.out_f = g32(b + 16);
  r.in_f = g32(b + 20);
  r.flags = g32(b + 24);
  r.payload_crc32 = g32(b + 28);
  r.num_elements = g64(b + 32);
  for (int s = 0; s < kStreams; ++s) {
    r.offset[s] = g64(b + 40 + 16 * s);
    r.length[s] = g64(b + 48 + 16 * s);
  }
  return GLACIER_HIP_GLRT_OK;
}

// Record.validateDescriptor (:435-541)
uint32_t validate_descriptor(const glacier_hip_glrt_record_t &r, int version, bool require_digest) {
  if (r.flags != 0) return GLACIER_HIP_GLRT_BAD_FLAGS;
  if (version == 1) {
    if (r.role != kTensor || r.pair_nibble_layout != 0xFFFF || !all_zero(r.payload_digest, 32))
      return GLACIER_HIP_GLRT_BAD_VERSIONED_RECORD;
    if (r.encoding == kPairNibble) return GLACIER_HIP_GLRT_BAD_ENCODING;
  } else if (require_digest && all_zero(r.payload_digest, 32)) {
    return GLACIER_HIP_GLRT_MISSING_DIGEST;
  }
  if (r.out_f == 0 || r.in_f == 0 || r.num_elements == 0) return GLACIER_HIP_GLRT_BAD_TENSOR_SHAPE;
  if ((uint64_t)r.out_f * r.in_f != r.num_elements) return GLACIER_HIP_GLRT_BAD_TENSOR_SHAPE;
  const uint64_t *L = r.length;
  const uint64_t n = r.num_elements;
  switch (r.encoding) {
    case kRawF32:
      if (r.role != kTensor || r.packed_layout != kLayoutNone || r.pair_nibble_layout != 0xFFFF ||
          r.group_size != 0)
        return GLACIER_HIP_GLRT_BAD_ENCODING;
      if (L[kRaw] == 0 || L[kPacked] || L[kScalesF32] || L[kScalesF16] || L[kScalesF16Rows4])
        return GLACIER_HIP_GLRT_BAD_ENCODING;
      if (n > UINT64_MAX / 4 || L[kRaw] != n * 4) return GLACIER_HIP_GLRT_BAD_TENSOR_SHAPE;
      break;
    case kInt4: {
      if (r.role != kTensor || r.pair_nibble_layout != 0xFFFF || r.packed_layout == kLayoutNone ||
          r.group_size == 0 || L[kPacked] == 0 || L[kRaw] != 0)
        return GLACIER_HIP_GLRT_BAD_ENCODING;
      if (L[kPacked] != n / 2 + n % 2) return GLACIER_HIP_GLRT_BAD_TENSOR_SHAPE;
      const uint64_t groups = n / r.group_size + (n % r.group_size != 0);
      if (L[kScalesF32] && L[kScalesF32] != groups * 4) return GLACIER_HIP_GLRT_BAD_TENSOR_SHAPE;
      if (L[kScalesF16] && L[kScalesF16] != groups * 2) return GLACIER_HIP_GLRT_BAD_TENSOR_SHAPE;
      if (L[kScalesF16Rows4] && L[kScalesF16Rows4] != groups * 2)
        return GLACIER_HIP_GLRT_BAD_TENSOR_SHAPE;
      if (!L[kScalesF32] && !L[kScalesF16] && !L[kScalesF16Rows4])
        return GLACIER_HIP_GLRT_MISSING_SCALES;
      if (r.packed_layout == kRows4K16 && (r.out_f % 4 || r.in_f % 16 || !L[kScalesF16Rows4]))
        return GLACIER_HIP_GLRT_BAD_PACKED_LAYOUT;
      break;
    }
    default: {  // PairNibble
      if (version != 2 || r.role != kMlpGateUpPair) return GLACIER_HIP_GLRT_BAD_ROLE;
      if (r.packed_layout != kLayoutNone || r.pair_nibble_layout != 0)
        return GLACIER_HIP_GLRT_BAD_PAIR_NIBBLE_LAYOUT;
      if ((r.group_size != 8 && r.group_size != 16) || r.out_f % 4 || r.in_f % 16 ||
          r.in_f % r.group_size)
        return GLACIER_HIP_GLRT_BAD_TENSOR_SHAPE;
      if (L[kRaw] || L[kScalesF32] || L[kScalesF16]) return GLACIER_HIP_GLRT_BAD_ENCODING;
      if (L[kPacked] != n) return GLACIER_HIP_GLRT_BAD_TENSOR_SHAPE;
      const uint64_t groups = (uint64_t)r.out_f * (r.in_f / r.group_size);
      if (L[kScalesF16Rows4] != groups * 2 * 2) return GLACIER_HIP_GLRT_BAD_TENSOR_SHAPE;
      break;
    }
  }
  return GLACIER_HIP_GLRT_OK;
}

bool overlap(uint64_t ao, uint64_t al, uint64_t bo, uint64_t bl) {
  return ao < bo + bl && bo < ao + al;
}

// Record.validateBoundsForVersion (:543-573)
uint32_t validate_bounds(const glacier_hip_glrt_record_t &r, uint64_t data_offset,
                         uint64_t file_size, int version, bool require_digest) {
  uint32_t e = validate_descriptor(r, version, require_digest);
  if (e) return e;
  for (int s = 0; s < kStreams; ++s) {
    const uint64_t off = r.offset[s], len = r.length[s];
    if ((off == 0) != (len == 0)) return GLACIER_HIP_GLRT_BAD_BOUNDS;
    if (len == 0) continue;
    if (off < data_offset || off % kAlign) return GLACIER_HIP_GLRT_BAD_ALIGNMENT;
    if (off > UINT64_MAX - len) return GLACIER_HIP_GLRT_BAD_BOUNDS;
    if (off + len > file_size) return GLACIER_HIP_GLRT_BAD_BOUNDS;
  }
  for (int a = 0; a < kStreams; ++a) {
    if (!r.length[a]) continue;
    for (int b = a + 1; b < kStreams; ++b)
      if (r.length[b] && overlap(r.offset[a], r.length[a], r.offset[b], r.length[b]))
        return GLACIER_HIP_GLRT_OVERLAPPING_PAYLOAD;
  }
  return GLACIER_HIP_GLRT_OK;
}

bool same_identity(const glacier_hip_glrt_record_t &a, const glacier_hip_glrt_record_t &b) {
  if (a.layer_idx != b.layer_idx || a.role != b.role) return false;
  return a.role != kTensor || a.kind == b.kind;
}

}  // namespace

// CRC-32, IEEE 802.3 polynomial, reflected (zlib crc32 / std.hash.Crc32),
// table-driven by the byte.
uint32_t crc32(const void *data, size_t n, uint32_t crc) {
  static uint32_t table[256];
  static bool init = [] {
    for (uint32_t i = 0; i < 256; ++i) {
      uint32_t c = i;
      for (int k = 0; k < 8; ++k) c = (c & 1) ? 0xEDB88320u ^ (c >> 1) : c >> 1;
      table[i] = c;
    }
    return true;
  }();
  (void)init;
  const uint8_t *p = (const uint8_t *)data;
  crc = ~crc;
  for (size_t i = 0; i < n; ++i) crc = table[(crc ^ p[i]) & 0xFF] ^ (crc >> 8);
  return ~crc;
}

Image::~Image() {
  if (bytes && bytes != MAP_FAILED) munmap((void *)bytes, size);
  if (fd >= 0) close(fd);
}

const char *error_name(uint32_t e) {
  static const char *names[] = {
      "Ok", "TruncatedHeader", "BadMagic", "BadVersion", "BadHeaderSize", "BadRecordSize",
      "BadAlignment", "BadConfig", "BadReservedField", "HeaderCrcMismatch",
      "LegacyVersionDisabled", "BadHeader", "BadBounds", "SourceFingerprintMismatch",
      "AbiFingerprintMismatch", "IndexCrcMismatch", "TruncatedIndex", "BadTensorKind",
      "BadEncoding", "BadPackedLayout", "BadRole", "BadPairNibbleLayout", "BadFlags",
      "BadVersionedRecord", "MissingDigest", "BadTensorShape", "MissingScales",
      "OverlappingPayload", "DuplicateRecord", "CrcMismatch", "DigestMismatch", "FileError",
      "MissingTensor", "BadPayload", "NoLayers", "Unsupported"};
  return e < sizeof(names) / sizeof(names[0]) ? names[e] : "Unknown";
}

static uint32_t validate(Image &img, const Options &opt) {
  const uint8_t *m = img.bytes;
  const size_t size = img.size;
  glacier_hip_glrt_info_t &info = img.info;
  if (size < kHeaderSize) return GLACIER_HIP_GLRT_TRUNCATED_HEADER;
  // ---- Header.decode ----
  if (memcmp(m, "GLRT", 4) != 0) return GLACIER_HIP_GLRT_BAD_MAGIC;
  const int version = g16(m + 4);
  if (version != 1 && version != 2) return GLACIER_HIP_GLRT_BAD_VERSION;
  if (g16(m + 6) != kHeaderSize) return GLACIER_HIP_GLRT_BAD_HEADER_SIZE;
  const size_t rsz = version == 2 ? kRecordSize : kV1RecordSize;
  if (g16(m + 8) != rsz) return GLACIER_HIP_GLRT_BAD_RECORD_SIZE;
  if (g16(m + 10) != kAlign) return GLACIER_HIP_GLRT_BAD_ALIGNMENT;
  if (m[140] > 1) return GLACIER_HIP_GLRT_BAD_CONFIG;
  if (!all_zero(m + 141, 3) || !all_zero(m + 160, kHeaderSize - 160))
    return GLACIER_HIP_GLRT_BAD_RESERVED_FIELD;
  info.version = (uint32_t)version;
  const uint32_t flags = g32(m + 12);
  info.record_count = g64(m + 16);
  const uint64_t index_offset = g64(m + 24);
  info.data_offset = g64(m + 32);
  info.file_size = g64(m + 40);
  memcpy(info.source_fingerprint, m + 48, 32);
  memcpy(info.abi_fingerprint, m + 80, 32);
  info.dim = g32(m + 112);
  info.hidden_dim = g32(m + 116);
  info.layers = g32(m + 120);
  info.vocab = g32(m + 124);
  info.heads = g32(m + 128);
  info.head_dim = g32(m + 132);
  info.kv_heads = g32(m + 136);
  info.tie_embeddings = m[140];
  uint32_t bits = g32(m + 144);
  memcpy(&info.rms_eps, &bits, 4);
  bits = g32(m + 148);
  memcpy(&info.rope_theta, &bits, 4);
  const uint32_t index_crc = g32(m + 152), header_crc = g32(m + kHeaderCrcOffset);
  // ConfigSnapshot.validate (:183-196)
  if (!info.dim || !info.hidden_dim || !info.layers || !info.vocab || !info.heads ||
      !info.head_dim || !info.kv_heads || !std::isfinite(info.rms_eps) || info.rms_eps <= 0 ||
      !std::isfinite(info.rope_theta) || info.rope_theta <= 0)
    return GLACIER_HIP_GLRT_BAD_CONFIG;
  // ---- validateHeaderBytes ----
  uint8_t hb[kHeaderSize];
  memcpy(hb, m, kHeaderSize);
  memset(hb + kHeaderCrcOffset, 0, 4);
  if (crc32(hb, kHeaderSize) != header_crc) return GLACIER_HIP_GLRT_HEADER_CRC_MISMATCH;
  if (version == 1 && !opt.allow_v1) return GLACIER_HIP_GLRT_LEGACY_VERSION_DISABLED;
  if (flags != 0 || info.record_count == 0) return GLACIER_HIP_GLRT_BAD_HEADER;
  if (index_offset != kHeaderSize || info.file_size != size) return GLACIER_HIP_GLRT_BAD_BOUNDS;
  if (info.record_count > (UINT64_MAX - index_offset) / rsz) return GLACIER_HIP_GLRT_BAD_BOUNDS;
  const uint64_t index_end = index_offset + info.record_count * rsz;
  if (info.data_offset < index_end || info.data_offset % kAlign || info.data_offset > info.file_size)
    return GLACIER_HIP_GLRT_BAD_ALIGNMENT;
  if (opt.check_source && memcmp(opt.expected_source, info.source_fingerprint, 32) != 0)
    return GLACIER_HIP_GLRT_SOURCE_FINGERPRINT_MISMATCH;
  uint8_t abi[32];
  abi_fingerprint(version, abi);
  if (memcmp(abi, info.abi_fingerprint, 32) != 0) return GLACIER_HIP_GLRT_ABI_FINGERPRINT_MISMATCH;
  // ---- validateIndexAndRecords ----
  if (index_end > size) return GLACIER_HIP_GLRT_BAD_BOUNDS;
  if (crc32(m + index_offset, (size_t)(index_end - index_offset)) != index_crc)
    return GLACIER_HIP_GLRT_INDEX_CRC_MISMATCH;
  img.records.resize((size_t)info.record_count);
  for (size_t i = 0; i < img.records.size(); ++i) {
    glacier_hip_glrt_record_t &r = img.records[i];
    uint32_t e = decode_record(m + index_offset + i * rsz, version, r);
    if (e) return e;
    if ((e = validate_bounds(r, info.data_offset, info.file_size, version, true))) return e;
    for (size_t p = 0; p < i; ++p) {
      const glacier_hip_glrt_record_t &q = img.records[p];
      if (same_identity(r, q)) return GLACIER_HIP_GLRT_DUPLICATE_RECORD;
      for (int a = 0; a < kStreams; ++a) {
        if (!r.length[a]) continue;
        for (int b = 0; b < kStreams; ++b)
          if (q.length[b] && overlap(r.offset[a], r.length[a], q.offset[b], q.length[b]))
            return GLACIER_HIP_GLRT_OVERLAPPING_PAYLOAD;
      }
    }
    // verifyRecord: payload CRC32 over the streams in order, then the v2
    // SHA-256 of descriptor bytes 0..128 followed by the same streams
    if (opt.verify_payload_crc) {
      uint32_t c = 0;
      for (int s = 0; s < kStreams; ++s)
        if (r.length[s]) c = crc32(m + r.offset[s], (size_t)r.length[s], c);
      if (c != r.payload_crc32) return GLACIER_HIP_GLRT_CRC_MISMATCH;
    }
    if (opt.verify_payload_digest && version == 2) {
      uint8_t desc[128], dg[32];
      encode_descriptor(r, desc);
      gh::Sha256 h;
      h.update(desc, 128);
      for (int s = 0; s < kStreams; ++s)
        if (r.length[s]) h.update(m + r.offset[s], (size_t)r.length[s]);
      h.final(dg);
      if (memcmp(dg, r.payload_digest, 32) != 0) return GLACIER_HIP_GLRT_DIGEST_MISMATCH;
    }
  }
  return GLACIER_HIP_GLRT_OK;
}

uint32_t open_image(const char *path, const Options &opt, Image **out,
                    glacier_hip_glrt_info_t *info) {
  *out = nullptr;
  auto *img = new Image();
  uint32_t e = GLACIER_HIP_GLRT_OK;
  struct stat st;
  img->fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (img->fd < 0 || fstat(img->fd, &st) != 0) {
    e = GLACIER_HIP_GLRT_FILE_ERROR;
  } else if ((size_t)st.st_size < kHeaderSize) {
    e = GLACIER_HIP_GLRT_TRUNCATED_HEADER;
  } else {
    img->size = (size_t)st.st_size;
    void *p = mmap(nullptr, img->size, PROT_READ, MAP_PRIVATE, img->fd, 0);
    if (p == MAP_FAILED) {
      e = GLACIER_HIP_GLRT_FILE_ERROR;
    } else {
      img->bytes = (const uint8_t *)p;
      e = validate(*img, opt);
    }
  }
  img->info.error = e;
  if (info) *info = img->info;
  if (e) {
    delete img;
    return e;
  }
  *out = img;
  return GLACIER_HIP_GLRT_OK;
}

const glacier_hip_glrt_record_t *find(const Image &img, uint32_t layer, uint32_t kind,
                                      uint16_t role) {
  for (const auto &r : img.records)
    if (r.layer_idx == layer && r.role == role && (role != kTensor || r.kind == kind)) return &r;
  return nullptr;
}

const uint8_t *stream(const Image &img, const glacier_hip_glrt_record_t &r, int s, uint64_t *len) {
  *len = r.length[s];
  return r.length[s] ? img.bytes + r.offset[s] : nullptr;
}

}  // namespace gri

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
struct glacier_hip_glrt_image {
  gri::Image *img;
};

extern "C" {

int glacier_hip_glrt_open(const char *path, const glacier_hip_glrt_open_options_t *opts,
                          glacier_hip_glrt_image **out, glacier_hip_glrt_info_t *info) {
  if (!path || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  *out = nullptr;
  gri::Options o;
  if (opts) {
    o.verify_payload_crc = opts->verify_payload_crc != 0;
    o.verify_payload_digest = opts->verify_payload_digest != 0;
    o.allow_v1 = opts->allow_v1 != 0;
    o.check_source = opts->check_source_fingerprint != 0;
    memcpy(o.expected_source, opts->expected_source_fingerprint, 32);
  }
  gri::Image *img = nullptr;
  glacier_hip_glrt_info_t tmp{};
  const uint32_t e = gri::open_image(path, o, &img, &tmp);
  if (info) *info = tmp;
  if (e) return GLACIER_HIP_BAD_IMAGE;
  *out = new glacier_hip_glrt_image{img};
  return GLACIER_HIP_OK;
}

void glacier_hip_glrt_close(glacier_hip_glrt_image *image) {
  if (!image) return;
  delete image->img;
  delete image;
}

int glacier_hip_glrt_record_at(const glacier_hip_glrt_image *image, uint64_t index,
                               glacier_hip_glrt_record_t *out) {
  if (!image || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  if (index >= image->img->records.size()) return GLACIER_HIP_NOT_FOUND;
  *out = image->img->records[(size_t)index];
  return GLACIER_HIP_OK;
}

int glacier_hip_glrt_find(const glacier_hip_glrt_image *image, uint32_t layer_idx, uint32_t kind,
                          uint32_t role, glacier_hip_glrt_record_t *out) {
  if (!image || !out || role > 0xFFFF) return GLACIER_HIP_INVALID_ARGUMENT;
  const glacier_hip_glrt_record_t *r = gri::find(*image->img, layer_idx, kind, (uint16_t)role);
  if (!r) return GLACIER_HIP_NOT_FOUND;
  *out = *r;
  return GLACIER_HIP_OK;
}

int glacier_hip_glrt_stream(const glacier_hip_glrt_image *image,
                            const glacier_hip_glrt_record_t *record, uint32_t stream,
                            const void **data, uint64_t *len) {
  if (!image || !record || !data || !len || stream >= gri::kStreams)
    return GLACIER_HIP_INVALID_ARGUMENT;
  // only records of this image (bounds were validated at open)
  bool mine = false;
  for (const auto &r : image->img->records)
    if (memcmp(&r, record, sizeof r) == 0) mine = true;
  if (!mine) return GLACIER_HIP_INVALID_HANDLE;
  *data = gri::stream(*image->img, *record, (int)stream, len);
  return GLACIER_HIP_OK;
}

int glacier_hip_glrt_identity(const glacier_hip_glrt_image *image, uint8_t container_sha256[32],
                              uint64_t *container_bytes) {
  if (!image || !container_sha256) return GLACIER_HIP_INVALID_ARGUMENT;
  gh::Sha256 h;
  h.update(image->img->bytes, image->img->size);
  h.final(container_sha256);
  if (container_bytes) *container_bytes = image->img->size;
  return GLACIER_HIP_OK;
}

}  // extern "C"

namespace gri {
const Image *image_of(const glacier_hip_glrt_image *h) { return h ? h->img : nullptr; }
}  // namespace gri
