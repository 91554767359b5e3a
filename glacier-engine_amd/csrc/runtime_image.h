// runtime_image.h — reader of Glacier's prepared runtime images (.glrt):
// the read-only mapping, the fail-closed header / index / record validation
// and the typed stream views the model loader uploads from
// (src/model/runtime_image.zig MappedImage).
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "glacier_hip.h"

namespace gri {

enum Stream { kPacked = 0, kScalesF32 = 1, kScalesF16 = 2, kScalesF16Rows4 = 3, kRaw = 4, kStreams = 5 };

// TensorKind values (src/model/format.zig:46-64)
enum Kind : uint32_t {
  kEmbedding = 0, kAttnQ = 1, kAttnK = 2, kAttnV = 3, kAttnO = 4, kMlpUp = 5, kMlpDown = 6,
  kMlpGate = 7, kInputNorm = 8, kLmHead = 9, kFinalNorm = 10, kPostAttnNorm = 11,
  kAttnQBias = 12, kAttnKBias = 13, kAttnVBias = 14, kAttnOBias = 15, kOther = 255,
};
enum Encoding : uint16_t { kRawF32 = 0, kInt4 = 1, kPairNibble = 2 };
enum Layout : uint16_t { kRowMajor = 0, kRows4K16 = 1, kLayoutNone = 0xFFFF };
enum Role : uint16_t { kTensor = 0, kMlpGateUpPair = 1 };
constexpr uint32_t kGlobalLayer = 0xFFFFFFFFu;

struct Options {
  bool verify_payload_crc = true;
  bool verify_payload_digest = true;
  bool allow_v1 = true;
  bool check_source = false;
  uint8_t expected_source[32] = {};
};

// One opened, validated image. `bytes` is the read-only mapping.
struct Image {
  int fd = -1;
  const uint8_t *bytes = nullptr;
  size_t size = 0;
  glacier_hip_glrt_info_t info{};
  std::vector<glacier_hip_glrt_record_t> records;
  ~Image();
};

uint32_t crc32(const void *data, size_t n, uint32_t crc = 0);
// Opens and validates; on failure returns the GLACIER_HIP_GLRT_E_* code and
// leaves *out null.
uint32_t open_image(const char *path, const Options &opt, Image **out, glacier_hip_glrt_info_t *info);
const glacier_hip_glrt_record_t *find(const Image &img, uint32_t layer, uint32_t kind, uint16_t role);
const uint8_t *stream(const Image &img, const glacier_hip_glrt_record_t &r, int s, uint64_t *len);
const char *error_name(uint32_t e);

}  // namespace gri
