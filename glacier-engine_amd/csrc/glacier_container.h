// glacier_container.h — reader of Glacier's portable `.glacier` source
// containers (src/model/format.zig FileReader), the quant-aware page payload
// codec (src/model/qio.zig over src/core/quant.zig) and the loader's tensor
// assembly (src/loader.zig loadWithOptions / concatInt4Pages) that the
// device model loader uploads from.
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <map>
#include <string>
#include <utility>
#include <vector>

#include "glacier_hip.h"

namespace gct {

constexpr uint64_t kHeaderSize = 256;          // format.zig:24
constexpr uint32_t kPageSizeLog2 = 18;         // :27
constexpr uint64_t kPageSizeBytes = 1ull << 18;
constexpr uint64_t kEntrySize = 64;            // :28
constexpr uint64_t kMaxMetadata = 16ull << 20;  // :32
constexpr uint64_t kMaxPages = 1ull << 20;      // :33
constexpr uint32_t kQioMagic = 0x514F4954;      // qio.zig:28 ("QOIT")
constexpr size_t kSubHeader = 16;               // qio.zig:29

// core.Precision (src/core/precision.zig:9-17)
enum Precision : uint32_t { kFp16 = 0, kBf16 = 1, kInt8 = 2, kInt4 = 3, kInt2 = 4, kTri = 5, kFp32 = 6 };
// core.quant.QuantPrecision (quant.zig:21)
enum QuantPrecision : uint32_t { kQInt8 = 0, kQInt4 = 1 };

// One admitted container: the read-only mapping, its header and index.
struct Container {
  int fd = -1;
  const uint8_t *bytes = nullptr;
  size_t size = 0;
  glacier_hip_glacier_header_t header{};
  std::vector<glacier_hip_glacier_page_t> pages;
  ~Container();
};

// FileReader.openFile (format.zig:409-478): admission in the reference's
// order; on failure returns the GLACIER_HIP_GLAC_* code and *out stays null.
uint32_t open_container(const char *path, Container **out);
// validatePayloadSchemaV1 (:351-376)
uint32_t validate_payload_schema(const Container &c, const glacier_hip_glacier_page_t &p);
// validateAllPageCrcsWithBufferV1 (:503-531)
uint32_t validate_all_crcs(const Container &c, uint64_t buffer_bytes);
// readPage (:488-494): the payload's bytes after the CRC check
uint32_t read_page(const Container &c, const glacier_hip_glacier_page_t &p, const uint8_t **data);
// readPageDequant (:638-662) to f32
uint32_t read_page_f32(const Container &c, const glacier_hip_glacier_page_t &p, std::vector<float> &out);
void source_fingerprint(const Container &c, uint8_t out[32]);  // loader.zig:167-189

// qio.readQuantHeader / encodePage / decodePage (qio.zig:52-167)
struct QuantHeader {
  uint32_t num_elements, group_size, precision;
};
uint32_t read_quant_header(const uint8_t *buf, size_t len, QuantHeader *h);
uint32_t qio_encode_f32(const float *src, uint64_t n, uint32_t precision, uint32_t group_size,
                        std::vector<uint8_t> &out);
uint32_t qio_decode_f32(const uint8_t *payload, size_t len, std::vector<float> &out);

// RFC 8259 JSON whose top-level value is an object (std.json.parseFromSlice
// into a Value, then the object check of openFile).
bool json_object(const uint8_t *p, size_t n);

// The loader's materialised (layer, kind) groups (loader.zig:1246-1434):
// INT4 groups of the compact tensor kinds merged by concatInt4Pages, every
// other group decoded page by page to f32 and concatenated.
struct Group {
  bool int4 = false;
  std::vector<uint8_t> packed;   // int4: row-major nibbles, low nibble = even element
  std::vector<float> scales;     // int4: f32 scales
  uint32_t group_size = 0;
  uint64_t elements = 0;
  std::vector<float> values;     // decoded groups
};
struct Geometry {
  uint32_t num_layers = 0;
  uint64_t dim = 0, hidden_dim = 0, vocab_size = 0;
};
using GroupKey = std::pair<uint32_t, uint32_t>;  // (layer, kind)
uint32_t derive_geometry(const Container &c, Geometry *g);
uint32_t materialize(const Container &c, std::map<GroupKey, Group> &groups);

const char *error_name(uint32_t e);

}  // namespace gct
