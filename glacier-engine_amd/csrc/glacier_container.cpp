// glacier_container.cpp — the portable `.glacier` container reader, the qio
// page codec and the loader's tensor assembly (see glacier_container.h).
#include "glacier_container.h"

#include <fcntl.h>
#include <math.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <set>

#include "host_util.h"
#include "runtime_image.h"

namespace gct {

namespace {

uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | p[1] << 8); }
uint32_t rd32(const uint8_t *p) { return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24; }
uint64_t rd64(const uint8_t *p) { return (uint64_t)rd32(p) | (uint64_t)rd32(p + 4) << 32; }
void wr32(uint8_t *p, uint32_t v) {
  for (int i = 0; i < 4; ++i) p[i] = (uint8_t)(v >> (8 * i));
}
bool add_ovf(uint64_t a, uint64_t b, uint64_t *out) { return __builtin_add_overflow(a, b, out); }
bool mul_ovf(uint64_t a, uint64_t b, uint64_t *out) { return __builtin_mul_overflow(a, b, out); }
uint64_t ceil_div(uint64_t n, uint64_t d) { return n / d + (n % d != 0); }
// @min / @max of finite floats (IEEE 754-2019 minimumNumber / maximumNumber:
// -0 orders below +0)
float min_number(float a, float b) {
  if (a < b) return a;
  if (b < a) return b;
  return signbit(a) ? a : b;
}
float max_number(float a, float b) {
  if (a > b) return a;
  if (b > a) return b;
  return signbit(a) ? b : a;
}
bool all_zero(const uint8_t *p, size_t n) {
  for (size_t i = 0; i < n; ++i)
    if (p[i]) return false;
  return true;
}

// ---- JSON (RFC 8259) -------------------------------------------------------
// Iterative, so no nesting depth exhausts the stack; strings must be UTF-8
// without control characters, escapes well formed (a high surrogate escape
// followed by a low one), and keys of one object distinct.
struct JsonScan {
  const uint8_t *p, *e;
  void ws() {
    while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  static int hex(uint8_t c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    return -1;
  }
  bool u4(uint32_t *v) {
    if (e - p < 4) return false;
    uint32_t x = 0;
    for (int i = 0; i < 4; ++i) {
      const int h = hex(p[i]);
      if (h < 0) return false;
      x = x << 4 | (uint32_t)h;
    }
    p += 4;
    *v = x;
    return true;
  }
  static void put_utf8(std::string *s, uint32_t cp) {
    if (!s) return;
    if (cp < 0x80) {
      s->push_back((char)cp);
    } else if (cp < 0x800) {
      s->push_back((char)(0xC0 | cp >> 6));
      s->push_back((char)(0x80 | (cp & 0x3F)));
    } else if (cp < 0x10000) {
      s->push_back((char)(0xE0 | cp >> 12));
      s->push_back((char)(0x80 | (cp >> 6 & 0x3F)));
      s->push_back((char)(0x80 | (cp & 0x3F)));
    } else {
      s->push_back((char)(0xF0 | cp >> 18));
      s->push_back((char)(0x80 | (cp >> 12 & 0x3F)));
      s->push_back((char)(0x80 | (cp >> 6 & 0x3F)));
      s->push_back((char)(0x80 | (cp & 0x3F)));
    }
  }
  // One UTF-8 scalar (RFC 3629: shortest form, no surrogates, <= U+10FFFF).
  bool utf8(std::string *s) {
    const uint8_t c = *p;
    int n;
    uint32_t cp, lo;
    if (c < 0x80) {
      if (s) s->push_back((char)c);
      ++p;
      return true;
    } else if (c >= 0xC2 && c <= 0xDF) {
      n = 1, cp = c & 0x1F, lo = 0x80;
    } else if (c >= 0xE0 && c <= 0xEF) {
      n = 2, cp = c & 0x0F, lo = 0x800;
    } else if (c >= 0xF0 && c <= 0xF4) {
      n = 3, cp = c & 0x07, lo = 0x10000;
    } else {
      return false;
    }
    if (e - p < n + 1) return false;
    for (int i = 1; i <= n; ++i) {
      if ((p[i] & 0xC0) != 0x80) return false;
      cp = cp << 6 | (p[i] & 0x3F);
    }
    if (cp < lo || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
    if (s) s->append((const char *)p, n + 1);
    p += n + 1;
    return true;
  }
  bool string(std::string *out) {  // at the opening quote
    ++p;
    while (p < e) {
      const uint8_t c = *p;
      if (c == '"') {
        ++p;
        return true;
      }
      if (c < 0x20) return false;
      if (c != '\\') {
        if (!utf8(out)) return false;
        continue;
      }
      if (++p >= e) return false;
      const uint8_t x = *p++;
      switch (x) {
        case '"': case '\\': case '/':
          if (out) out->push_back((char)x);
          break;
        case 'b': if (out) out->push_back('\b'); break;
        case 'f': if (out) out->push_back('\f'); break;
        case 'n': if (out) out->push_back('\n'); break;
        case 'r': if (out) out->push_back('\r'); break;
        case 't': if (out) out->push_back('\t'); break;
        case 'u': {
          uint32_t v;
          if (!u4(&v)) return false;
          if (v >= 0xDC00 && v <= 0xDFFF) return false;  // a low surrogate alone
          if (v >= 0xD800 && v <= 0xDBFF) {
            uint32_t w;
            if (e - p < 2 || p[0] != '\\' || p[1] != 'u') return false;
            p += 2;
            if (!u4(&w) || w < 0xDC00 || w > 0xDFFF) return false;
            v = 0x10000 + ((v - 0xD800) << 10) + (w - 0xDC00);
          }
          put_utf8(out, v);
          break;
        }
        default:
          return false;
      }
    }
    return false;
  }
  bool number() {
    if (p < e && *p == '-') ++p;
    if (p >= e) return false;
    if (*p == '0') {
      ++p;
    } else if (*p >= '1' && *p <= '9') {
      while (p < e && *p >= '0' && *p <= '9') ++p;
    } else {
      return false;
    }
    if (p < e && *p == '.') {
      ++p;
      if (p >= e || *p < '0' || *p > '9') return false;
      while (p < e && *p >= '0' && *p <= '9') ++p;
    }
    if (p < e && (*p == 'e' || *p == 'E')) {
      ++p;
      if (p < e && (*p == '+' || *p == '-')) ++p;
      if (p >= e || *p < '0' || *p > '9') return false;
      while (p < e && *p >= '0' && *p <= '9') ++p;
    }
    return true;
  }
  bool literal(const char *w) {
    const size_t n = strlen(w);
    if ((size_t)(e - p) < n || memcmp(p, w, n) != 0) return false;
    p += n;
    return true;
  }
};

}  // namespace

bool json_object(const uint8_t *data, size_t n) {
  JsonScan s{data, data + n};
  s.ws();
  if (s.p >= s.e || *s.p != '{') return false;  // the top-level value must be an object
  struct Frame {
    bool object;
    std::set<std::string> keys;
  };
  std::vector<Frame> stack;
  enum { kValue, kAfter } need = kValue;
  for (;;) {
    s.ws();
    if (need == kValue) {
      if (s.p >= s.e) return false;
      const uint8_t c = *s.p;
      if (c == '{' || c == '[') {
        ++s.p;
        stack.push_back({c == '{', {}});
        s.ws();
        if (s.p < s.e && *s.p == (c == '{' ? '}' : ']')) {
          ++s.p;
          stack.pop_back();
        } else if (c == '{') {
          // the first key
          if (s.p >= s.e || *s.p != '"') return false;
          std::string k;
          if (!s.string(&k)) return false;
          stack.back().keys.insert(std::move(k));
          s.ws();
          if (s.p >= s.e || *s.p != ':') return false;
          ++s.p;
          continue;  // a value follows
        } else {
          continue;  // an element follows
        }
      } else if (c == '"') {
        if (!s.string(nullptr)) return false;
      } else if (c == '-' || (c >= '0' && c <= '9')) {
        if (!s.number()) return false;
      } else if (!s.literal("true") && !s.literal("false") && !s.literal("null")) {
        return false;
      }
      need = kAfter;
      continue;
    }
    // after a complete value
    if (stack.empty()) return s.p == s.e;
    if (s.p >= s.e) return false;
    Frame &f = stack.back();
    const uint8_t c = *s.p++;
    if (c == (f.object ? '}' : ']')) {
      stack.pop_back();
      continue;  // the container is a complete value
    }
    if (c != ',') return false;
    if (f.object) {
      s.ws();
      if (s.p >= s.e || *s.p != '"') return false;
      std::string k;
      if (!s.string(&k)) return false;
      if (!f.keys.insert(std::move(k)).second) return false;  // DuplicateField
      s.ws();
      if (s.p >= s.e || *s.p != ':') return false;
      ++s.p;
    }
    need = kValue;
  }
}

// ---- container admission ---------------------------------------------------
Container::~Container() {
  if (bytes && bytes != MAP_FAILED) munmap((void *)bytes, size);
  if (fd >= 0) close(fd);
}

namespace {

// Header.readFrom (format.zig:103-137)
uint32_t read_header(const uint8_t *h, glacier_hip_glacier_header_t *out) {
  if (memcmp(h, "GLAC", 4) != 0) return GLACIER_HIP_GLAC_BAD_MAGIC;
  out->version = rd16(h + 4);
  if (out->version != 1) return GLACIER_HIP_GLAC_BAD_VERSION;
  out->header_size = rd16(h + 6);
  if (out->header_size != kHeaderSize) return GLACIER_HIP_GLAC_BAD_HEADER_SIZE;
  out->meta_offset = rd64(h + 8);
  out->meta_len = rd64(h + 16);
  out->num_pages = rd64(h + 24);
  out->page_index_offset = rd64(h + 32);
  out->page_data_offset = rd64(h + 40);
  out->page_size_log2 = rd32(h + 48);
  if (out->page_size_log2 != kPageSizeLog2) return GLACIER_HIP_GLAC_BAD_PAGE_SIZE;
  out->reserved = rd32(h + 52);
  if (out->reserved != 0) return GLACIER_HIP_GLAC_BAD_RESERVED_FIELD;
  if (!all_zero(h + 56, kHeaderSize - 56)) return GLACIER_HIP_GLAC_BAD_RESERVED_FIELD;
  return GLACIER_HIP_GLAC_OK;
}

// validateHeaderLayoutV1 (:211-247)
uint32_t validate_layout(const glacier_hip_glacier_header_t &h, uint64_t file_size) {
  if (h.meta_offset != kHeaderSize) return GLACIER_HIP_GLAC_BAD_LAYOUT;
  if (h.meta_len > kMaxMetadata) return GLACIER_HIP_GLAC_METADATA_TOO_LARGE;
  if (h.num_pages > kMaxPages) return GLACIER_HIP_GLAC_INDEX_TOO_LARGE;
  uint64_t meta_end, index_bytes, index_end;
  if (add_ovf(h.meta_offset, h.meta_len, &meta_end)) return GLACIER_HIP_GLAC_LAYOUT_OVERFLOW;
  if (h.page_index_offset != meta_end) return GLACIER_HIP_GLAC_BAD_LAYOUT;
  if (mul_ovf(h.num_pages, kEntrySize, &index_bytes)) return GLACIER_HIP_GLAC_LAYOUT_OVERFLOW;
  if (add_ovf(h.page_index_offset, index_bytes, &index_end)) return GLACIER_HIP_GLAC_LAYOUT_OVERFLOW;
  if (h.page_data_offset != index_end) return GLACIER_HIP_GLAC_BAD_LAYOUT;
  if (meta_end > file_size) return GLACIER_HIP_GLAC_TRUNCATED_META;
  if (index_end > file_size) return GLACIER_HIP_GLAC_TRUNCATED_INDEX;
  return GLACIER_HIP_GLAC_OK;
}

bool tensor_kind_valid(uint32_t k) { return k <= 15 || k == 255; }

// PageEntry.readFrom (:169-199): reserved fields, then the enums
uint32_t read_entry(const uint8_t *b, glacier_hip_glacier_page_t *p) {
  memset(p, 0, sizeof *p);
  p->page_id = rd64(b);
  p->layer_idx = rd32(b + 8);
  p->tensor_kind = rd32(b + 12);
  p->row_start = rd64(b + 16);
  p->row_end = rd64(b + 24);
  p->precision = b[32];
  p->quant_group = b[33];
  const uint16_t reserved = rd16(b + 34);
  p->data_offset = rd64(b + 36);
  p->data_len = rd64(b + 44);
  p->crc32 = rd32(b + 52);
  if (reserved != 0 || rd32(b + 56) != 0 || rd32(b + 60) != 0)
    return GLACIER_HIP_GLAC_BAD_RESERVED_FIELD;
  if (!tensor_kind_valid(p->tensor_kind)) return GLACIER_HIP_GLAC_BAD_TENSOR_KIND;
  if (p->precision > kFp32) return GLACIER_HIP_GLAC_BAD_PRECISION;
  return GLACIER_HIP_GLAC_OK;
}

// validatePageGeometryV1 (:277-341)
uint32_t validate_geometry(const glacier_hip_glacier_page_t &p) {
  const uint64_t n = p.row_end - p.row_start;
  uint64_t expected;
  switch (p.precision) {
    case kFp32:
    case kFp16:
    case kBf16:
      if (p.quant_group != 0) return GLACIER_HIP_GLAC_BAD_QUANT_GROUP;
      if (mul_ovf(n, p.precision == kFp32 ? 4 : 2, &expected)) return GLACIER_HIP_GLAC_LAYOUT_OVERFLOW;
      break;
    case kInt8:
    case kInt4: {
      if (p.quant_group == 0) return GLACIER_HIP_GLAC_BAD_QUANT_GROUP;
      if (n > kPageSizeBytes / 4) return GLACIER_HIP_GLAC_PAGE_GEOMETRY_TOO_LARGE;
      const uint64_t groups = ceil_div(n, p.quant_group);
      const uint64_t packed = p.precision == kInt8 ? n : ceil_div(n, 2);
      expected = kSubHeader + groups * 4 + packed;  // bounded: n <= 65536
      break;
    }
    default:
      return GLACIER_HIP_GLAC_UNSUPPORTED_PRECISION;
  }
  if (expected != p.data_len) return GLACIER_HIP_GLAC_BAD_PAGE_GEOMETRY;
  if ((p.precision == kFp32 || p.precision == kFp16 || p.precision == kBf16) && expected > kPageSizeBytes)
    return GLACIER_HIP_GLAC_PAGE_GEOMETRY_TOO_LARGE;
  return GLACIER_HIP_GLAC_OK;
}

// validatePagesV1 (:249-275)
uint32_t validate_pages(const std::vector<glacier_hip_glacier_page_t> &pages, uint64_t data_offset,
                        uint64_t file_size) {
  uint64_t expected = data_offset;
  for (size_t i = 0; i < pages.size(); ++i) {
    const auto &p = pages[i];
    if (p.page_id != i) return GLACIER_HIP_GLAC_BAD_PAGE_ID;
    if (p.row_end <= p.row_start) return GLACIER_HIP_GLAC_BAD_ROW_RANGE;
    if (p.data_len == 0) return GLACIER_HIP_GLAC_EMPTY_PAGE;
    if (uint32_t e = validate_geometry(p)) return e;
    if (p.data_offset != expected) return GLACIER_HIP_GLAC_NON_CONTIGUOUS_PAYLOAD;
    if (add_ovf(p.data_offset, p.data_len, &expected)) return GLACIER_HIP_GLAC_LAYOUT_OVERFLOW;
    if (expected > file_size) return GLACIER_HIP_GLAC_TRUNCATED_PAGE;
  }
  if (expected != file_size) return GLACIER_HIP_GLAC_TRAILING_BYTES;
  return GLACIER_HIP_GLAC_OK;
}

}  // namespace

uint32_t open_container(const char *path, Container **out) {
  *out = nullptr;
  auto *c = new Container();
  auto fail = [&](uint32_t e) {
    delete c;
    return e;
  };
  struct stat st;
  c->fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (c->fd < 0 || fstat(c->fd, &st) != 0) return fail(GLACIER_HIP_GLAC_FILE_ERROR);
  if ((uint64_t)st.st_size < kHeaderSize) return fail(GLACIER_HIP_GLAC_TRUNCATED_HEADER);
  c->size = (size_t)st.st_size;
  void *m = mmap(nullptr, c->size, PROT_READ, MAP_PRIVATE, c->fd, 0);
  if (m == MAP_FAILED) return fail(GLACIER_HIP_GLAC_FILE_ERROR);
  c->bytes = (const uint8_t *)m;
  glacier_hip_glacier_header_t &h = c->header;
  if (uint32_t e = read_header(c->bytes, &h)) return fail(e);
  h.container_bytes = c->size;
  if (uint32_t e = validate_layout(h, c->size)) return fail(e);
  if (!json_object(c->bytes + h.meta_offset, (size_t)h.meta_len)) return fail(GLACIER_HIP_GLAC_BAD_METADATA);
  c->pages.resize((size_t)h.num_pages);
  for (size_t i = 0; i < c->pages.size(); ++i)
    if (uint32_t e = read_entry(c->bytes + h.page_index_offset + i * kEntrySize, &c->pages[i])) return fail(e);
  if (uint32_t e = validate_pages(c->pages, h.page_data_offset, c->size)) return fail(e);
  *out = c;
  return GLACIER_HIP_GLAC_OK;
}

// ---- qio -------------------------------------------------------------------
uint32_t read_quant_header(const uint8_t *buf, size_t len, QuantHeader *h) {
  // readQuantHeader (qio.zig:52-69)
  if (len < kSubHeader) return GLACIER_HIP_GLAC_TRUNCATED_HEADER;
  if (rd32(buf) != kQioMagic) return GLACIER_HIP_GLAC_BAD_MAGIC;
  h->num_elements = rd32(buf + 4);
  h->group_size = rd32(buf + 8);
  if (h->group_size == 0) return GLACIER_HIP_GLAC_BAD_GROUP_SIZE;
  if (buf[12] > kQInt4) return GLACIER_HIP_GLAC_BAD_PRECISION;
  h->precision = buf[12];
  return GLACIER_HIP_GLAC_OK;
}

uint32_t qio_encode_f32(const float *src, uint64_t n, uint32_t precision, uint32_t group_size,
                        std::vector<uint8_t> &out) {
  // quant.quantize (quant.zig:36-112) into encodePage's payload (qio.zig:72-112)
  if (precision > kQInt4) return GLACIER_HIP_GLAC_BAD_PRECISION;
  if (n > 0xFFFFFFFFull) return GLACIER_HIP_GLAC_INVALID_PAYLOAD_SIZE;  // num_elements is a u32
  for (uint64_t i = 0; i < n; ++i)
    if (!isfinite(src[i])) return GLACIER_HIP_GLAC_INVALID_VALUE;
  if (n > 0 && group_size == 0) return GLACIER_HIP_GLAC_BAD_GROUP_SIZE;
  const int bits = precision == kQInt8 ? 8 : 4;
  const int qzero = (1 << (bits - 1)) - 1;  // 127 or 7
  const int qmin = -qzero;
  // INT4 groups of 16 or more use the spare code 15 for +8
  const int qmax = precision == kQInt4 && group_size >= 16 ? qzero + 1 : qzero;
  const uint64_t groups = n ? ceil_div(n, group_size) : 0;
  const uint64_t packed_len = ceil_div(n * bits, 8);
  out.assign(kSubHeader + groups * 4 + packed_len, 0);
  uint8_t *o = out.data();
  wr32(o, kQioMagic);
  wr32(o + 4, (uint32_t)n);
  wr32(o + 8, group_size);
  o[12] = (uint8_t)precision;
  uint8_t *packed = o + kSubHeader + groups * 4;
  for (uint64_t g = 0, i = 0; i < n; ++g) {
    const uint64_t end = i + std::min<uint64_t>(group_size, n - i);
    float lo = 0.0f, hi = 0.0f;
    for (uint64_t j = i; j < end; ++j) {
      lo = min_number(lo, src[j]);
      hi = max_number(hi, src[j]);
    }
    const float neg = -lo / (float)(-qmin);
    const float pos = hi / (float)qmax;
    const float scale = max_number(neg, pos);
    uint32_t sb;
    memcpy(&sb, &scale, 4);
    wr32(o + kSubHeader + g * 4, sb);
    const float inv = scale == 0.0f ? 0.0f : 1.0f / scale;
    for (uint64_t j = i; j < end; ++j) {
      int q = (int)roundf(src[j] * inv);  // @round: half away from zero
      q = std::min(std::max(q, qmin), qmax);
      const uint8_t u = (uint8_t)(q + qzero);
      if (bits == 8) {
        packed[j] = u;
      } else if (j % 2 == 0) {
        packed[j / 2] = (uint8_t)((packed[j / 2] & 0xF0) | (u & 0x0F));
      } else {
        packed[j / 2] = (uint8_t)((packed[j / 2] & 0x0F) | (u & 0x0F) << 4);
      }
    }
    i = end;
  }
  return GLACIER_HIP_GLAC_OK;
}

uint32_t qio_decode_f32(const uint8_t *payload, size_t len, std::vector<float> &out) {
  // decodePage (qio.zig:115-162) and quant.dequantize (quant.zig:114-163)
  QuantHeader h;
  if (uint32_t e = read_quant_header(payload, len, &h)) return e;
  const uint64_t n = h.num_elements, groups = ceil_div(n, h.group_size);
  const uint64_t packed_off = kSubHeader + groups * 4;  // bounded: n < 2^32
  if (len < packed_off) return GLACIER_HIP_GLAC_TRUNCATED_SCALES;
  const int bits = h.precision == kQInt8 ? 8 : 4;
  const uint64_t packed_len = ceil_div(n * bits, 8);
  if (len - packed_off < packed_len) return GLACIER_HIP_GLAC_TRUNCATED_PACKED;
  const int qmax = (1 << (bits - 1)) - 1;
  const uint8_t *packed = payload + packed_off;
  out.resize(n);
  for (uint64_t i = 0; i < n; ++i) {
    uint32_t sb = rd32(payload + kSubHeader + (i / h.group_size) * 4);
    float scale;
    memcpy(&scale, &sb, 4);
    const int u = bits == 8 ? packed[i] : (i % 2 == 0 ? packed[i / 2] & 0x0F : packed[i / 2] >> 4);
    out[i] = (float)(u - qmax) * scale;
  }
  return GLACIER_HIP_GLAC_OK;
}

// ---- pages -----------------------------------------------------------------
uint32_t validate_payload_schema(const Container &c, const glacier_hip_glacier_page_t &p) {
  switch (p.precision) {
    case kFp32: case kFp16: case kBf16: return GLACIER_HIP_GLAC_OK;
    case kInt8: case kInt4: break;
    default: return GLACIER_HIP_GLAC_UNSUPPORTED_PRECISION;
  }
  if (p.data_offset + kSubHeader > c.size) return GLACIER_HIP_GLAC_TRUNCATED_PAGE;
  const uint8_t *b = c.bytes + p.data_offset;
  if (!all_zero(b + 13, 3)) return GLACIER_HIP_GLAC_BAD_QUANT_PAYLOAD;
  QuantHeader h;
  if (read_quant_header(b, kSubHeader, &h)) return GLACIER_HIP_GLAC_BAD_QUANT_PAYLOAD;
  if (h.num_elements != p.row_end - p.row_start || h.group_size != p.quant_group)
    return GLACIER_HIP_GLAC_BAD_QUANT_PAYLOAD;
  if (h.precision != (p.precision == kInt8 ? kQInt8 : kQInt4)) return GLACIER_HIP_GLAC_BAD_QUANT_PAYLOAD;
  return GLACIER_HIP_GLAC_OK;
}

uint32_t validate_all_crcs(const Container &c, uint64_t buffer_bytes) {
  if (buffer_bytes == 0) return GLACIER_HIP_GLAC_EMPTY_STREAM_BUFFER;
  for (const auto &p : c.pages) {
    if (uint32_t e = validate_payload_schema(c, p)) return e;
    // the CRC is the same over any chunking; one pass over the mapping
    if (gri::crc32(c.bytes + p.data_offset, (size_t)p.data_len) != p.crc32)
      return GLACIER_HIP_GLAC_CRC_MISMATCH;
  }
  return GLACIER_HIP_GLAC_OK;
}

uint32_t read_page(const Container &c, const glacier_hip_glacier_page_t &p, const uint8_t **data) {
  const uint8_t *b = c.bytes + p.data_offset;
  if (gri::crc32(b, (size_t)p.data_len) != p.crc32) return GLACIER_HIP_GLAC_CRC_MISMATCH;
  *data = b;
  return GLACIER_HIP_GLAC_OK;
}

uint32_t read_page_f32(const Container &c, const glacier_hip_glacier_page_t &p, std::vector<float> &out) {
  const uint8_t *b;
  if (uint32_t e = read_page(c, p, &b)) return e;
  const uint64_t n = p.row_end - p.row_start;
  switch (p.precision) {
    case kFp32: case kFp16: case kBf16: {  // decodeRawPageV1 (:665-717)
      const uint64_t w = p.precision == kFp32 ? 4 : 2;
      if (n * w != p.data_len) return GLACIER_HIP_GLAC_SIZE_MISMATCH;
      out.resize(n);
      for (uint64_t i = 0; i < n; ++i) {
        if (p.precision == kFp32) {
          const uint32_t v = rd32(b + 4 * i);
          memcpy(&out[i], &v, 4);
        } else if (p.precision == kFp16) {
          out[i] = gh::f16_to_f32(rd16(b + 2 * i));
        } else {
          const uint32_t v = (uint32_t)rd16(b + 2 * i) << 16;
          memcpy(&out[i], &v, 4);
        }
      }
      return GLACIER_HIP_GLAC_OK;
    }
    case kInt8: case kInt4:
      if (uint32_t e = validate_payload_schema(c, p)) return e;
      return qio_decode_f32(b, (size_t)p.data_len, out);
    default:
      return GLACIER_HIP_GLAC_UNSUPPORTED_PRECISION;
  }
}

void source_fingerprint(const Container &c, uint8_t out[32]) {
  gh::Sha256 h;
  static const char dom[] = "glacier-source-fingerprint-v1";
  h.update(dom, sizeof dom);  // with its NUL
  const uint8_t v[2] = {(uint8_t)c.header.version, (uint8_t)(c.header.version >> 8)};
  h.update(v, 2);
  h.u64(c.header.meta_len);
  h.update(c.bytes + c.header.meta_offset, (size_t)c.header.meta_len);
  h.u64(c.pages.size());
  for (const auto &p : c.pages) {
    h.u64(p.page_id);
    h.u32(p.layer_idx);
    h.u32(p.tensor_kind);
    h.u64(p.row_start);
    h.u64(p.row_end);
    const uint8_t pq[2] = {(uint8_t)p.precision, (uint8_t)p.quant_group};
    h.update(pq, 2);
    h.u32(p.crc32);
    h.u64(p.data_len);
  }
  h.final(out);
}

// ---- loader assembly -------------------------------------------------------
uint32_t derive_geometry(const Container &c, Geometry *g) {
  // loadWithOptions' first pass (loader.zig:1226-1268)
  *g = Geometry{};
  if (c.pages.empty()) return GLACIER_HIP_GLAC_NO_LAYERS;
  for (const auto &p : c.pages) {
    g->num_layers = std::max<uint32_t>(g->num_layers, p.layer_idx + 1);
    switch (p.tensor_kind) {
      case 8: case 11: case 10: g->dim = std::max(g->dim, p.row_end); break;        // norms
      case 5: case 7: case 6: g->hidden_dim = std::max(g->hidden_dim, p.row_end); break;  // mlp
      case 0: case 9: g->vocab_size = std::max(g->vocab_size, p.row_end); break;   // embedding / head
      default: break;
    }
  }
  if (g->dim > 0) {
    if (g->hidden_dim > g->dim) g->hidden_dim /= g->dim;
    if (g->vocab_size > g->dim) g->vocab_size /= g->dim;
  } else {
    g->dim = g->hidden_dim > 0 ? g->hidden_dim / 4 : 16;
    g->hidden_dim = 4 * g->dim;
  }
  if (g->num_layers == 0 || g->dim == 0) return GLACIER_HIP_GLAC_MISSING_TENSOR;
  return GLACIER_HIP_GLAC_OK;
}

namespace {

bool compact_kind(uint32_t k) {  // isCompactTensorKind (:1594-1607)
  switch (k) {
    case 0: case 1: case 2: case 3: case 4: case 7: case 5: case 6: case 9: return true;
    default: return false;
  }
}

// concatInt4Pages (:1636-1720)
uint32_t concat_int4(const Container &c, const std::vector<const glacier_hip_glacier_page_t *> &pages,
                     Group &g) {
  if (pages.empty()) return GLACIER_HIP_GLAC_BAD_PAYLOAD;
  uint32_t group = 0;
  uint64_t total = 0, total_scales = 0;
  for (size_t i = 0; i < pages.size(); ++i) {
    const auto &p = *pages[i];
    if (p.precision != kInt4 || p.quant_group == 0 || p.row_end < p.row_start) return GLACIER_HIP_GLAC_BAD_PAYLOAD;
    if (group == 0) group = p.quant_group;
    if (p.quant_group != group) return GLACIER_HIP_GLAC_BAD_PAYLOAD;
    const uint64_t n = p.row_end - p.row_start;
    if (i + 1 < pages.size() && n % group) return GLACIER_HIP_GLAC_BAD_PAYLOAD;
    const uint64_t ps = ceil_div(n, group);
    if (p.data_len != kSubHeader + ps * 4 + ceil_div(n, 2)) return GLACIER_HIP_GLAC_BAD_PAYLOAD;
    total += n;
    total_scales += ps;
  }
  if (total_scales != ceil_div(total, group)) return GLACIER_HIP_GLAC_BAD_PAYLOAD;
  g.int4 = true;
  g.group_size = group;
  g.elements = total;
  g.packed.assign(ceil_div(total, 2), 0);
  g.scales.resize(total_scales);
  uint64_t de = 0, ds = 0;
  for (const auto *pp : pages) {
    const auto &p = *pp;
    const uint8_t *b;
    if (read_page(c, p, &b)) return GLACIER_HIP_GLAC_BAD_PAYLOAD;
    QuantHeader h;
    if (read_quant_header(b, (size_t)p.data_len, &h)) return GLACIER_HIP_GLAC_BAD_PAYLOAD;
    const uint64_t n = h.num_elements;
    if (h.precision != kQInt4 || h.group_size != group || n != p.row_end - p.row_start)
      return GLACIER_HIP_GLAC_BAD_PAYLOAD;
    const uint64_t ps = ceil_div(n, h.group_size), off = kSubHeader + ps * 4, plen = (n + 1) / 2;
    if (p.data_len < off || p.data_len - off < plen) return GLACIER_HIP_GLAC_BAD_PAYLOAD;
    for (uint64_t s = 0; s < ps; ++s) {
      const uint32_t v = rd32(b + kSubHeader + s * 4);
      memcpy(&g.scales[ds + s], &v, 4);
    }
    const uint8_t *src = b + off;
    if (de % 2 == 0 && n % 2 == 0) {
      memcpy(g.packed.data() + de / 2, src, (size_t)plen);
    } else {
      for (uint64_t i = 0; i < n; ++i) {
        const uint8_t u = (i % 2 == 0) ? src[i / 2] & 0x0F : src[i / 2] >> 4;
        const uint64_t d = de + i;
        uint8_t &t = g.packed[d / 2];
        t = d % 2 == 0 ? (uint8_t)((t & 0xF0) | u) : (uint8_t)((t & 0x0F) | u << 4);
      }
    }
    de += n;
    ds += ps;
  }
  if (de != total || ds != total_scales) return GLACIER_HIP_GLAC_BAD_PAYLOAD;
  return GLACIER_HIP_GLAC_OK;
}

// decodePageF32 (:1759-1822): the qio magic selects the quantized decode;
// otherwise the bytes are read by the stored precision (fp32 for the rest)
uint32_t decode_page_loader(const Container &c, const glacier_hip_glacier_page_t &p,
                            std::vector<float> &out) {
  const uint8_t *b;
  if (read_page(c, p, &b)) return GLACIER_HIP_GLAC_BAD_PAYLOAD;
  const uint64_t len = p.data_len;
  if (len >= 4 && rd32(b) == kQioMagic)
    return qio_decode_f32(b, (size_t)len, out) ? GLACIER_HIP_GLAC_BAD_PAYLOAD : GLACIER_HIP_GLAC_OK;
  if (p.precision == kFp16 || p.precision == kBf16) {
    if (len % 2) return GLACIER_HIP_GLAC_BAD_PAYLOAD;
    out.resize(len / 2);
    for (uint64_t i = 0; i < len / 2; ++i) {
      if (p.precision == kFp16) {
        out[i] = gh::f16_to_f32(rd16(b + 2 * i));
      } else {
        const uint32_t v = (uint32_t)rd16(b + 2 * i) << 16;
        memcpy(&out[i], &v, 4);
      }
    }
    return GLACIER_HIP_GLAC_OK;
  }
  if (len % 4) return GLACIER_HIP_GLAC_BAD_PAYLOAD;
  out.resize(len / 4);
  memcpy(out.data(), b, (size_t)len);
  return GLACIER_HIP_GLAC_OK;
}

}  // namespace

uint32_t materialize(const Container &c, std::map<GroupKey, Group> &groups) {
  // bucket by (layer, kind) in page order, visit groups by (layer, kind)
  std::map<GroupKey, std::vector<const glacier_hip_glacier_page_t *>> byk;
  for (const auto &p : c.pages) byk[{p.layer_idx, p.tensor_kind}].push_back(&p);
  for (auto &kv : byk) {
    auto &pages = kv.second;
    std::sort(pages.begin(), pages.end(), [](auto *a, auto *b) { return a->page_id < b->page_id; });
    Group &g = groups[kv.first];
    const bool all_int4 = std::all_of(pages.begin(), pages.end(), [](auto *p) { return p->precision == kInt4; });
    if (compact_kind(kv.first.second) && all_int4) {
      if (uint32_t e = concat_int4(c, pages, g)) return e;
      continue;
    }
    for (const auto *p : pages) {  // decodePageF32 per page, concatenated
      if (p->row_end < p->row_start) return GLACIER_HIP_GLAC_BAD_PAYLOAD;
      std::vector<float> part;
      if (decode_page_loader(c, *p, part)) return GLACIER_HIP_GLAC_BAD_PAYLOAD;
      if (part.size() != p->row_end - p->row_start) return GLACIER_HIP_GLAC_BAD_PAYLOAD;
      g.values.insert(g.values.end(), part.begin(), part.end());
    }
    g.elements = g.values.size();
  }
  return GLACIER_HIP_GLAC_OK;
}

const char *error_name(uint32_t e) {
  static const char *names[] = {
      "Ok", "TruncatedHeader", "BadMagic", "BadVersion", "BadHeaderSize", "BadPageSize",
      "BadReservedField", "BadLayout", "MetadataTooLarge", "IndexTooLarge", "LayoutOverflow",
      "TruncatedMeta", "TruncatedIndex", "BadMetadata", "BadTensorKind", "BadPrecision",
      "BadPageId", "BadRowRange", "EmptyPage", "BadQuantGroup", "PageGeometryTooLarge",
      "BadPageGeometry", "UnsupportedPrecision", "NonContiguousPayload", "TruncatedPage",
      "TrailingBytes", "CrcMismatch", "BadQuantPayload", "BufferTooSmall", "EmptyStreamBuffer",
      "FileError", "SizeMismatch", "BadGroupSize", "TruncatedScales", "TruncatedPacked",
      "InvalidPayloadSize", "InvalidValue", "NoLayers", "MissingTensor", "BadPayload",
      "Unsupported", "InvalidArgument"};
  return e < sizeof(names) / sizeof(names[0]) ? names[e] : "Unknown";
}

}  // namespace gct

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
struct glacier_hip_glacier {
  gct::Container *c;
};

namespace gct {
const Container *container_of(const glacier_hip_glacier *h) { return h ? h->c : nullptr; }
}  // namespace gct

extern "C" {

const char *glacier_hip_glacier_error_name(uint32_t code) { return gct::error_name(code); }

int glacier_hip_glacier_open(const char *path, glacier_hip_glacier **out) {
  if (!path || !out) return GLACIER_HIP_GLAC_INVALID_ARGUMENT;
  *out = nullptr;
  gct::Container *c = nullptr;
  if (uint32_t e = gct::open_container(path, &c)) return (int)e;
  *out = new glacier_hip_glacier{c};
  return GLACIER_HIP_GLAC_OK;
}

void glacier_hip_glacier_close(glacier_hip_glacier *c) {
  if (!c) return;
  delete c->c;
  delete c;
}

int glacier_hip_glacier_header(const glacier_hip_glacier *c, glacier_hip_glacier_header_t *out) {
  if (!c || !out) return GLACIER_HIP_GLAC_INVALID_ARGUMENT;
  *out = c->c->header;
  return GLACIER_HIP_GLAC_OK;
}

int glacier_hip_glacier_page(const glacier_hip_glacier *c, uint64_t index, glacier_hip_glacier_page_t *out) {
  if (!c || !out || index >= c->c->pages.size()) return GLACIER_HIP_GLAC_INVALID_ARGUMENT;
  *out = c->c->pages[index];
  return GLACIER_HIP_GLAC_OK;
}

int glacier_hip_glacier_metadata(const glacier_hip_glacier *c, const void **data, uint64_t *len) {
  if (!c || !data || !len) return GLACIER_HIP_GLAC_INVALID_ARGUMENT;
  *data = c->c->bytes + c->c->header.meta_offset;
  *len = c->c->header.meta_len;
  return GLACIER_HIP_GLAC_OK;
}

int glacier_hip_glacier_read_page(const glacier_hip_glacier *c, uint64_t index, void *dst, uint64_t dst_len) {
  if (!c || (!dst && dst_len) || index >= c->c->pages.size()) return GLACIER_HIP_GLAC_INVALID_ARGUMENT;
  const auto &p = c->c->pages[index];
  if (dst_len < p.data_len) return GLACIER_HIP_GLAC_BUFFER_TOO_SMALL;
  const uint8_t *b;
  if (uint32_t e = gct::read_page(*c->c, p, &b)) return (int)e;
  memcpy(dst, b, (size_t)p.data_len);
  return GLACIER_HIP_GLAC_OK;
}

int glacier_hip_glacier_read_page_f32(const glacier_hip_glacier *c, uint64_t index, float *dst,
                                      uint64_t capacity, uint64_t *count) {
  if (!c || !count || index >= c->c->pages.size()) return GLACIER_HIP_GLAC_INVALID_ARGUMENT;
  std::vector<float> v;
  if (uint32_t e = gct::read_page_f32(*c->c, c->c->pages[index], v)) return (int)e;
  *count = v.size();
  if (capacity < v.size() || (!dst && !v.empty())) return GLACIER_HIP_GLAC_BUFFER_TOO_SMALL;
  if (!v.empty()) memcpy(dst, v.data(), v.size() * 4);
  return GLACIER_HIP_GLAC_OK;
}

int glacier_hip_glacier_validate_crcs(const glacier_hip_glacier *c, uint64_t buffer_bytes) {
  if (!c) return GLACIER_HIP_GLAC_INVALID_ARGUMENT;
  return (int)gct::validate_all_crcs(*c->c, buffer_bytes);
}

int glacier_hip_glacier_identity(const glacier_hip_glacier *c, uint8_t container_sha256[32],
                                 uint64_t *container_bytes) {
  if (!c || !container_sha256) return GLACIER_HIP_GLAC_INVALID_ARGUMENT;
  gh::Sha256 h;
  h.update(c->c->bytes, c->c->size);
  h.final(container_sha256);
  if (container_bytes) *container_bytes = c->c->size;
  return GLACIER_HIP_GLAC_OK;
}

int glacier_hip_glacier_source_fingerprint(const glacier_hip_glacier *c, uint8_t out[32]) {
  if (!c || !out) return GLACIER_HIP_GLAC_INVALID_ARGUMENT;
  gct::source_fingerprint(*c->c, out);
  return GLACIER_HIP_GLAC_OK;
}

int glacier_hip_glacier_assemble(const glacier_hip_glacier *c, glacier_hip_glacier_assembly_t *out) {
  if (!c || !out) return GLACIER_HIP_GLAC_INVALID_ARGUMENT;
  memset(out, 0, sizeof *out);
  gct::Geometry g;
  std::map<gct::GroupKey, gct::Group> groups;
  uint32_t e = gct::derive_geometry(*c->c, &g);
  if (!e) e = gct::materialize(*c->c, groups);
  out->error = e;
  out->num_layers = g.num_layers;
  out->dim = g.dim;
  out->hidden_dim = g.hidden_dim;
  out->vocab_size = g.vocab_size;
  if (e) return (int)e;
  gh::Sha256 h;
  static const char dom[] = "glacier-hip-assembly-v1";
  h.update(dom, sizeof dom);
  h.u64(groups.size());
  for (const auto &kv : groups) {
    const gct::Group &gr = kv.second;
    h.u32(kv.first.first);
    h.u32(kv.first.second);
    h.u32(gr.int4 ? 1 : 0);
    h.u32(gr.group_size);
    h.u64(gr.elements);
    if (gr.int4) {
      h.update(gr.packed.data(), gr.packed.size());
      h.update(gr.scales.data(), gr.scales.size() * 4);  // little-endian host
    } else {
      h.update(gr.values.data(), gr.values.size() * 4);
    }
    out->groups++;
    out->int4_groups += gr.int4;
  }
  h.final(out->sha256);
  return GLACIER_HIP_GLAC_OK;
}

int glacier_hip_qio_encode_f32(const float *src, uint64_t count, uint32_t precision,
                               uint32_t group_size, uint8_t *out, uint64_t capacity, uint64_t *len) {
  if ((!src && count) || !len) return GLACIER_HIP_GLAC_INVALID_ARGUMENT;
  std::vector<uint8_t> b;
  if (uint32_t e = gct::qio_encode_f32(src, count, precision, group_size, b)) return (int)e;
  *len = b.size();
  if (capacity < b.size() || !out) return GLACIER_HIP_GLAC_BUFFER_TOO_SMALL;
  memcpy(out, b.data(), b.size());
  return GLACIER_HIP_GLAC_OK;
}

int glacier_hip_qio_decode_f32(const uint8_t *payload, uint64_t len, float *out, uint64_t capacity,
                               uint64_t *count) {
  if ((!payload && len) || !count) return GLACIER_HIP_GLAC_INVALID_ARGUMENT;
  std::vector<float> v;
  if (uint32_t e = gct::qio_decode_f32(payload, (size_t)len, v)) return (int)e;
  *count = v.size();
  if (capacity < v.size() || (!out && !v.empty())) return GLACIER_HIP_GLAC_BUFFER_TOO_SMALL;
  if (!v.empty()) memcpy(out, v.data(), v.size() * 4);
  return GLACIER_HIP_GLAC_OK;
}

}  // extern "C"
