// host_util.h — host-side helpers of the runtime: SHA-256 (FIPS 180-4),
// fp16 conversion, little-endian hashing of integers, and a row-split
// parallel-for over std::thread.
#pragma once
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <thread>
#include <vector>

namespace gh {

struct Sha256 {
  uint32_t h[8];
  uint64_t len = 0;
  uint8_t buf[64];
  size_t fill = 0;
  Sha256();
  // bytes that fit the partial block are buffered inline (most fields are a
  // few bytes); whole blocks go to the compression
  void update(const void *data, size_t n) {
    if (n < 64 - fill) {
      if (n) memcpy(buf + fill, data, n);
      fill += n;
      len += n;
      return;
    }
    update_blocks(data, n);
  }
  void update_blocks(const void *data, size_t n);
  void final(uint8_t out[32]);
  void u64(uint64_t v) {
    uint8_t b[8];
    for (int i = 0; i < 8; ++i) b[i] = (uint8_t)(v >> (8 * i));
    update(b, 8);
  }
  void u32(uint32_t v) {
    uint8_t b[4];
    for (int i = 0; i < 4; ++i) b[i] = (uint8_t)(v >> (8 * i));
    update(b, 4);
  }
};

// tokenSequenceSha256 (generate.zig:3193-3203): domain, count (u64 LE),
// then every token (u32 LE)
void token_sequence_sha256(const uint32_t *tokens, size_t count, uint8_t out[32]);

uint16_t f32_to_f16(float f);
float f16_to_f32(uint16_t h);

template <class F>
void parallel_for(size_t n, F fn, size_t min_chunk = 1024) {
  unsigned hw = std::thread::hardware_concurrency();
  size_t nt = std::min<size_t>(hw ? hw : 1, 32);
  if (n < min_chunk * 2 || nt <= 1) {
    fn(0, n);
    return;
  }
  nt = std::min(nt, (n + min_chunk - 1) / min_chunk);
  std::vector<std::thread> th;
  size_t chunk = (n + nt - 1) / nt;
  for (size_t i = 1; i < nt; ++i) {
    size_t b = i * chunk, e = std::min(n, b + chunk);
    if (b < e) th.emplace_back(fn, b, e);
  }
  fn(0, std::min(n, chunk));
  for (auto &t : th) t.join();
}

}  // namespace gh
