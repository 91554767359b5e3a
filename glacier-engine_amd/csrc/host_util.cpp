// host_util.cpp — SHA-256 from FIPS 180-4 and IEEE binary16 conversion.
#include "host_util.h"

#include <cpuid.h>
#include <immintrin.h>

namespace gh {

static const uint32_t K[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4,
    0xab1c5ed5, 0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe,
    0x9bdc06a7, 0xc19bf174, 0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f,
    0x4a7484aa, 0x5cb0a9dc, 0x76f988da, 0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7,
    0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967, 0x27b70a85, 0x2e1b2138, 0x4d2c6dfc,
    0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85, 0xa2bfe8a1, 0xa81a664b,
    0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070, 0x19a4c116,
    0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7,
    0xc67178f2};

static inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

static void compress(uint32_t h[8], const uint8_t *p) {
  uint32_t w[64];
  for (int i = 0; i < 16; ++i)
    w[i] = ((uint32_t)p[4 * i] << 24) | ((uint32_t)p[4 * i + 1] << 16) |
           ((uint32_t)p[4 * i + 2] << 8) | (uint32_t)p[4 * i + 3];
  for (int i = 16; i < 64; ++i) {
    uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
    uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
    w[i] = w[i - 16] + s0 + w[i - 7] + s1;
  }
  uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
  for (int i = 0; i < 64; ++i) {
    uint32_t t1 = hh + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + K[i] + w[i];
    uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
    hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
  }
  h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
}

// The same compression with the x86 SHA extensions (SHA-256 rounds two at
// a time, the message schedule in 4-word groups), used when the CPU has them.
// State registers hold (A, B, E, F) and (C, D, G, H).
__attribute__((target("sha,sse4.1,ssse3"))) static void compress_shani(uint32_t h[8],
                                                                        const uint8_t *p,
                                                                        size_t blocks) {
  const __m128i bswap = _mm_set_epi64x(0x0c0d0e0f08090a0bLL, 0x0405060700010203LL);
  __m128i tmp = _mm_shuffle_epi32(_mm_loadu_si128((const __m128i *)&h[0]), 0xB1);  // C D A B
  __m128i s1 = _mm_shuffle_epi32(_mm_loadu_si128((const __m128i *)&h[4]), 0x1B);   // H G F E
  __m128i s0 = _mm_alignr_epi8(tmp, s1, 8);                                         // A B E F
  s1 = _mm_blend_epi16(s1, tmp, 0xF0);                                              // C D G H
  for (; blocks; --blocks, p += 64) {
    const __m128i save0 = s0, save1 = s1;
    __m128i w[4];
    for (int g = 0; g < 16; ++g) {
      __m128i m;
      if (g < 4) {
        m = _mm_shuffle_epi8(_mm_loadu_si128((const __m128i *)(p + 16 * g)), bswap);
      } else {  // W[t..t+3] = sigma1 terms + W[t-7..] + W[t-16..] + sigma0 terms
        m = _mm_sha256msg1_epu32(w[g & 3], w[(g + 1) & 3]);
        m = _mm_add_epi32(m, _mm_alignr_epi8(w[(g + 3) & 3], w[(g + 2) & 3], 4));
        m = _mm_sha256msg2_epu32(m, w[(g + 3) & 3]);
      }
      w[g & 3] = m;
      __m128i k = _mm_add_epi32(m, _mm_loadu_si128((const __m128i *)&K[4 * g]));
      s1 = _mm_sha256rnds2_epu32(s1, s0, k);
      s0 = _mm_sha256rnds2_epu32(s0, s1, _mm_shuffle_epi32(k, 0x0E));
    }
    s0 = _mm_add_epi32(s0, save0);
    s1 = _mm_add_epi32(s1, save1);
  }
  tmp = _mm_shuffle_epi32(s0, 0x1B);       // F E B A
  s1 = _mm_shuffle_epi32(s1, 0xB1);        // D C H G
  s0 = _mm_blend_epi16(tmp, s1, 0xF0);     // D C B A
  s1 = _mm_alignr_epi8(s1, tmp, 8);        // H G F E
  _mm_storeu_si128((__m128i *)&h[0], s0);
  _mm_storeu_si128((__m128i *)&h[4], s1);
}

static bool have_shani() {
  static const bool yes = [] {
    unsigned a, b, c, d;
    if (!__get_cpuid(1, &a, &b, &c, &d) || !(c & bit_SSE4_1) || !(c & bit_SSSE3)) return false;
    if (!__get_cpuid_count(7, 0, &a, &b, &c, &d)) return false;
    return (b & (1u << 29)) != 0;  // CPUID.(7,0):EBX.SHA
  }();
  return yes;
}

static void compress_blocks(uint32_t h[8], const uint8_t *p, size_t blocks) {
  if (have_shani()) {
    compress_shani(h, p, blocks);
    return;
  }
  for (; blocks; --blocks, p += 64) compress(h, p);
}

Sha256::Sha256() {
  static const uint32_t iv[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                                 0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
  memcpy(h, iv, sizeof iv);
}

void Sha256::update_blocks(const void *data, size_t n) {
  const uint8_t *p = (const uint8_t *)data;
  len += n;
  if (fill == 0 && n >= 64) {  // whole blocks straight from the input
    compress_blocks(h, p, n / 64);
    p += n / 64 * 64;
    n %= 64;
  }
  while (n) {
    size_t take = std::min(64 - fill, n);
    memcpy(buf + fill, p, take);
    fill += take;
    p += take;
    n -= take;
    if (fill == 64) {
      compress_blocks(h, buf, 1);
      fill = 0;
    }
  }
}

void Sha256::final(uint8_t out[32]) {
  uint64_t bits = len * 8;
  uint8_t pad = 0x80, z = 0;
  update(&pad, 1);
  while (fill != 56) update(&z, 1);
  uint8_t lb[8];
  for (int i = 0; i < 8; ++i) lb[i] = (uint8_t)(bits >> (56 - 8 * i));
  update(lb, 8);
  for (int i = 0; i < 8; ++i) {
    out[4 * i] = (uint8_t)(h[i] >> 24);
    out[4 * i + 1] = (uint8_t)(h[i] >> 16);
    out[4 * i + 2] = (uint8_t)(h[i] >> 8);
    out[4 * i + 3] = (uint8_t)h[i];
  }
}

uint16_t f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7FFFFFFFu;
  if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
  if (ax < 0x38800000u) {
    if (ax < 0x33000000u) return (uint16_t)sign;
    const uint32_t e = ax >> 23, m = (ax & 0x7FFFFFu) | 0x800000u;
    const uint32_t shift = 126 - e;
    uint32_t r = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1), halfv = 1u << (shift - 1);
    if (rem > halfv || (rem == halfv && (r & 1))) ++r;
    return (uint16_t)(sign | r);
  }
  uint32_t r = (ax >> 13) - (112u << 10);
  const uint32_t rem = ax & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1))) ++r;
  return (uint16_t)(sign | r);
}

float f16_to_f32(uint16_t hv) {
  const uint32_t sign = (uint32_t)(hv >> 15) << 31;
  const uint32_t e = (hv >> 10) & 0x1F, m = hv & 0x3FF;
  uint32_t bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {
      float f = (float)m * 5.9604644775390625e-8f;
      memcpy(&bits, &f, 4);
      bits |= sign;
    }
  } else if (e == 31) {
    bits = sign | 0x7F800000u | (m << 13);
  } else {
    bits = sign | ((e + 112) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

void token_sequence_sha256(const uint32_t *tokens, size_t count, uint8_t out[32]) {
  Sha256 h;
  h.update("glacier-output-token-state-v1\0", 30);
  h.u64(count);
  for (size_t i = 0; i < count; ++i) h.u32(tokens[i]);
  h.final(out);
}

}  // namespace gh
