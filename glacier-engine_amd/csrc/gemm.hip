// gemm.hip — K2: INT4 x int8-digit prefill GEMM on gfx950 MFMA.
//
// y[M][N] = planes(x)[M][K] . W^T for prompt chunks (M > 32 rows), with the
// same digit planes, tile layout and fused epilogues as the decode GEMV (K1):
// the per-group arithmetic is the reference's Q8 dot
// (int4_matmul.zig:365-418): an exact integer dot per 32-element group,
// scaled by the weight and activation group scales and summed in f32.
//
// One v_mfma_i32_16x16x32_i8 covers exactly one group of a 16x16 output tile.
// The weight codes are turned into signed int8 (u - 7) in registers, so the
// MFMA result is the group dot itself (no correction term). The MFMA
// accumulator input is preset to 0x4B400000, the bit pattern of 1.5 * 2^23:
// for |T| < 2^22 the integer sum 0x4B400000 + T read as f32 is exactly
// 12582912 + T, so  fma(that, ws, -12582912 * ws)  yields RN(T * ws) (the
// reference's f32(T) * s_w) in one instruction with no int->float convert;
// -12582912 * ws is exact because ws is an fp16 value. The activation scale is
// then applied with one fma into the running sum. Three-digit (f32
// activation) planes chain three MFMAs with a 7-bit shift between them, which
// gives the exact 128-adic integer T; |T| can exceed 2^22 there, so that path
// converts explicitly.
//
// Block = 4 waves in a 2 x 2 arrangement, a wave owns MT x NT 16x16 output
// tiles, loads straight from HBM/L2 (A rows of one group are 512 contiguous
// bytes per tile, B codes 256 contiguous bytes per tile) and keeps the next
// group's operands in flight while it computes the current one. Block ids are
// remapped so that the blocks of one weight column tile run on one XCD
// (hardware places block b on XCD b % 8), which keeps that tile in the XCD's
// L2 for every row tile that reads it.
#include "epilogue.h"
#include "kernels.h"

#include <algorithm>

namespace gk {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kMagic = 0x4B400000;        // bits of 12582912.0f = 1.5 * 2^23
constexpr float kMagicF = 12582912.0f;

// 8 codes (u32 word: low nibbles k0..3, high nibbles k4..7) -> 8 signed bytes
// (u - 7). Per byte, u + 0x79 stays below 0x100, and flipping bit 7 of
// (u + 121) gives (u - 7) in two's complement.
__device__ __forceinline__ long signed_codes(uint32_t w) {
  const uint32_t lo = ((w & 0x0F0F0F0Fu) + 0x79797979u) ^ 0x80808080u;
  const uint32_t hi = (((w >> 4) & 0x0F0F0F0Fu) + 0x79797979u) ^ 0x80808080u;
  return (long)(((uint64_t)hi << 32) | (uint64_t)lo);
}

__device__ __forceinline__ float h2f(uint32_t bits16) {
  return __half2float(__ushort_as_half((unsigned short)bits16));
}

template <int D, int MT, int NT>
struct GroupOps {
  long a[MT][D];
  uint32_t w[NT];
  uint32_t s[NT];
  float as[MT][4];
};

template <int D, int MT, int NT>
__device__ __forceinline__ void load_group(const GemvArgs &p, int g, int m0, int nb0, int KQ,
                                           int NB, int n_local, int c, GroupOps<D, MT, NT> &o) {
  const int M = p.M;
  const uint32_t *codes = (const uint32_t *)p.codes;
  const uint16_t *scales = (const uint16_t *)p.scales;
  const int kq = g >> 2, j = g & 3;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int nb = nb0 + nt;
    if (nb < NB) {
      const size_t lane_slot = ((size_t)nb * KQ + kq) * 64 + 16 * j + n_local;
      o.w[nt] = codes[lane_slot * 4 + c];
      o.s[nt] = scales[lane_slot];
    } else {
      o.w[nt] = 0x77777777u;  // code 7 decodes to 0
      o.s[nt] = 0;
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = m0 + 16 * mt + n_local;
#pragma unroll
    for (int d = 0; d < D; ++d)
      o.a[mt][d] = m < M ? *(const long *)(p.act_q + (((size_t)g * D + d) * M + m) * 32 + 8 * c)
                         : 0l;
    const int mr = m0 + 16 * mt + 4 * c;
#pragma unroll
    for (int r = 0; r < 4; ++r) o.as[mt][r] = mr + r < M ? p.act_meta[(size_t)g * M + mr + r].scale : 0.0f;
  }
}

template <int D, int MT, int NT>
__global__ __launch_bounds__(256) void gemm_kernel(GemvArgs p, int m_tiles) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n_local = lane & 15, c = lane >> 4;
  const int NB = p.N >> 4, KQ = p.K >> 7, G = p.K >> 5;
  // XCD-aware block order: XCD x runs logical blocks [first_x, first_x + cnt_x)
  const int nblk = gridDim.x, b = blockIdx.x;
  const int xcd = b & 7, idx = b >> 3;
  const int logical = xcd * (nblk >> 3) + min(xcd, nblk & 7) + idx;
  const int n_tile = logical / m_tiles, m_tile = logical % m_tiles;
  const int m0 = m_tile * (32 * MT) + (wave & 1) * (16 * MT);
  const int nb0 = n_tile * (2 * NT) + (wave >> 1) * NT;
  if (m0 >= p.M || nb0 >= NB) return;

  float acc[MT][NT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[mt][nt][r] = 0.0f;

  GroupOps<D, MT, NT> cur, nxt;
  load_group<D, MT, NT>(p, 0, m0, nb0, KQ, NB, n_local, c, cur);
  const v4i magic = {kMagic, kMagic, kMagic, kMagic};
  const v4i zero = {0, 0, 0, 0};
  for (int g = 0; g < G; ++g) {
    if (g + 1 < G) load_group<D, MT, NT>(p, g + 1, m0, nb0, KQ, NB, n_local, c, nxt);
    long bs[NT];
    float ws[NT], wc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      bs[nt] = signed_codes(cur.w[nt]);
      ws[nt] = h2f(cur.s[nt]);
      wc[nt] = -kMagicF * ws[nt];
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        if constexpr (D == 1) {
          const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(cur.a[mt][0], bs[nt], magic, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float t = fmaf(__int_as_float(d[r]), ws[nt], wc[nt]);
            acc[mt][nt][r] = fmaf(t, cur.as[mt][r], acc[mt][nt][r]);
          }
        } else {
          v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(cur.a[mt][0], bs[nt], zero, 0, 0, 0);
#pragma unroll
          for (int dd = 1; dd < D; ++dd) {
#pragma unroll
            for (int r = 0; r < 4; ++r) d[r] = d[r] << 7;
            d = __builtin_amdgcn_mfma_i32_16x16x32_i8(cur.a[mt][dd], bs[nt], d, 0, 0, 0);
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float t = (float)d[r] * ws[nt];
            acc[mt][nt][r] = fmaf(t, cur.as[mt][r], acc[mt][nt][r]);
          }
        }
      }
    cur = nxt;
  }

  const bool paired = p.epi == EPI_SWIGLU || p.epi == EPI_QKV;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float tot = acc[mt][nt][r];
        const float partner = paired ? __shfl_xor(tot, 8) : 0.0f;
        const int m = m0 + 16 * mt + 4 * c + r;
        const int nb = nb0 + nt;
        if (m < p.M && nb < NB)
          store_output(p, p.epi, nb, n_local, m, tot, partner, epi_load(p, p.epi, nb, n_local, m));
      }
}

}  // namespace

GemmShape plan_gemm(int N, int M) {
  GemmShape s;
  const int NB = N / 16;
  // 128 x 64 block tiles while that still gives two workgroups per CU, else
  // 64 x 64
  const long big = (long)((M + 127) / 128) * ((NB + 3) / 4);
  if (big >= 512) {
    s.mt = 4;
    s.nt = 2;
  } else {
    s.mt = 2;
    s.nt = 2;
  }
  s.m_tiles = (M + 32 * s.mt - 1) / (32 * s.mt);
  s.n_tiles = (NB + 2 * s.nt - 1) / (2 * s.nt);
  s.grid = s.m_tiles * s.n_tiles;
  return s;
}

hipError_t launch_gemm(const GemvArgs &a, hipStream_t st) {
  if (a.N % 16 || a.K % 128 || a.M < 1 || !a.act_q || !a.act_meta || (a.D != 1 && a.D != 3))
    return hipErrorInvalidValue;
  const GemmShape s = plan_gemm(a.N, a.M);
  const dim3 grid(s.grid), block(256);
#define GK_GEMM(DD, MM, NN) \
  hipLaunchKernelGGL((gemm_kernel<DD, MM, NN>), grid, block, 0, st, a, s.m_tiles)
  if (a.D == 1) {
    if (s.mt == 4) GK_GEMM(1, 4, 2); else GK_GEMM(1, 2, 2);
  } else {
    if (s.mt == 4) GK_GEMM(3, 4, 2); else GK_GEMM(3, 2, 2);
  }
#undef GK_GEMM
  return hipGetLastError();
}

}  // namespace gk
