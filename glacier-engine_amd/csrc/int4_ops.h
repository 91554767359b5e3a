// int4_ops.h — register-level helpers shared by the INT4 GEMV (K1) and the
// prefill GEMM (K2): code unpacking, the magic-constant scale trick and the
// cross-lane moves that turn one coalesced 16-byte load per lane into MFMA
// operands.
//
// Device tile layout (see kernels.h): lane l = 16 j + n of a quad holds the 32
// codes of group j of weight row n as four u32 words; word w holds codes
// 8w .. 8w + 3 in its low nibbles and 8w + 4 .. 8w + 7 in its high nibbles.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gk {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));

// bits of 12582912.0f = 1.5 * 2^23: for |T| < 2^22 the integer 0x4B400000 + T
// read as f32 is exactly 12582912 + T, so fma(that, ws, -12582912 * ws) is
// RN(T * ws) in one instruction (-12582912 * ws is exact for an fp16 ws).
static constexpr int kMagic = 0x4B400000;
static constexpr float kMagicF = 12582912.0f;

// Streaming 16-byte load of weight codes (read once per token).
static __device__ __forceinline__ uint4 load_stream(const uint4 *p) {
  const v4u v = __builtin_nontemporal_load((const v4u *)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

static __device__ __forceinline__ float h2f(uint32_t bits16) {
  return __half2float(__ushort_as_half((unsigned short)bits16));
}

// Eight 4-bit codes of one u32 word -> eight signed int8 lanes (u - 7),
// k0..k7. Per byte u + 0x79 stays below 0x100 and flipping bit 7 of
// (u + 121) gives u - 7 in two's complement, so an integer dot with these
// lanes is the group dot of the dequantised codes itself (no correction).
static __device__ __forceinline__ long signed_codes(uint32_t w) {
  const uint32_t lo = ((w & 0x0F0F0F0Fu) + 0x79797979u) ^ 0x80808080u;
  const uint32_t hi = (((w >> 4) & 0x0F0F0F0Fu) + 0x79797979u) ^ 0x80808080u;
  return (long)(((uint64_t)hi << 32) | (uint64_t)lo);
}

// Even lanes: (own u16) | (u16 of the next lane) << 16; DPP quad_perm
// [1, 0, 3, 2] reads the neighbour's value without a trip through LDS.
static __device__ __forceinline__ uint32_t scale_pair(uint32_t s) {
  const uint32_t nb = (uint32_t)__builtin_amdgcn_mov_dpp((int)s, 0xB1, 0xF, 0xF, false);
  return (s & 0xFFFFu) | (nb << 16);
}

// 4 x 4 transpose of u32 words across the four 16-lane rows of a wave: on
// entry lane (c, n) = 16c + n holds words 0..3 of its tile slot (group c of
// weight row n); on return it holds word c of groups 0..3 of row n, which is
// the operand layout of v_mfma_i32_16x16x32_i8 for each of the four groups
// (lane (c, n) = codes 8c .. 8c + 7 of row n). The 32-lane swap exchanges the
// upper rows of one register with the lower rows of the other, the 16-lane
// swap the odd rows of one with the even rows of the other.
static __device__ __forceinline__ uint4 quad_transpose(uint4 v) {
  const v2u a = __builtin_amdgcn_permlane32_swap(v.x, v.z, false, false);
  const v2u b = __builtin_amdgcn_permlane32_swap(v.y, v.w, false, false);
  const v2u c = __builtin_amdgcn_permlane16_swap(a.x, b.x, false, false);
  const v2u d = __builtin_amdgcn_permlane16_swap(a.y, b.y, false, false);
  return make_uint4(c.x, c.y, d.x, d.y);
}

// All four 16-lane rows' values of this lane's column: on return out[j] is
// x of lane 16 j + (lane & 15). The 32-lane swap of x with itself leaves
// rows (0, 1, 0, 1) in one result and (2, 3, 2, 3) in the other; a 16-lane
// swap of each with itself splits those into single rows.
static __device__ __forceinline__ void column_gather(uint32_t x, uint32_t out[4]) {
  const v2u a = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  const v2u b = __builtin_amdgcn_permlane16_swap(a.x, a.x, false, false);
  const v2u c = __builtin_amdgcn_permlane16_swap(a.y, a.y, false, false);
  out[0] = b.x;
  out[1] = b.y;
  out[2] = c.x;
  out[3] = c.y;
}

// v combined with the value of lane ^ 16 (rows 0/1 and 2/3 of the wave) or
// lane ^ 32 (the two halves), through the permlane swaps instead of LDS
// permutes. A swap of v with itself leaves the pair's two values in r.x and
// r.y of both lanes, so the commutative result is bit-identical to
// v + shuffle_xor(v, 16 or 32).
static __device__ __forceinline__ float xor16_add(float v) {
  const v2u r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r.x) + __uint_as_float(r.y);
}
static __device__ __forceinline__ float xor32_add(float v) {
  const v2u r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r.x) + __uint_as_float(r.y);
}
static __device__ __forceinline__ float xor16_max(float v) {
  const v2u r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r.x), __uint_as_float(r.y));
}
static __device__ __forceinline__ float xor32_max(float v) {
  const v2u r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r.x), __uint_as_float(r.y));
}

// DPP lane exchanges inside a 16-lane row (no LDS round trip): the value of
// lane ^ 8 (a rotation by 8 within the row), and of lane ^ 1 / lane ^ 2
// (quad permutations [1, 0, 3, 2] / [2, 3, 0, 1]).
static __device__ __forceinline__ float row_xor8(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, false));
}
static __device__ __forceinline__ float quad_xor1(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
}
static __device__ __forceinline__ float quad_xor2(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));
}
static __device__ __forceinline__ int quad_xor1(int v) { return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false); }
static __device__ __forceinline__ int quad_xor2(int v) { return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false); }
// Sum over the 16 lanes of each row by rotations 8, 4, 2, 1: every lane
// gets the row's sum, each in its own (fixed) association order, so a
// caller that needs one deterministic value reads it from one lane.
static __device__ __forceinline__ float row16_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x124, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x122, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x121, 0xF, 0xF, false));
  return v;
}
// Maximum over the whole wave (exact: every lane gets it).
static __device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x124, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x122, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x121, 0xF, 0xF, false)));
  return xor32_max(xor16_max(v));
}
// Sum over the whole wave (lane 0's value is the deterministic one).
static __device__ __forceinline__ float wave_sum(float v) { return xor32_add(xor16_add(row16_sum(v))); }

// Reductions over each 32-lane half of a wave (every lane of the half gets
// the result): DPP row rotations by 8, 4, 2, 1 combine the 16 lanes of a row,
// then a 16-lane swap of the value with itself puts the even row's and the
// odd row's results side by side in every lane (rows 0/1 and 2/3 pair up,
// which are exactly the two halves). Max and integer sums are exact in any
// order, so the results equal a butterfly's.
static __device__ __forceinline__ float half_wave_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x124, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x122, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x121, 0xF, 0xF, false)));
  const v2u r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r.x), __uint_as_float(r.y));
}
static __device__ __forceinline__ int half_wave_sum(int v) {
  v += __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, false);
  v += __builtin_amdgcn_mov_dpp(v, 0x124, 0xF, 0xF, false);
  v += __builtin_amdgcn_mov_dpp(v, 0x122, 0xF, 0xF, false);
  v += __builtin_amdgcn_mov_dpp(v, 0x121, 0xF, 0xF, false);
  const v2u r = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
  return (int)(r.x + r.y);
}

}  // namespace gk
