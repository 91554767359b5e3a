// kernels.hip — hand-written gfx950 kernels for Glacier's text token loop.
//
//  K1  gemv_kernel     INT4 x (Q8 | f32-as-3-digit) GEMV for one or two rows
//                      (v_dot4_i32_i8; more rows run the GEMM, gemm.hip);
//                      split-K reduced inside the workgroup through LDS;
//                      fused epilogues (residual, SwiGLU, RoPE + paged KV
//                      write, greedy candidates).
//  K4  prep_act_kernel RMSNorm (kernels.zig:141-220) fused with the activation
//                      quantiser (int4_matmul.zig:380-398).
//  K3  attn_*          paged-KV GQA decode attention (split over context chunks).
//  K5  argmax_*        wavefront masked argmax (sampling.zig:55-105, :194-206).
//
// Compiled with -ffp-contract=off so that the element-wise f32 arithmetic
// rounds where the reference rounds; explicit fmaf() marks the places where a
// fused multiply-add is intended.
#include "kernels.h"
#include "epilogue.h"
#include "int4_ops.h"

#include <hip/hip_fp16.h>
#include <math.h>

#include <algorithm>
#include <type_traits>

namespace gk {


// ---------------------------------------------------------------------------
// K4: activation planes (+ optional RMSNorm)
// ---------------------------------------------------------------------------
static __device__ __forceinline__ float load_x(const void *x, int bf16, size_t i) {
  if (bf16) {
    uint32_t b = ((const uint16_t *)x)[i];
    return __uint_as_float(b << 16);
  }
  return ((const float *)x)[i];
}

// Quantises one 32-value group (one value per lane of a half-wave) into
// the planes pd describes, when it is set.
static __device__ __forceinline__ void emit_group(const PlanesDst &pd, float v, int hl, int g,
                                                  int m, int M) {
  if (!pd.q) return;
  if (pd.D == 1) quantize_group<1>(v, hl, g, m, M, pd.q, pd.meta);
  else quantize_group<3>(v, hl, g, m, M, pd.q, pd.meta);
}

// grid = (ceil(G / 8), M): each block converts 8 groups of one row; with a
// norm weight every block first reduces the row's full sum of squares.
template <int D>
__global__ __launch_bounds__(256) void prep_act_kernel(const void *x, int x_bf16,
                                                       const float *norm_w, float eps, int M,
                                                       int K, int8_t *act_q, ActMeta *meta,
                                                       float *normed_out) {
  const int m = blockIdx.y;
  const int t = threadIdx.x;
  const size_t row = (size_t)m * K;
  __shared__ float red[8];
  float inv = 1.0f;
  if (norm_w) {
    float ss = 0.0f;
    if (!x_bf16 && (K & 3) == 0) {
      // every load of a pass is issued before the first is used: one memory
      // round trip per 8192 elements instead of one per 256
      constexpr int U = 8;
      const float4 *x4 = (const float4 *)((const float *)x + row);
      const int K4 = K >> 2;
      for (int base = 0; base < K4; base += 256 * U) {
        float4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int i = base + t + 256 * u;
          v[u] = i < K4 ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
          ss = fmaf(v[u].w, v[u].w, fmaf(v[u].z, v[u].z, fmaf(v[u].y, v[u].y, fmaf(v[u].x, v[u].x, ss))));
      }
    } else {
      for (int i = t; i < K; i += 256) {
        float v = load_x(x, x_bf16, row + i);
        ss = fmaf(v, v, ss);
      }
    }
    ss = wave_sum(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    if (t == 0) {
      float s = red[0] + red[1] + red[2] + red[3];
      float rms = sqrtf(s / (float)K + eps);
      red[4] = 1.0f / rms;
    }
    __syncthreads();
    inv = red[4];
  }
  // One 32-lane half-wave per 32-element group.
  const int half = t >> 5, hl = t & 31;
  const int G = K >> 5;
  {
    const int g = blockIdx.x * 8 + half;
    if (g >= G) return;
    const int k = (g << 5) + hl;
    float v = load_x(x, x_bf16, row + k);
    if (norm_w) {
      float tt = v * inv;
      v = tt * norm_w[k];
    }
    if (normed_out) normed_out[row + k] = v;
    quantize_group<D>(v, hl, g, m, M, act_q, meta);
  }
}

hipError_t launch_prep_act(const void *x, int x_bf16, const float *norm_w, float eps, int M,
                           int K, int D, int8_t *act_q, ActMeta *meta, float *normed_out,
                           hipStream_t st) {
  const dim3 grid((K / 32 + 7) / 8, M);
  if (D == 1)
    hipLaunchKernelGGL(prep_act_kernel<1>, grid, dim3(256), 0, st, x, x_bf16, norm_w, eps, M,
                       K, act_q, meta, normed_out);
  else
    hipLaunchKernelGGL(prep_act_kernel<3>, grid, dim3(256), 0, st, x, x_bf16, norm_w, eps, M,
                       K, act_q, meta, normed_out);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// K1: INT4 GEMV
// ---------------------------------------------------------------------------
// Tile = 16 rows x 128 columns (4 groups of 32): 1 KB of codes as 64 lanes x
// 16 B, lane (j, n) = 16 * j + n holding group j of row n, plus 64 fp16
// scales in the same lane order. A workgroup of W = RB * KS waves owns RB
// row blocks; the KS waves of a row block split its K range and reduce their
// partial sums through LDS in a fixed order (deterministic, no workgroup ever
// waits on another). Activation planes are staged in LDS when they fit.
//
// Every lane dots its whole group with v_dot4_i32_i8 (exact integer per
// group) and applies the group's f32 scales itself; the four lanes of a row
// are summed once at the end. 4 quads per wave are in flight (8 measured
// slower on every 7B shape).
// Activation planes are staged in LDS when they fit in 144 KB of the 160 KB
// a gfx950 workgroup may use (the rest holds the epilogue buffers; launches
// above 64 KB raise the kernel's dynamic-LDS limit first).
static constexpr size_t kLdsLimit = 144 * 1024;
static constexpr int kMaxSsParts = 256;  // deferred-RMSNorm partial sums per row

static size_t planes_bytes(int groups, int M, int D) {
  return (size_t)groups * ((size_t)D * M * 32 + (size_t)M * sizeof(ActMeta));
}

// Launch shape of the GEMV. From cold-cache sweeps at M = 1, 2 with
// one- and three-digit planes on the 7B and C2 shapes:
//  * K split until the grid holds about 4096 waves, keeping >= 4 quads per
//    wave, at most 8 split waves (the 3-digit down projection, 224 row
//    blocks, measured best there), 4 quads in flight per wave;
//  * 512-4095 row blocks: workgroups of 4 waves (11008x4096: 7.8 us
//    against 9.6 with 6 waves; 18944x3584: 9.4 against 11.1; the fused
//    gate/up: 15.1 against 16.3 with 8);
//  * 257-511 row blocks: 4 split waves x 2 row blocks, so the grid stays
//    within one workgroup per CU (4608x3584: 5.7 us against 6.5 with 288
//    workgroups of 7 waves);
//  * otherwise workgroups of about 8 waves.
static void plan_rows2(int NB, int KQ, int &ks, int &rb) {
  ks = std::max(1, std::min(std::min(8, std::max(1, KQ / 4)), (4096 + NB - 1) / NB));
  rb = std::max(1, std::min(8, 8 / ks));
  if (NB >= 512 && NB < 4096) {
    ks = std::min(ks, 4);
    rb = std::max(1, 4 / ks);
  } else if (NB > 256 && NB < 512 && KQ >= 16) {
    ks = 4;
    rb = 2;
  }
}

GemvShape plan_gemv(int N, int K, int M, int D) {
  GemvShape p;
  const int NB = N / 16, KQ = K / 128;
  int ks, rb;
  plan_rows2(NB, KQ, ks, rb);
  p.unroll = 4;
  p.ksplit = ks;
  p.rb = rb;
  p.waves = ks * rb;
  const size_t red = (size_t)p.waves * 4 * 64 * sizeof(float);
  const size_t planes = planes_bytes(K / 32, M, D) + (size_t)M * sizeof(float);
  p.lds_a = planes <= kLdsLimit;
  p.lds_bytes = std::max(p.lds_a ? planes : 0, red);
  p.grid = (NB + rb - 1) / rb;
  return p;
}

// EPI >= 0: the epilogue type as a compile-time constant (so a launch only
// carries its own epilogue's loads and branches); EPI < 0: a.epi at run time.
// XIN: input mode (planes built in LDS from a.x_in, deferred RMSNorm).
template <int D, bool LDS_A, int LB, int EPI, bool XIN>
__global__ __launch_bounds__(LB) void gemv_kernel(GemvArgs a) {
  // one or two activation rows, each lane dotting its own group (dot4), U
  // quads of weights in flight per wave
  constexpr int MT = 1, U = 4, MR = 2;
  constexpr bool DOT4 = true;
  const int epi = EPI >= 0 ? EPI : a.epi;
  extern __shared__ __align__(16) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  // (wave-uniform by construction; readfirstlane tells the compiler, so the
  // weight loop's bounds and branches are scalar and a load under a branch
  // needs no merge that waits for its data)
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int KS = a.ksplit;
  const int NB = a.N >> 4, KQ = a.K >> 7, G = a.K >> 5;
  const int M = a.M;
  const int ks = wave % KS;
  const int nb = blockIdx.x * (int)(blockDim.x >> 6) / KS + wave / KS;
  const int kq0 = (ks * KQ) / KS, kq1 = ((ks + 1) * KQ) / KS;
  // Prehead eligibility (int4_executor.zig:968-1150 skips empty rows4 tiles):
  // a row block none of whose 16 rows is eligible for any activation row
  // streams no weights; its accumulators stay 0 and no row of it becomes a
  // candidate.
  // (compiled only into the head's variants: a plain or run-time epilogue)
  bool skip_block = false;
  if ((EPI == EPI_PLAIN || EPI < 0) && a.prehead) {
    const int nbq = min(nb, NB - 1);
    uint32_t any = 0;
    for (int m = 0; m < M; ++m)
      any |= (uint32_t)(a.arg_words[(size_t)m * a.arg_word_count + (nbq >> 2)] >> ((nbq & 3) * 16)) &
             0xFFFFu;
    skip_block = any == 0;
  }
  const int nq = skip_block ? 0 : kq1 - kq0;
  const int n_local = lane & 15, c = lane >> 4;

  // Request order: the activation staging first (L2-resident, consumed
  // first), then the first U quads of weights, then the first level of the
  // epilogue inputs. Loads complete in issue order, so staging issued after
  // the weights would wait out the weights' HBM latency before the next
  // quads could be requested.
  const size_t tile0 = (size_t)min(nb, NB - 1) * KQ + kq0;
  // (every lane loads its own 16-byte tile slot; a skipped row block reads
  // the first tile, which stays cached, so no branch changes the number of
  // loads in flight)
  const size_t tq = nq > 0 ? tile0 : 0;
  const uint4 *cp = a.codes + tq * 64 + lane;
  // (the scales too: one u16 per lane in its slot's order, read as the dword
  // that holds the lane's pair; a 16-bit load's register is merged with
  // others, and the merge waits for the data, serialising the loads)
  const uint32_t *spp = (const uint32_t *)a.scales + tq * 32 + (lane >> 1);
  const int shalf = (lane & 1) * 16;
  // Epilogue inputs of the (at most two) rows of a dot4 launch: the first
  // level with the weights in flight; the second level (page slot, RoPE
  // factors) after the staging barrier, under the weight stream.
  // (every lane loads, with the row block clamped into range, so no branch
  // splits the wave and the loads issue back to back)
  EpiIn epre[2];
  const int nb_c = min(nb, NB - 1);
  // Two register buffers of U quads alternate: the quads of one are dotted
  // while the next U quads stream into the other, so a wave always has a
  // buffer's loads in flight (refilling a single buffer drains it to zero
  // first); both are requested before the staging wait.
  // (a refill loads all U slots, a slot past the wave's last quad from the
  // last quad again, computed and not added: loads under a per-slot branch
  // leave the compiler a path with fewer loads in flight, and its waits are
  // then counted for that path)
  uint4 wb[U], wd[U];
  uint32_t sb[U], sd[U];
  // (scheduling barriers keep a refill after the dot of the buffer it
  // overwrites: hoisted above it, the refill needs fresh registers and a
  // wait for the data in flight)
  auto fetch = [&](uint4(&w)[U], uint32_t(&sv)[U], int qb) {
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int uq = max(min(qb + u, nq - 1), 0);
      w[u] = load_stream(cp + (size_t)uq * 64);
      sv[u] = spp[(size_t)uq * 32];
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto prefetch0 = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    fetch(wb, sb, 0);
    fetch(wd, sd, U);
    if constexpr (DOT4 && MR == 2) {
#pragma unroll
      for (int m = 0; m < 2; ++m)
        if (ks == 0 && m < M) epi_load1(epre[m], a, epi, nb_c, n_local, m);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  const int nthr = (int)blockDim.x;
  const size_t qbytes = (size_t)G * D * M * 32;
  const size_t mbytes = (size_t)G * M * sizeof(ActMeta);
  __shared__ float sinv[32];
  if constexpr (XIN) {
    static_assert(LDS_A, "input mode builds the planes in LDS");
    constexpr int XU = 2, PU = kMaxSsParts / 64;
    const int nwv = (int)(blockDim.x >> 6);
    float ssv[PU];
    // (loads are clamped into range rather than branched around, so they
    // all issue back to back)
    if (a.in_ss && wave < M) {
      const float *src = a.in_ss + (size_t)wave * a.in_ss_count;
#pragma unroll
      for (int u = 0; u < PU; ++u) ssv[u] = src[min(lane + 64 * u, a.in_ss_count - 1)];
    }
    // 8 consecutive elements of x (and of the norm weight) per thread, so
    // the 4 threads of a 32-element group quantise it together
    const int nchunk = M * (a.K >> 3);
    float4 xr[XU][2], wr[XU][2];
#pragma unroll
    for (int u = 0; u < XU; ++u)
#pragma unroll
      for (int h = 0; h < 2; ++h) xr[u][h] = wr[u][h] = make_float4(1.f, 1.f, 1.f, 1.f);
    auto load_chunks = [&](int base) {
#pragma unroll
      for (int u = 0; u < XU; ++u) {
        const int c8 = min(base + (int)threadIdx.x + nthr * u, nchunk - 1);
        const float4 *xp = (const float4 *)(a.x_in + (size_t)c8 * 8);
        xr[u][0] = xp[0];
        xr[u][1] = xp[1];
        if (a.norm_w) {
          const float4 *wp = (const float4 *)(a.norm_w + (size_t)(c8 * 8) % a.K);
          wr[u][0] = wp[0];
          wr[u][1] = wp[1];
        }
      }
    };
    load_chunks(0);
    prefetch0();
    // 1/rms of each input row from the producer's partial sums of squares
    // (wave w reduces rows w, w + waves, ...; fixed order)
    if (a.in_ss) {
      for (int m = wave; m < M; m += nwv) {
        if (m != wave) {
          const float *src = a.in_ss + (size_t)m * a.in_ss_count;
#pragma unroll
          for (int u = 0; u < PU; ++u) ssv[u] = src[min(lane + 64 * u, a.in_ss_count - 1)];
        }
        float ss = 0.0f;
#pragma unroll
        for (int u = 0; u < PU; ++u) ss += lane + 64 * u < a.in_ss_count ? ssv[u] : 0.0f;
        ss = wave_sum(ss);
        if (lane == 0) sinv[m] = 1.0f / sqrtf(ss / (float)a.K + a.in_eps);
      }
    }
    // Group quantiser (int4_matmul.zig:380-398) of x * norm_w: the RMSNorm
    // factor is a per-row scalar that cancels in q = round(v * 127 / max|v|),
    // so it is applied to the outputs instead (sinv).
    for (int base = 0; base < nchunk; base += nthr * XU) {
      if (base > 0) load_chunks(base);
#pragma unroll
      for (int u = 0; u < XU; ++u) {
        const int c8 = base + (int)threadIdx.x + nthr * u;
        const bool valid = c8 < nchunk;  // uniform over the 4 threads of a group
        float v[8] = {xr[u][0].x, xr[u][0].y, xr[u][0].z, xr[u][0].w,
                      xr[u][1].x, xr[u][1].y, xr[u][1].z, xr[u][1].w};
        if (a.norm_w) {
          const float w8[8] = {wr[u][0].x, wr[u][0].y, wr[u][0].z, wr[u][0].w,
                               wr[u][1].x, wr[u][1].y, wr[u][1].z, wr[u][1].w};
#pragma unroll
          for (int i = 0; i < 8; ++i) v[i] = v[i] * w8[i];
        }
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
        amax = fmaxf(amax, quad_xor1(amax));
        amax = fmaxf(amax, quad_xor2(amax));
        const float scale = amax / 127.0f;
        const float inv_s = scale == 0.0f ? 0.0f : 1.0f / scale;
        uint64_t packed[D];
#pragma unroll
        for (int d = 0; d < D; ++d) packed[d] = 0;
        int csum = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float y = v[i] * inv_s;
          float q0f = roundf(y);
          q0f = fminf(fmaxf(q0f, -127.0f), 127.0f);
          int qd[3] = {(int)q0f, 0, 0};
          if (D == 3) {
            const float r1 = (y - q0f) * 128.0f;
            const float q1f = roundf(r1);
            const float r2 = (r1 - q1f) * 128.0f;
            qd[1] = (int)q1f;
            qd[2] = (int)roundf(r2);
          }
          int comb = 0;
#pragma unroll
          for (int d = 0; d < D; ++d) {
            packed[d] |= (uint64_t)(uint8_t)(int8_t)qd[d] << (8 * i);
            comb = comb * 128 + qd[d];
          }
          csum += comb;
        }
        csum += quad_xor1(csum);
        csum += quad_xor2(csum);
        if (valid) {
          const int e = c8 * 8, m = e / a.K, g = (e % a.K) >> 5, part = (e >> 3) & 3;
#pragma unroll
          for (int d = 0; d < D; ++d)
            *(uint64_t *)(smem + (((size_t)g * D + d) * M + m) * 32 + part * 8) = packed[d];
          if (part == 0) {
            ActMeta mm;
            mm.scale = D == 3 ? scale * (1.0f / 16384.0f) : scale;
            mm.corr = 7 * csum;
            ((ActMeta *)(smem + qbytes))[(size_t)g * M + m] = mm;
          }
        }
      }
    }
    __syncthreads();
  } else if (LDS_A) {
    // copy the producer's planes and meta into LDS: the first pass (all of
    // it at one or two rows up to K = 32768 with 512 threads) requests its
    // loads before the weights and stores after them
    constexpr int SP = 8, SM = 2;
    const int n16 = (int)(qbytes / 16), n8 = (int)(mbytes / 8);
    const uint4 *src = (const uint4 *)a.act_q;
    uint4 *dst = (uint4 *)smem;
    const uint2 *msrc = (const uint2 *)a.act_meta;
    uint2 *mdst = (uint2 *)(smem + qbytes);
    const int t = (int)threadIdx.x;
    // (named registers: an array of them is kept in scratch memory)
#define GK_LDQ(i) const uint4 v##i = src[min(t + i * nthr, n16 - 1)]
    GK_LDQ(0); GK_LDQ(1); GK_LDQ(2); GK_LDQ(3); GK_LDQ(4); GK_LDQ(5); GK_LDQ(6); GK_LDQ(7);
#undef GK_LDQ
    const uint2 m0 = msrc[min(t, n8 - 1)];
    const uint2 m1 = msrc[min(t + nthr, n8 - 1)];
    prefetch0();
#define GK_STQ(i) \
  if (t + i * nthr < n16) dst[t + i * nthr] = v##i
    GK_STQ(0); GK_STQ(1); GK_STQ(2); GK_STQ(3); GK_STQ(4); GK_STQ(5); GK_STQ(6); GK_STQ(7);
#undef GK_STQ
    if (t < n8) mdst[t] = m0;
    if (t + nthr < n8) mdst[t + nthr] = m1;
    for (int i = t + SP * nthr; i < n16; i += nthr) dst[i] = src[i];
    for (int i = t + SM * nthr; i < n8; i += nthr) mdst[i] = msrc[i];
    __syncthreads();
  } else {
    prefetch0();
  }
  if constexpr (DOT4 && MR == 2) {
#pragma unroll
    for (int m = 0; m < 2; ++m)
      if (ks == 0 && m < M) epi_load2(epre[m], a, epi, nb_c, n_local);
  }
  const int8_t *aq = LDS_A ? (const int8_t *)smem : a.act_q;
  const ActMeta *am = LDS_A ? (const ActMeta *)(smem + qbytes) : a.act_meta;

  float acc[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[mt][r] = 0.0f;

  if (nb < NB && nq > 0) {
    auto dot = [&](const uint4(&w)[U], const uint32_t(&sv)[U], int qb) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool live = qb + u < nq;
        // lane (j = c, n): all 32 codes of group g of row n (a slot past the
        // end reads the last quad's planes: finite, and not added)
        const int g = (kq0 + min(qb + u, nq - 1)) * 4 + c;
        const uint32_t wj[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
        const float ws = h2f((uint16_t)(sv[u] >> shalf));
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          if (m > 0 && m >= M) break;
          int T = 0;
#pragma unroll
          for (int d = 0; d < D; ++d) {
            const int4 q0 = *(const int4 *)(aq + (((size_t)g * D + d) * M + m) * 32);
            const int4 q1 = *(const int4 *)(aq + (((size_t)g * D + d) * M + m) * 32 + 16);
            const int qa[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
            int t = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              t = __builtin_amdgcn_sdot4((int)(wj[i] & 0x0F0F0F0Fu), qa[2 * i], t, false);
              t = __builtin_amdgcn_sdot4((int)((wj[i] >> 4) & 0x0F0F0F0Fu), qa[2 * i + 1], t, false);
            }
            T = T * 128 + t;
          }
          const ActMeta mm = am[(size_t)g * M + m];
          const float v = (float)(T - mm.corr);
          float tt = v * ws;
          tt = tt * mm.scale;
          acc[0][m] = live ? acc[0][m] + tt : acc[0][m];
        }
      }
    };
    // Buffers i (wb) and i + 1 (wd) are in flight at the top of each
    // iteration. (a straight-line body with one exit: the compiler counts its
    // waits along this one path, each dot waiting for its own buffer only)
    const int nbuf = (nq + U - 1) / U;
    int i = 0;
    for (; i + 4 <= nbuf; i += 2) {
      dot(wb, sb, i * U);
      fetch(wb, sb, (i + 2) * U);
      dot(wd, sd, (i + 1) * U);
      fetch(wd, sd, (i + 3) * U);
    }
    const int rest = nbuf - i;  // 1..3
    dot(wb, sb, i * U);
    if (rest == 3) {
      fetch(wb, sb, (i + 2) * U);
      dot(wd, sd, (i + 1) * U);
      dot(wb, sb, (i + 2) * U);
    } else if (rest == 2) {
      dot(wd, sd, (i + 1) * U);
    }
  }

  {
    // acc[0][m] of lane (j, n) sums the groups j, j + 4, ... of row n; add
    // the four lanes of the row so lanes j = 0 hold m = 0.. M-1 as (c=0, r=m)
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      float v = acc[0][m];
      v = xor32_add(xor16_add(v));
      acc[0][m] = v;
    }
  }

  // ---- split-K reduction through LDS, fixed order over ks ----
  // (no early return: the SwiGLU plane epilogue below synchronises the
  // whole workgroup again)
  const bool lead = ks == 0 && nb < NB;
  if (KS > 1) {
    if (LDS_A) __syncthreads();  // the planes region is reused below
    float *red = (float *)smem;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[((wave * MT + mt) * 4 + r) * 64 + lane] = acc[mt][r];
    __syncthreads();
    if (ks == 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float tot = acc[mt][r];
          for (int s2 = 1; s2 < KS; ++s2) tot += red[(((wave + s2) * MT + mt) * 4 + r) * 64 + lane];
          acc[mt][r] = tot;
        }
    }
  }

  if (XIN && a.in_ss) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = mt * 16 + c * 4 + r;
        if (m < M) acc[mt][r] *= sinv[m];
      }
  }

  // ---- fused epilogues: lane (c, n) owns rows m = 16 mt + 4 c + r of column n ----
  const bool paired = epi == EPI_SWIGLU || epi == EPI_QKV;
  const bool emit_planes = epi == EPI_SWIGLU && a.out_q;
  const bool resid_ss = epi == EPI_RESID && a.ss_out;
  // SwiGLU outputs of this workgroup's rb row blocks: [M][8 * rb] floats
  // after the reduction area; residual sums of squares: [waves][M]
  const int RB = (int)(blockDim.x >> 6) / KS;
  float *actbuf = (float *)(smem + a.ksplit_lds_off);
  float *sspart = (float *)(smem + a.ksplit_lds_off);
  const int nb_wg0 = blockIdx.x * RB;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = mt * 16 + c * 4 + r;
      const float tot = acc[mt][r];
      // partner row (n_local ^ 8) lives in lane ^ 8 with the same (c, r)
      const float partner = paired ? row_xor8(tot) : 0.0f;
      if (resid_ss) {
        // residual output y = resid + tot, and this wave's sum of y^2 of row m
        float y = 0.0f;
        if (lead && m < M) {
          const EpiIn e = (DOT4 && MR == 2) ? epre[m & 1] : epi_load(a, epi, nb, n_local, m);
          y = e.resid + tot;
          a.y[(size_t)m * a.N + nb * 16 + n_local] = y;
        }
        // the row of 16 lanes (c, n), n = 0..15, summed; lane n = 0 stores
        const float sq = row16_sum(y * y);
        if (n_local == 0 && m < M) sspart[wave * M + m] = sq;
        continue;
      }
      if (!lead || m >= M) continue;
      if (emit_planes) {
        if (n_local < 8) {
          const float v = silu_mul(tot, partner);
          actbuf[m * (8 * RB) + (nb - nb_wg0) * 8 + n_local] = v;
          if (a.y) a.y[(size_t)m * (a.N / 2) + nb * 8 + n_local] = v;
        }
      } else if (epi != EPI_PLAIN || a.y) {  // (a fused head may store no logits)
        store_output(a, epi, nb, n_local, m, tot, partner,
                     (DOT4 && MR == 2) ? epre[m & 1] : epi_load(a, epi, nb, n_local, m));
      }
    }
  if (resid_ss) {
    // this workgroup's sum of y^2 per row (the deferred RMSNorm of the next
    // projection), waves added in a fixed order
    __syncthreads();
    for (int m = threadIdx.x; m < M; m += blockDim.x) {
      float tot = 0.0f;
      for (int w = 0; w < (int)(blockDim.x >> 6); ++w) tot += sspart[w * M + m];
      a.ss_out[(size_t)m * gridDim.x + blockIdx.x] = tot;
    }
  }
  if (a.arg_parts) {
    // Fused greedy head: this workgroup's best eligible logit of each row m
    // (arg_better order), reduced over its 16-row blocks and then its waves.
    __syncthreads();  // the reduction / planes area of smem is reused
    ArgPartial *wpart = (ArgPartial *)smem;  // [waves][M]
    const int nwv = (int)(blockDim.x >> 6);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = mt * 16 + c * 4 + r;
        ArgPartial p;
        p.v = 0.0f;
        p.i = -1;
        p.nan_flag = 0;
        p.rows = 0;
        p.bad_mask = 0;
        p.nan0 = 0;
        if (lead && m < M) {
          const int nrow = nb * 16 + n_local;
          const float v = a.bias ? a.bias[nrow] + acc[mt][r] : acc[mt][r];
          const bool elig =
              !a.arg_words ||
              ((a.arg_words[(size_t)m * a.arg_word_count + (nrow >> 6)] >> (nrow & 63)) & 1ull);
          if (elig) {
            if (isnan(v)) p.nan_flag = 1;
            else {
              p.v = v;
              p.i = nrow;
            }
          }
          if (nrow == 0 && isnan(v)) p.nan0 = 1;
        }
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) arg_merge(p, arg_shfl_xor(p, o));
        if (n_local == 0 && m < M) wpart[wave * M + m] = p;
      }
    __syncthreads();
    for (int m = threadIdx.x; m < M; m += blockDim.x) {
      ArgPartial p = wpart[m];
      for (int w = 1; w < nwv; ++w) arg_merge(p, wpart[w * M + m]);
      a.arg_parts[(size_t)m * gridDim.x + blockIdx.x] = p;
    }
  }
  if (!emit_planes) return;
  __syncthreads();
  // Groups of 32 consecutive SwiGLU outputs = 4 row blocks; each half-wave
  // quantises one (group, row) into the next projection's planes.
  const int half = threadIdx.x >> 5, hl = threadIdx.x & 31, nh = blockDim.x >> 5;
  const int groups = RB / 4;
  const int Gout = a.N / 64;
  for (int gi = half; gi < groups * M; gi += nh) {
    const int m = gi % M, gl = gi / M;
    const int g = nb_wg0 / 4 + gl;
    if (g >= Gout) continue;
    const float v = actbuf[m * (8 * RB) + gl * 32 + hl];
    if (a.out_D == 1)
      quantize_group<1>(v, hl, g, m, M, a.out_q, a.out_meta);
    else
      quantize_group<3>(v, hl, g, m, M, a.out_q, a.out_meta);
  }
}

// 3..5 rows of one-digit planes that fit in LDS run the batched dot4 kernel
// (its cost grows with every row; from 8 rows on the MFMA kernel measured
// faster on the 7B shapes, about even at 5).
// Launch shape for these arguments; also fills the fields launch_gemv
// derives (ksplit, LDS offsets). False when the arguments are invalid.
static bool gemv_shape(GemvArgs &a, GemvShape &p) {
  if (a.M < 1 || a.M > kGemvMaxRows || a.N % 16 || a.K % 128 ||
      (!a.x_in && (!a.act_q || !a.act_meta)))
    return false;
  const bool emit_planes = a.epi == EPI_SWIGLU && a.out_q;
  const bool resid_ss = a.epi == EPI_RESID && a.ss_out;
  // the workgroup must own whole 32-wide output groups (4 row blocks)
  if (emit_planes && ((a.N / 16) % 4 || !a.out_meta || (a.out_D != 1 && a.out_D != 3)))
    return false;
  if (a.ss_out && (a.epi != EPI_RESID || !a.y || !a.resid)) return false;
  if (a.arg_parts && a.epi != EPI_PLAIN) return false;
  if (a.prehead && (!a.arg_parts || !a.arg_words || a.arg_word_count < (a.N + 63) / 64)) return false;
  if (a.in_ss && (!a.x_in || a.in_ss_count <= 0 || a.in_ss_count > kMaxSsParts)) return false;
  p = plan_gemv(a.N, a.K, a.M, a.D);
  const size_t red0 = (size_t)4 * 64 * sizeof(float);  // per wave
  if (a.x_in) {
    // input mode: every workgroup quantises the whole input row, so fewer
    // workgroups than the plane-reading shapes: 8 waves with the K split for
    // short row counts (7B QKV), whole K per wave for tall ones, in
    // workgroups of 4 row blocks for one input row (7B gate/up: 18.7 us
    // against 20.4 with 8 row blocks) and 8 for more (22.7 against 23.4
    // at two rows)
    const int NB = a.N / 16, KQ = a.K / 128;
    p.ksplit = NB >= 1024 ? 1 : std::max(1, std::min(4, KQ / 4));
    p.rb = NB >= 1024 && a.M == 1 ? 4 : 8 / p.ksplit;
    p.waves = p.ksplit * p.rb;
    p.grid = (NB + p.rb - 1) / p.rb;
    p.lds_bytes = std::max(p.lds_a ? planes_bytes(a.K / 32, a.M, a.D) + a.M * 4 : 0,
                           p.waves * red0);
  }
  if (emit_planes && p.rb % 4) {
    p.rb = 4;
    while (p.ksplit * p.rb > 16) p.ksplit /= 2;
    p.waves = p.ksplit * p.rb;
    p.grid = (a.N / 16 + p.rb - 1) / p.rb;
    p.lds_bytes = std::max(p.lds_a ? planes_bytes(a.K / 32, a.M, a.D) + a.M * 4 : 0,
                           p.waves * red0);
  }
  if (a.ksplit_override > 0) {
    if (a.arg_parts) return false;
    p.ksplit = a.ksplit_override;
    p.rb = a.rb_override > 0 ? a.rb_override : std::max(1, 4 / p.ksplit);
    p.waves = p.ksplit * p.rb;
    if (p.waves > 16 || p.ksplit > a.K / 128) return false;
    p.grid = (a.N / 16 + p.rb - 1) / p.rb;
    p.lds_bytes = std::max(p.lds_a ? planes_bytes(a.K / 32, a.M, a.D) + a.M * 4 : 0,
                           p.waves * red0);
    if (emit_planes && p.rb % 4) return false;
  }
  // input mode: the planes are built in LDS, so they must fit there
  if (a.x_in && !p.lds_a) return false;
  if (resid_ss && p.grid > kMaxSsParts) return false;
  if (a.arg_parts)  // one candidate per (wave, row) in LDS
    p.lds_bytes = std::max(p.lds_bytes, (size_t)p.waves * a.M * sizeof(ArgPartial));
  a.ksplit = p.ksplit;
  a.ksplit_lds_off = (int)((p.lds_bytes + 15) & ~(size_t)15);
  if (emit_planes) p.lds_bytes = a.ksplit_lds_off + (size_t)a.M * 8 * p.rb * sizeof(float);
  if (resid_ss) p.lds_bytes = a.ksplit_lds_off + (size_t)p.waves * a.M * sizeof(float);
  return true;
}

bool gemv_launch_shape(const GemvArgs &a0, GemvShape *out) {
  GemvArgs a = a0;
  GemvShape p;
  if (!gemv_shape(a, p)) return false;
  *out = p;
  return true;
}

hipError_t launch_gemv(const GemvArgs &a0, hipStream_t st) {
  GemvArgs a = a0;
  GemvShape p;
  if (!gemv_shape(a, p)) return hipErrorInvalidValue;
  dim3 grid(p.grid), block(64 * p.waves);
  const bool small = p.waves <= 4;
  const size_t lds = p.lds_bytes;
#define GK_LAUNCH(KERNEL)                                                                       \
  do {                                                                                          \
    if (lds > 64 * 1024)                                                                        \
      (void)hipFuncSetAttribute((const void *)KERNEL, hipFuncAttributeMaxDynamicSharedMemorySize, \
                                (int)lds);                                                      \
    hipLaunchKernelGGL(KERNEL, grid, block, lds, st, a);                                        \
  } while (0)
  // workgroups of up to 4 waves (256-thread bound) or up to 16 (1024)
#define GK_GO(DD, LL, EE, XX)                                                                   \
  do {                                                                                          \
    if (small) GK_LAUNCH((gemv_kernel<DD, LL, 256, EE, XX>));                                   \
    else GK_LAUNCH((gemv_kernel<DD, LL, 1024, EE, XX>));                                        \
  } while (0)
  // the epilogue type is a template parameter
#define GK_DOT4(DD, LL, XX)                                                \
  do {                                                                     \
    switch (a.epi) {                                                       \
      case EPI_PLAIN: GK_GO(DD, LL, EPI_PLAIN, XX); break;                 \
      case EPI_RESID: GK_GO(DD, LL, EPI_RESID, XX); break;                 \
      case EPI_SWIGLU: GK_GO(DD, LL, EPI_SWIGLU, XX); break;               \
      default: GK_GO(DD, LL, EPI_QKV, XX); break;                          \
    }                                                                      \
  } while (0)
  if (a.x_in) {
    if (a.D == 1) GK_DOT4(1, true, true); else GK_DOT4(3, true, true);
  } else if (a.D == 1) {
    if (p.lds_a) GK_DOT4(1, true, false); else GK_DOT4(1, false, false);
  } else {
    if (p.lds_a) GK_DOT4(3, true, false); else GK_DOT4(3, false, false);
  }
#undef GK_DOT4
#undef GK_GO
#undef GK_LAUNCH
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// plain RMSNorm (kernels.zig:141-220) and the embedding gather
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *x, const float *w, int dim,
                                                      float eps, float *out) {
  const int row = blockIdx.x, t = threadIdx.x;
  const float *xr = x + (size_t)row * dim;
  __shared__ float red[8];
  float ss = 0.0f;
  for (int i = t; i < dim; i += 256) ss = fmaf(xr[i], xr[i], ss);
  ss = wave_sum(ss);
  if ((t & 63) == 0) red[t >> 6] = ss;
  __syncthreads();
  if (t == 0) red[4] = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)dim + eps);
  __syncthreads();
  const float inv = red[4];
  for (int i = t; i < dim; i += 256) {
    float tt = xr[i] * inv;
    out[(size_t)row * dim + i] = tt * w[i];
  }
}

hipError_t launch_rmsnorm(const float *x, const float *w, int rows, int dim, float eps,
                          float *out, hipStream_t st) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, st, x, w, dim, eps, out);
  return hipGetLastError();
}

// Embedding gather (generate.zig:3653-3663): one element per thread, a
// block covers 256 columns of one row; with ss_out set it also writes the
// block's sum of x^2 to ss_out [M][gridDim.x] (the next projection's
// deferred RMSNorm).
__global__ __launch_bounds__(256) void gather_rows_kernel(const float *table, const int32_t *ids,
                                                         int dim, float *out, float *ss_out) {
  const int m = blockIdx.y, t = threadIdx.x;
  const int i = blockIdx.x * 256 + t;
  const size_t src = (size_t)ids[m] * dim;
  float v = 0.0f;
  if (i < dim) {
    v = table[src + i];
    out[(size_t)m * dim + i] = v;
  }
  if (!ss_out) return;
  __shared__ float red[4];
  float sq = v * v;
  sq = wave_sum(sq);
  if ((t & 63) == 0) red[t >> 6] = sq;
  __syncthreads();
  if (t == 0) ss_out[(size_t)m * gridDim.x + blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

int gather_ss_parts(int dim) { return (dim + 255) / 256; }

hipError_t launch_gather_rows(const float *table, const int32_t *ids, int M, int dim, float *out,
                              hipStream_t st, float *ss_out) {
  hipLaunchKernelGGL(gather_rows_kernel, dim3(gather_ss_parts(dim), M), dim3(256), 0, st, table,
                     ids, dim, out, ss_out);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// K3: paged GQA decode attention
// ---------------------------------------------------------------------------
// grid (chunks, kv heads, rows). A workgroup serves the G = Hq / Hkv query
// heads that share one KV head over one context chunk. HD/8 threads cooperate
// on a position (one 16-byte fp16 load each), so K and V rows are read fully
// coalesced straight from the lane's pages. One chunk: the output is written
// directly with the weights normalised first (forward.zig:515-528); several
// chunks: (max, sum, unnormalised output) records are merged by the combine
// kernel with the usual log-sum-exp rescaling.
static constexpr int kMaxChunk = 512;
static constexpr int kMaxRecords = 1024;  // chunk records one combine merges
static constexpr int kMaxGroup = 8;
static constexpr long kAttnMaxGrid = 4096;  // fp16 attention: workgroups per launch at most
static constexpr int kF16MinChunk = 64;      // fewest positions per fp16-KV work item

// Chunk length: short contexts stay one chunk (no combine launch); long ones
// are split until (chunks x KV heads x rows) >= 2048 work items or chunks of
// 64 positions, so a few long lanes still spread over the whole chip.
int attention_chunk(int max_ctx, int num_kv_heads, int M) {
  int ch = kMaxChunk;
  if (max_ctx > 2 * kMaxChunk)
    while (ch > 64 && ((max_ctx + ch - 1) / ch) * num_kv_heads * M < 2048) ch /= 2;
  return ch;
}

size_t attention_scratch_floats(int max_rows, int num_heads, int num_kv_heads, int head_dim,
                                int max_ctx) {
  // fp16 KV: a chunk record per kF16MinChunk positions and (row, query head)
  size_t most = (size_t)max_rows * num_heads * ((max_ctx + kF16MinChunk - 1) / kF16MinChunk) *
                (2 + head_dim);
  // f32 KV: the largest chunk-record set the planner produces for any row count
  for (int M = 1; M <= max_rows; ++M) {
    const int ch = attention_chunk(max_ctx, num_kv_heads, M);
    const size_t nch = (size_t)(max_ctx + ch - 1) / ch;
    most = std::max(most, (size_t)M * num_heads * nch * (2 + head_dim));
  }
  return most;
}

template <int HD, int F16>
static __device__ __forceinline__ void load8(const void *pool, size_t idx, float *v) {
  if (F16) {
    const uint4 raw = *(const uint4 *)((const __half *)pool + idx);
    const __half *hp = (const __half *)&raw;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = __half2float(hp[e]);
  } else {
    const float4 r0 = *(const float4 *)((const float *)pool + idx);
    const float4 r1 = *(const float4 *)((const float *)pool + idx + 4);
    v[0] = r0.x; v[1] = r0.y; v[2] = r0.z; v[3] = r0.w;
    v[4] = r1.x; v[5] = r1.y; v[6] = r1.z; v[7] = r1.w;
  }
}

template <int HD, int F16, int HPW>
__global__ __launch_bounds__(256) void attn_decode_kernel(
    const float *q, const void *kv_pool, const int32_t *page_table, int max_pages,
    const int32_t *lane_of_row, const int32_t *ctx_len, int layer, int num_layers, int Hq,
    int Hkv, int chunk, int n_chunks_max, int max_ctx, float *scratch, float *out,
    PlanesDst pd) {
  constexpr int TPP = HD / 8;        // threads per position
  constexpr int PPP = 256 / TPP;     // positions per pass
  constexpr int PPW = 64 / TPP;      // positions per wave
  const int ch = blockIdx.x, m = blockIdx.z, t = threadIdx.x;
  // HPW == 1: one query head per workgroup (blockIdx.y = query head);
  // otherwise all G query heads of one KV head (blockIdx.y = KV head).
  const int Gfull = Hq / Hkv;
  const int h = HPW == 1 ? (int)blockIdx.y / Gfull : (int)blockIdx.y;
  const int qh0 = HPW == 1 ? (int)blockIdx.y : h * Gfull;
  const int G = HPW == 1 ? 1 : Gfull;
  const int ctx = min(ctx_len[m], max_ctx);
  const int j0 = ch * chunk;
  if (j0 >= ctx) return;
  const int n = min(chunk, ctx - j0);
  const int nch = (ctx + chunk - 1) / chunk;
  const int kv_dim = Hkv * HD;
  const int lane_id = lane_of_row[m];
  __shared__ float sq[HPW][HD];
  __shared__ float ss[HPW][kMaxChunk];
  __shared__ float red[4][HPW][HD];
  __shared__ float smax[HPW], ssum[HPW];
  __shared__ int spage[kMaxChunk / 16];
  for (int i = t; i < G * HD; i += 256)
    sq[i / HD][i % HD] = q[(size_t)m * Hq * HD + (size_t)qh0 * HD + i];
  for (int i = t; i < (n + 15) / 16; i += 256)
    spage[i] = page_table[(size_t)lane_id * max_pages + (j0 / 16) + i];
  __syncthreads();

  const int sub = t % TPP, pp = t / TPP;
  const float scale = 1.0f / sqrtf((float)HD);
  const size_t lay = (size_t)num_layers;
  // ---- scores ----
  if constexpr (F16 && HPW == kMaxGroup) {
    // fp16 KV: S[head][pos] = q . k on v_mfma_f32_16x16x16_f16, one 16-position
    // tile (one page) per MFMA column block, query heads as MFMA rows. q is
    // split into fp16 hi + lo parts (q = hi + lo to ~2^-22 relative); the
    // fp16 x fp16 products are exact in the f32 accumulator, so the score is
    // the f32 dot product up to summation order. Lane (c, j) loads 16-byte
    // pieces 4*tt + c of position j's K row, which fixes the dims of k-chunk c
    // in step s: 8 * (4 * (s / 2) + c) + 4 * (s % 2) + 0..3.
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    typedef float f4 __attribute__((ext_vector_type(4)));
    constexpr int S = HD / 16;
    const int wv = t >> 6, l = t & 63, c = l >> 4, jr = l & 15;
    h4 qhi[S], qlo[S];
#pragma unroll
    for (int st = 0; st < S; ++st) {
      const int base = 8 * (4 * (st >> 1) + c) + 4 * (st & 1);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = jr < G ? sq[jr][base + e] : 0.0f;
        const _Float16 hv = (_Float16)v;
        qhi[st][e] = hv;
        qlo[st][e] = (_Float16)(v - (float)hv);
      }
    }
    for (int T = wv; T * 16 < n; T += 4) {
      const int pl = T * 16 + jr;  // position within the chunk; page = spage[T]
      const bool valid = pl < n;
      const __half *krow = (const __half *)kv_pool +
                           ((((size_t)spage[T] * lay + layer) * 2 + 0) * 16 + jr) * kv_dim +
                           (size_t)h * HD;
      uint4 kr[HD / 32];
#pragma unroll
      for (int tt = 0; tt < HD / 32; ++tt)
        kr[tt] = valid ? *(const uint4 *)(krow + 8 * (4 * tt + c)) : make_uint4(0, 0, 0, 0);
      f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int st = 0; st < S; ++st) {
        const uint4 w = kr[st >> 1];
        const uint2 bw = (st & 1) ? make_uint2(w.z, w.w) : make_uint2(w.x, w.y);
        h4 b;
        __builtin_memcpy(&b, &bw, 8);
        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(qhi[st], b, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(qlo[st], b, acc, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int head = 4 * c + r;
        if (head < G && valid) ss[head][pl] = acc[r] * scale;
      }
    }
  } else {
    float qf[HPW][8];
#pragma unroll
    for (int g = 0; g < HPW; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[g][e] = g < G ? sq[g][sub * 8 + e] : 0.0f;
    constexpr int B = 8;  // rows in flight per thread
    for (int i0 = pp; i0 < n; i0 += B * PPP) {
      float kv[B][8];
#pragma unroll
      for (int b = 0; b < B; ++b) {
        const int i = i0 + b * PPP;
        if (i < n) {
          const int j = j0 + i;
          const size_t idx =
              ((((size_t)spage[i >> 4] * lay + layer) * 2 + 0) * 16 + (j & 15)) * kv_dim +
              (size_t)h * HD + sub * 8;
          load8<HD, F16>(kv_pool, idx, kv[b]);
        }
      }
#pragma unroll
      for (int b = 0; b < B; ++b) {
        const int i = i0 + b * PPP;
        if (i >= n) break;
#pragma unroll
        for (int g = 0; g < HPW; ++g) {
          if (g >= G) break;
          float d = 0.0f;
#pragma unroll
          for (int e = 0; e < 8; ++e) d = fmaf(qf[g][e], kv[b][e], d);
#pragma unroll
          for (int o = TPP / 2; o > 0; o >>= 1) d += __shfl_xor(d, o);
          if (sub == 0) ss[g][i] = d * scale;
        }
      }
    }
  }
  __syncthreads();
  // ---- softmax statistics: wave w handles heads w, w + 4 ----
  {
    const int w = t >> 6, l = t & 63;
    for (int g = w; g < G; g += 4) {
      float mx = -INFINITY;
      for (int i = l; i < n; i += 64) mx = fmaxf(mx, ss[g][i]);
      for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
      float sum = 0.0f;
      for (int i = l; i < n; i += 64) {
        const float e = expf(ss[g][i] - mx);
        ss[g][i] = e;
        sum += e;
      }
      for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
      if (nch == 1) {
        const float inv = 1.0f / sum;
        for (int i = l; i < n; i += 64) ss[g][i] = ss[g][i] * inv;
      }
      if (l == 0) {
        smax[g] = mx;
        ssum[g] = sum;
      }
    }
  }
  __syncthreads();
  // ---- weighted V ----
  float acc[HPW][8];
#pragma unroll
  for (int g = 0; g < HPW; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.0f;
  {
    constexpr int B = 8;
    for (int i0 = pp; i0 < n; i0 += B * PPP) {
      float v[B][8];
#pragma unroll
      for (int b = 0; b < B; ++b) {
        const int i = i0 + b * PPP;
        if (i < n) {
          const int j = j0 + i;
          const size_t idx =
              ((((size_t)spage[i >> 4] * lay + layer) * 2 + 1) * 16 + (j & 15)) * kv_dim +
              (size_t)h * HD + sub * 8;
          load8<HD, F16>(kv_pool, idx, v[b]);
        }
      }
#pragma unroll
      for (int b = 0; b < B; ++b) {
        const int i = i0 + b * PPP;
        if (i >= n) break;
#pragma unroll
        for (int g = 0; g < HPW; ++g) {
          if (g >= G) break;
          const float w = ss[g][i];
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(w, v[b][e], acc[g][e]);
        }
      }
    }
  }
  // reduce over the positions of a wave (lanes sub + TPP * k), then over waves
#pragma unroll
  for (int g = 0; g < HPW; ++g) {
    if (g >= G) break;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = acc[g][e];
#pragma unroll
      for (int o = TPP; o < 64; o <<= 1) v += __shfl_xor(v, o);
      acc[g][e] = v;
    }
  }
  const int w = t >> 6, l = t & 63;
  if (l < TPP) {
#pragma unroll
    for (int g = 0; g < HPW; ++g) {
      if (g >= G) break;
#pragma unroll
      for (int e = 0; e < 8; ++e) red[w][g][l * 8 + e] = acc[g][e];
    }
  }
  __syncthreads();
  (void)PPW;
  for (int o = t; o < G * HD; o += 256) {
    const int g = o / HD, d = o % HD;
    const float sum = ((red[0][g][d] + red[1][g][d]) + red[2][g][d]) + red[3][g][d];
    const int qh = qh0 + g;
    if (nch == 1) {
      out[((size_t)m * Hq + qh) * HD + d] = sum;
      emit_group(pd, sum, t & 31, (qh * HD + d) >> 5, m, (int)gridDim.z);
    } else {
      float *rec = scratch + (((size_t)m * Hq + qh) * n_chunks_max + ch) * (2 + HD);
      if (d == 0) {
        rec[0] = smax[g];
        rec[1] = ssum[g];
      }
      rec[2 + d] = sum;
    }
  }
}

// ---------------------------------------------------------------------------
// fp16-KV streaming attention. The work list is every (row, KV head, chunk
// of CH = NW * NT * 16 positions) with each row's chunks counted from its own
// context length, rows in order; workgroup b takes items b, b + grid, ...,
// so no chunk past a row's context is ever launched for it. A wave owns NT
// pages of its chunk (16 positions each): it reads their page ids once
// (wave-uniform scalar loads), issues every K and V load of them together
// and keeps the softmax in registers:
//   scores  S^T[pos][head] = K . Q^T on v_mfma_f32_16x16x16f16, q split into
//           fp16 hi + lo so every product is exact in f32; lane (c, j) ends
//           with head j's scores of positions 4c + r (r = 0..3) of a page,
//   softmax max / exp / sum per head over the wave's positions (in-lane, then
//           two cross-row shuffles),
//   P.V     on v_mfma_f32_16x16x16f16 as well: the A operand is P[head j]
//           [positions 4c .. 4c+3], which is exactly what lane (c, j) holds,
//           split into fp16 hi + lo (V is exact in fp16, so the products
//           are exact in f32); lane (c, j) supplies V[4c + r][DPL * j + e]
//           for output block e from the DPL consecutive dims it read of each
//           of its four V rows (one 16-byte load per row at hd 128), so V is
//           read row-major and fully coalesced.
// The waves' (max, sum, output) states merge by log-sum-exp in LDS. A row
// whose context is one chunk writes its output normalised once by the sum
// (forward.zig:515-528); otherwise every chunk writes a (max, sum, output)
// record per query head for the combine kernel.
// ---------------------------------------------------------------------------
// LDS of one fp16 attention work item: every wave's (output, max, sum)
// state and the log-sum-exp merge weights.
template <int HD, int NW>
struct AttnF16Lds {
  float so[NW][kMaxGroup][HD];
  float sm[NW][16], sl[NW][16];
  float fw[NW][kMaxGroup], mg[kMaxGroup];
};

// One work item of fp16-KV attention: positions j0 .. j0 + n - 1 of one
// row's context for KV head h (qrow = the row's q at its first query head
// h * G, ptab = the row's page table at page j0 / 16). Every thread of the
// NW-wave workgroup calls it; on return (after two barriers) each wave's
// state is in s.so / s.sm / s.sl and the merge weights in s.fw / s.mg, so
// the merged output of query head g, dim d is
//   O = sum_w s.so[w][g][d] * s.fw[w][g],  L = sum_w s.sl[w][g] * s.fw[w][g],
// with maximum s.mg[g] (waves added in order). The caller must pass a
// barrier before the next call reuses s. after_issue() runs in every wave
// once the item's q, K and V loads are requested and before any of them is
// waited for: loads the caller requests there return after the item's
// (vector loads complete in issue order), so they never delay it.
struct AttnNoHook {
  __device__ void operator()() const {}
};

typedef float attn_f4 __attribute__((ext_vector_type(4)));

// The end of an attention work item: each wave's (output, max, sum) state
// into s (lane (c, j) holds O[head 4c + r][dim (HD / 16) * j + e] in
// o[e][r], and head j's max and sum), then the log-sum-exp weights of the
// waves. The weight of wave w for head g, exp(m_w - M) (0 for a wave
// without positions), is computed once per (wave, head); every output is
// then two short dot products over the waves, in wave order.
template <int HD, int NW>
static __device__ __forceinline__ void attn_item_merge(const attn_f4 (&o)[HD / 16], float mx,
                                                       float sum, int G, AttnF16Lds<HD, NW> &s) {
  constexpr int DPL = HD / 16, NTH = 64 * NW;
  const int t = threadIdx.x, l = t & 63;
  const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
  const int c = l >> 4, j = l & 15;
  if (c < 2) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr)
#pragma unroll
      for (int e = 0; e < DPL; ++e) s.so[wv][4 * c + rr][DPL * j + e] = o[e][rr];
  }
  if (c == 0) {
    s.sm[wv][j] = mx;
    s.sl[wv][j] = sum;
  }
  __syncthreads();
  for (int i = t; i < NW * G; i += NTH) {
    const int w = i / G, g = i % G;
    float Mx = -INFINITY;
#pragma unroll
    for (int w2 = 0; w2 < NW; ++w2)
      if (s.sl[w2][g] > 0.0f) Mx = fmaxf(Mx, s.sm[w2][g]);
    s.fw[w][g] = s.sl[w][g] > 0.0f ? expf(s.sm[w][g] - Mx) : 0.0f;
    if (w == 0) s.mg[g] = Mx;
  }
  __syncthreads();
}
template <int HD, int NT, int NW, class Hook = AttnNoHook>
static __device__ __forceinline__ void attn_f16_item(const float *qrow, const __half *pool,
                                                     const int32_t *ptab, int n, int layer,
                                                     size_t lay, int kv_dim, int h, int G,
                                                     AttnF16Lds<HD, NW> &s,
                                                     const Hook &after_issue = Hook()) {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  typedef attn_f4 f4;
  constexpr int S = HD / 16;    // f16 MFMA steps over the head dim
  constexpr int DPL = HD / 16;  // dims per lane and V row = output blocks of P.V
  constexpr int WP = 16 * NT;   // positions per wave
  constexpr int NTH = 64 * NW;
  typedef typename std::conditional<DPL == 8, uint4, uint2>::type vrow_t;
  const int t = threadIdx.x, l = t & 63;
  const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
  const float scale = 1.0f / sqrtf((float)HD);
  const int wbase = wv * WP;
  const int c = l >> 4, j = l & 15;
  const int wn = max(0, min(WP, n - wbase));

  f4 o[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) o[e] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  float mx = -INFINITY, sum = 0.0f;
  float4 qv[S];
  uint4 kr[NT][HD / 32];
  vrow_t vr[NT][4];
  if (wn > 0) {
    // q first (it depends on nothing the page walk reads), as the B operand:
    // lane (c, j) holds head j's dims of k-chunk c
    // (every load of the item is unconditional, from an address clamped into
    // range: a conditional load whose lanes are zeroed instead makes the
    // compiler wait for it before the next one, serialising the batch;
    // validity is applied by value when the data is used)
    const float *qr = qrow + (size_t)(j < G ? j : 0) * HD;
#pragma unroll
    for (int st = 0; st < S; ++st) {
      const int base = 8 * (4 * (st >> 1) + c) + 4 * (st & 1);
      qv[st] = *(const float4 *)(qr + base);
    }
    // page ids of this wave's pages (wave-uniform)
    const int32_t *pt = ptab + wbase / 16;
    int pg[NT];
#pragma unroll
    // (an unconditional load from a wave-uniform clamped index is a scalar
    // load; a conditional one becomes a vector load, which completes only
    // after every vector load issued before it, q's included)
    for (int T = 0; T < NT; ++T) pg[T] = pt[16 * T < wn ? T : 0];
    // K: lane (c, j) loads 16-byte pieces 4 * tt + c of position j of each
    // page; V: lane (c, j) loads dims DPL*j .. DPL*j + DPL-1 of positions
    // 4c + r (r = 0..3) of each page. Pages past the item read page 0 and
    // positions past it stay inside their page, so every load is in range;
    // their scores are masked and their V rows zeroed before use.
#pragma unroll
    for (int T = 0; T < NT; ++T) {
      const size_t pbase = ((size_t)pg[T] * lay + layer) * 2;
      const __half *krow = pool + ((pbase + 0) * 16 + j) * kv_dim + (size_t)h * HD;
#pragma unroll
      for (int tt = 0; tt < HD / 32; ++tt) kr[T][tt] = *(const uint4 *)(krow + 8 * (4 * tt + c));
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int pos = 4 * c + rr;
        const __half *vrow = pool + ((pbase + 1) * 16 + pos) * kv_dim + (size_t)h * HD + DPL * j;
        vr[T][rr] = *(const vrow_t *)vrow;
      }
    }
  }
  if constexpr (!std::is_same<Hook, AttnNoHook>::value) {
    // (the scheduler would otherwise hoist the hook's loads above the item's)
    __builtin_amdgcn_sched_barrier(0);
    after_issue();
    __builtin_amdgcn_sched_barrier(0);
  }
  if (wn > 0) {
    // q split into f16 hi + lo (after the K/V loads are in flight); lanes of
    // heads past G hold zeros
    h4 qhi[S], qlo[S];
#pragma unroll
    for (int st = 0; st < S; ++st) {
      const float qa[4] = {j < G ? qv[st].x : 0.0f, j < G ? qv[st].y : 0.0f,
                           j < G ? qv[st].z : 0.0f, j < G ? qv[st].w : 0.0f};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const _Float16 hv = (_Float16)qa[e];
        qhi[st][e] = hv;
        qlo[st][e] = (_Float16)(qa[e] - (float)hv);
      }
    }
    // scores: S^T = K . Q^T, one 16x16 tile per page
    f4 sc[NT];
#pragma unroll
    for (int T = 0; T < NT; ++T) {
      f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int st = 0; st < S; ++st) {
        const uint4 w = kr[T][st >> 1];
        const uint2 bw = (st & 1) ? make_uint2(w.z, w.w) : make_uint2(w.x, w.y);
        h4 a;
        __builtin_memcpy(&a, &bw, 8);
        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(a, qhi[st], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(a, qlo[st], acc, 0, 0, 0);
      }
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const float v = acc[rr] * scale;
        sc[T][rr] = 16 * T + 4 * c + rr < wn ? v : -INFINITY;
        mx = fmaxf(mx, sc[T][rr]);
      }
    }
    mx = xor32_max(xor16_max(mx));
#pragma unroll
    for (int T = 0; T < NT; ++T)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const float p = expf(sc[T][rr] - mx);
        sc[T][rr] = p;
        sum += p;
      }
    sum = xor32_add(xor16_add(sum));
    // P.V: A = P[head j][pos 4c .. 4c+3] (this lane's own registers, fp16
    // hi + lo), B_e = V[pos 4c + r][dim DPL * j + e]
#pragma unroll
    for (int T = 0; T < NT; ++T) {
      h4 phi, plo;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const _Float16 hv = (_Float16)sc[T][rr];
        phi[rr] = hv;
        plo[rr] = (_Float16)(sc[T][rr] - (float)hv);
      }
      // V rows past the item are zeroed (P is 0 there, but a stale row
      // might hold an infinity)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr)
        if (16 * T + 4 * c + rr >= wn) __builtin_memset(&vr[T][rr], 0, sizeof(vrow_t));
      const _Float16 *v0 = (const _Float16 *)&vr[T][0];
      const _Float16 *v1 = (const _Float16 *)&vr[T][1];
      const _Float16 *v2 = (const _Float16 *)&vr[T][2];
      const _Float16 *v3 = (const _Float16 *)&vr[T][3];
#pragma unroll
      for (int e = 0; e < DPL; ++e) {
        const h4 bv = {v0[e], v1[e], v2[e], v3[e]};
        o[e] = __builtin_amdgcn_mfma_f32_16x16x16f16(phi, bv, o[e], 0, 0, 0);
        o[e] = __builtin_amdgcn_mfma_f32_16x16x16f16(plo, bv, o[e], 0, 0, 0);
      }
    }
  }
  attn_item_merge<HD, NW>(o, mx, sum, G, s);
}

// The same work item over f32 KV pages (the reference's KV storage), with
// the same lane layout, softmax and merge as attn_f16_item, on
// v_mfma_f32_16x16x16f16 with every f32 operand split into fp16 hi + lo
// (x = hi + lo to ~2^-22 relative): a product is hi*hi + hi*lo + lo*hi, each
// term exact in the f32 accumulator (the lo*lo term, ~2^-22 of the product,
// is dropped), so scores and outputs carry f32 accuracy as in the
// reference's f32 attention (forward.zig:478-533) up to summation order.
// (Against v_mfma_f32_16x16x4f32 on the f32 values: three MFMAs of a
// quarter of the cost each instead of four, 620 against 615 tok/s in the 7B
// batch-1 token and 1261 against 1245 for the 0.5B model.)
//   scores  S^T[pos][head] = K . Q^T, 4 dims per lane and step: lane (c, j)
//           gives K[pos j] and q[head j] at dims c * HD / 4 + 4 st + 0..3 in
//           step st (a dot product may take its dims in any order, so each
//           lane reads a contiguous quarter of the K row and of q, as
//           float4s); the result tile is laid out as attn_f16_item's (lane
//           (c, j): head j's scores of positions 4c + r);
//   P.V     one MFMA triple per page and output block e over positions
//           4c .. 4c + 3: the A operand is P[head j][pos 4c + r], the lane's
//           own registers, the B operand V[4c + r][DPL * j + e] from the DPL
//           consecutive dims the lane read of each of its four V rows; lane
//           (c, j) ends with O[head 4c + r][dim DPL * j + e].
// Every load is unconditional from an in-range address (as there). q is
// staged in LDS (qs, kMaxGroup * HD floats) by the whole workgroup and read
// a float4 per step: f32 K and V rows take twice the registers of fp16 ones.
template <int HD, int NT, int NW, class Hook = AttnNoHook>
static __device__ __forceinline__ void attn_f32_item(const float *qrow, const float *pool,
                                                     const int32_t *ptab, int n, int layer,
                                                     size_t lay, int kv_dim, int h, int G,
                                                     AttnF16Lds<HD, NW> &s, float *qs,
                                                     const Hook &after_issue = Hook()) {
  typedef attn_f4 f4;
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  // x = hi + lo to ~2^-22 relative, each part fp16
  auto split_f16 = [](const float (&x)[4], h4 &hi, h4 &lo) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const _Float16 hv = (_Float16)x[e];
      hi[e] = hv;
      lo[e] = (_Float16)(x[e] - (float)hv);
    }
  };
  constexpr int QD = HD / 4;    // dims per lane of q and of a K row (4 per MFMA step)
  constexpr int DPL = HD / 16;  // dims per lane and V row = output blocks of P.V
  constexpr int WP = 16 * NT;   // positions per wave
  const int t = threadIdx.x, l = t & 63;
  const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
  const float scale = 1.0f / sqrtf((float)HD);
  const int wbase = wv * WP;
  const int c = l >> 4, j = l & 15;
  const int wn = max(0, min(WP, n - wbase));

  f4 o[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) o[e] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  float mx = -INFINITY, sum = 0.0f;
  // q first (G * HD floats, a float4 per thread; HD is a multiple of 4)
  constexpr int NTH = 64 * NW;
  static_assert(kMaxGroup * HD / 4 <= NTH, "one float4 of q per thread");
  const int nq4 = G * HD / 4;
  const float4 qload = *(const float4 *)(qrow + 4 * min(t, nq4 - 1));
  float4 kr[NT][QD / 4];
  float4 vr[NT][4][DPL / 4];
  if (wn > 0) {
    const int32_t *pt = ptab + wbase / 16;
    int pg[NT];
#pragma unroll
    for (int T = 0; T < NT; ++T) pg[T] = pt[16 * T < wn ? T : 0];
#pragma unroll
    for (int T = 0; T < NT; ++T) {
      const size_t pbase = ((size_t)pg[T] * lay + layer) * 2;
      const float *krow = pool + ((pbase + 0) * 16 + j) * kv_dim + (size_t)h * HD + c * QD;
#pragma unroll
      for (int i = 0; i < QD / 4; ++i) kr[T][i] = *(const float4 *)(krow + 4 * i);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const float *vrow =
            pool + ((pbase + 1) * 16 + 4 * c + rr) * kv_dim + (size_t)h * HD + DPL * j;
#pragma unroll
        for (int i = 0; i < DPL / 4; ++i) vr[T][rr][i] = *(const float4 *)(vrow + 4 * i);
      }
    }
  }
  if constexpr (!std::is_same<Hook, AttnNoHook>::value) {
    __builtin_amdgcn_sched_barrier(0);
    after_issue();
    __builtin_amdgcn_sched_barrier(0);
  }
  // (q's load was the first issued, so this wait leaves K and V in flight)
  if (t < nq4) *(float4 *)(qs + 4 * t) = qload;
  __syncthreads();
  if (wn > 0) {
    // lanes of heads past G take q = 0 (their rows are never read)
    const bool qon = j < G;
    const float *qr = qs + (j < G ? j : 0) * HD + c * QD;
    f4 sc[NT];
#pragma unroll
    for (int T = 0; T < NT; ++T) {
      f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int i = 0; i < QD / 4; ++i) {
        const float4 qv = *(const float4 *)(qr + 4 * i);
        const float qa[4] = {qon ? qv.x : 0.0f, qon ? qv.y : 0.0f, qon ? qv.z : 0.0f,
                             qon ? qv.w : 0.0f};
        const float ka[4] = {kr[T][i].x, kr[T][i].y, kr[T][i].z, kr[T][i].w};
        h4 kh, kl, qh, ql;
        split_f16(ka, kh, kl);
        split_f16(qa, qh, ql);
        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(kh, qh, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(kh, ql, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(kl, qh, acc, 0, 0, 0);
      }
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const float v = acc[rr] * scale;
        sc[T][rr] = 16 * T + 4 * c + rr < wn ? v : -INFINITY;
        mx = fmaxf(mx, sc[T][rr]);
      }
    }
    mx = xor32_max(xor16_max(mx));
#pragma unroll
    for (int T = 0; T < NT; ++T)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const float p = expf(sc[T][rr] - mx);
        sc[T][rr] = p;
        sum += p;
      }
    sum = xor32_add(xor16_add(sum));
#pragma unroll
    for (int T = 0; T < NT; ++T) {
      // V rows past the item are zeroed (P is 0 there, but a stale row
      // might hold an infinity)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr)
        if (16 * T + 4 * c + rr >= wn)
#pragma unroll
          for (int i = 0; i < DPL / 4; ++i) vr[T][rr][i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      const float pa[4] = {sc[T][0], sc[T][1], sc[T][2], sc[T][3]};
      h4 ph, pl;
      split_f16(pa, ph, pl);
      const float *v0 = (const float *)&vr[T][0][0], *v1 = (const float *)&vr[T][1][0];
      const float *v2 = (const float *)&vr[T][2][0], *v3 = (const float *)&vr[T][3][0];
#pragma unroll
      for (int e = 0; e < DPL; ++e) {
        const float va[4] = {v0[e], v1[e], v2[e], v3[e]};
        h4 vh, vl;
        split_f16(va, vh, vl);
        o[e] = __builtin_amdgcn_mfma_f32_16x16x16f16(ph, vh, o[e], 0, 0, 0);
        o[e] = __builtin_amdgcn_mfma_f32_16x16x16f16(ph, vl, o[e], 0, 0, 0);
        o[e] = __builtin_amdgcn_mfma_f32_16x16x16f16(pl, vh, o[e], 0, 0, 0);
      }
    }
  }
  attn_item_merge<HD, NW>(o, mx, sum, G, s);
}

// ---------------------------------------------------------------------------
// fp16-KV streaming attention. The work list is every (row, KV head, chunk
// of CH = NW * NT * 16 positions) with each row's chunks counted from its own
// context length, rows in order; workgroup b takes items b, b + grid, ...,
// so no chunk past a row's context is ever launched for it. A wave owns NT
// pages of its chunk (16 positions each): it reads their page ids once
// (wave-uniform scalar loads), issues every K and V load of them together
// and keeps the softmax in registers:
//   scores  S^T[pos][head] = K . Q^T on v_mfma_f32_16x16x16f16, q split into
//           fp16 hi + lo so every product is exact in f32; lane (c, j) ends
//           with head j's scores of positions 4c + r (r = 0..3) of a page,
//   softmax max / exp / sum per head over the wave's positions (in-lane, then
//           two cross-row shuffles),
//   P.V     on v_mfma_f32_16x16x16f16 as well: the A operand is P[head j]
//           [positions 4c .. 4c+3], which is exactly what lane (c, j) holds,
//           split into fp16 hi + lo (V is exact in fp16, so the products
//           are exact in f32); lane (c, j) supplies V[4c + r][DPL * j + e]
//           for output block e from the DPL consecutive dims it read of each
//           of its four V rows (one 16-byte load per row at hd 128), so V is
//           read row-major and fully coalesced.
// The waves' (max, sum, output) states merge by log-sum-exp in LDS. A row
// whose context is one chunk writes its output normalised once by the sum
// (forward.zig:515-528); otherwise every chunk writes a (max, sum, output)
// record per query head for the combine kernel.
// ---------------------------------------------------------------------------
template <int HD, int NT, int NW>
__global__ __launch_bounds__(64 * NW) void attn_f16_kernel(
    const float *q, const __half *pool, const int32_t *page_table, int max_pages,
    const int32_t *lane_of_row, const int32_t *ctx_len, int M, int layer, int num_layers, int Hq,
    int Hkv, int n_chunks_max, int max_ctx, float *scratch, float *out, PlanesDst pd) {
  constexpr int WP = 16 * NT;   // positions per wave
  constexpr int CH = NW * WP;   // positions per work item
  constexpr int NTH = 64 * NW;
  const int t = threadIdx.x, l = t & 63;
  const int G = Hq / Hkv;
  const int kv_dim = Hkv * HD;
  __shared__ AttnF16Lds<HD, NW> s;

  // the work list (every wave holds it; lane r describes row r, M <= 64)
  const int cl = l < M ? min(ctx_len[l], max_ctx) : 0;
  const int ln = l < M ? lane_of_row[l] : 0;
  const int nchl = (cl + CH - 1) / CH;
  int incl = nchl * Hkv;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int v = __shfl_up(incl, o, 64);
    if (l >= o) incl += v;
  }
  const int total = __builtin_amdgcn_readfirstlane(__shfl(incl, 63, 64));

  for (int item = blockIdx.x; item < total; item += gridDim.x) {
    // the item's row: the lanes whose running count is <= item precede it
    const int k = __popcll(__ballot(incl <= item));
    const int m = __builtin_amdgcn_readfirstlane(k);
    const int ctx = __builtin_amdgcn_readfirstlane(__shfl(cl, k, 64));
    const int lane = __builtin_amdgcn_readfirstlane(__shfl(ln, k, 64));
    const int before = __builtin_amdgcn_readfirstlane(__shfl(incl, k > 0 ? k - 1 : 0, 64));
    const int nch = (ctx + CH - 1) / CH;
    const int r = item - (m > 0 ? before : 0);
    const int h = r / nch, ch = r - h * nch;
    const int qh0 = h * G;
    const int j0 = ch * CH;
    attn_f16_item<HD, NT, NW>(q + ((size_t)m * Hq + qh0) * HD, pool,
                              page_table + (size_t)lane * max_pages + j0 / 16, min(CH, ctx - j0),
                              layer, (size_t)num_layers, kv_dim, h, G, s);
    constexpr int RS = 2 + HD;  // floats per record
    const size_t hstride = (size_t)n_chunks_max * RS;
    float *rbase = scratch + ((size_t)m * Hq + qh0) * hstride;
    for (int oi = t; oi < G * HD; oi += NTH) {
      const int g = oi / HD, d = oi % HD;
      float L = 0.0f, O = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float f = s.fw[w][g];
        L = fmaf(s.sl[w][g], f, L);
        O = fmaf(s.so[w][g][d], f, O);
      }
      if (nch == 1) {
        const float v = O * (1.0f / L);
        out[((size_t)m * Hq + qh0 + g) * HD + d] = v;
        emit_group(pd, v, t & 31, ((qh0 + g) * HD + d) >> 5, m, M);
      } else {
        float *rec = rbase + g * hstride + (size_t)ch * RS;
        if (d == 0) {
          rec[0] = s.mg[g];
          rec[1] = L;
        }
        rec[2 + d] = O;
      }
    }
    __syncthreads();  // LDS is reused by the next item
  }
}

// Batch-1 decode: the attention of KV head h fused with h's K slice of the
// O projection (AttnOArgs). Workgroup (bg, h) first requests its wave's O
// weights (row block bg * NW + wave, the KQS quads of slice h) and its rows'
// residuals, then runs the attention items of row 0's context for KV head h
// (attn_f16_item over fp16 pages, attn_f32_item over f32 pages)
// (CH positions each; more than one merge in registers by log-sum-exp),
// quantises the G * hd outputs into Q8 planes in LDS exactly as the O
// projection's input planes are quantised (int4_matmul.zig:380-398), and
// each wave forms its row block's partial dot over the slice with the
// GEMV's group arithmetic ((f32(T - corr) * w_scale) * a_scale, groups in
// order). With a.y set, the group's Hkv workgroups meet at a counter: each
// publishes its partial vector (agent-scope stores, completed before a
// barrier, then the counter increment) and the last to arrive reads the
// Hkv vectors with agent-scope loads and adds them in head order, whatever
// the arrival order, so the result is reproducible.
// With the round-robin placement of workgroups on the 8 XCDs, blockIdx % Hkv
// = h puts every workgroup of one KV head on the same 8 / Hkv XCDs, whose L2s
// then serve its K/V rows after the first read.
template <int HD, int NT, int NW, bool KV32>
__global__ __launch_bounds__(64 * NW) void attn_o_kernel(AttnOArgs a) {
  constexpr int WP = 16 * NT, CH = NW * WP, NTH = 64 * NW, RG = 16 * NW;
  constexpr int KQM = kMaxGroup * HD / 128;  // quads of the largest slice
  constexpr int KO = (kMaxGroup * HD + NTH - 1) / NTH;
  static_assert(RG <= NTH, "one thread per row of the group in the epilogue");
  const int t = threadIdx.x, l = t & 63;
  const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
  const int Hkv = a.num_kv_heads;
  const int h = blockIdx.x % Hkv, bg = blockIdx.x / Hkv;
  const int G = a.num_heads / Hkv, SL = G * HD;
  const int KQ = a.K >> 7, NB = a.N >> 4;
  // slice h of the O input: groups g_first .. g_first + SG - 1, over quads
  // q_first .. q_first + KQS - 1 (4 groups a quad; with head_dim 64 the
  // first and last quad can be shared with the neighbouring slice)
  const int SG = SL >> 5, g_first = h * SG, q_first = g_first >> 2;
  const int KQS = ((g_first + SG + 3) >> 2) - q_first;
  const int nb = bg * NW + wv;
  const int n_local = l & 15, c = l >> 4;
  // the row's context and lane first: the page walk waits for them
  const int ctx = __builtin_amdgcn_readfirstlane(min(a.row0 ? a.row0[1] : a.ctx_len[0], a.max_ctx));
  const int lane = __builtin_amdgcn_readfirstlane(a.row0 ? a.row0[0] : a.lane_of_row[0]);
  // this wave's O weights (tile slot i of quads q_first + i, clamped into
  // the slice so every slot loads) and its epilogue row's residual are
  // requested once the first attention item's loads are: vector loads
  // complete in issue order, so requested earlier they would hold up the
  // page walk
  const size_t tile0 = (size_t)min(nb, NB - 1) * KQ + (size_t)q_first;
  const uint4 *cp = a.codes + tile0 * 64 + l;
  const uint16_t *sp = (const uint16_t *)a.scales + tile0 * 64 + l;
  uint4 wq[KQM];
  uint32_t wsc[KQM];
  const int r0 = bg * RG, nrows = min(RG, a.N - r0);
  float resid = 0.0f;
  auto load_weights = [&]() {
#pragma unroll
    for (int i = 0; i < KQM; ++i) {
      const int ic = min(i, KQS - 1);
      wq[i] = load_stream(cp + (size_t)ic * 64);
      wsc[i] = sp[(size_t)ic * 64];
    }
    resid = a.y ? a.resid[r0 + min(t, nrows - 1)] : 0.0f;
  };
  __shared__ AttnF16Lds<HD, NW> s;
  __shared__ __align__(16) int8_t aq[kMaxGroup * HD];
  __shared__ ActMeta am[kMaxGroup * HD / 32];
  __shared__ float wsq[NW];
  __shared__ int last;
  __shared__ __align__(16) float qs[KV32 ? kMaxGroup * HD : 4];  // f32 items' q
  float orun[KO], lrun[KO], mrun[KO];
#pragma unroll
  for (int k = 0; k < KO; ++k) {
    orun[k] = 0.0f;
    lrun[k] = 0.0f;
    mrun[k] = -INFINITY;
  }
  const int32_t *prow = a.row0 && ctx <= 16 * a.row0_pages
                            ? a.row0 + 4
                            : a.page_table + (size_t)lane * a.max_pages;
  const int nch = (ctx + CH - 1) / CH;
  if (nch == 0) load_weights();
  for (int ch = 0; ch < nch; ++ch) {
    const int j0 = ch * CH;
    const auto hook = [&]() {
      if (ch == 0) load_weights();
    };
    if constexpr (KV32)
      attn_f32_item<HD, NT, NW>(a.q + (size_t)h * SL, (const float *)a.kv_pool, prow + j0 / 16,
                                min(CH, ctx - j0), a.layer, (size_t)a.num_layers, Hkv * HD, h, G,
                                s, qs, hook);
    else
      attn_f16_item<HD, NT, NW>(a.q + (size_t)h * SL, (const __half *)a.kv_pool, prow + j0 / 16,
                                min(CH, ctx - j0), a.layer, (size_t)a.num_layers, Hkv * HD, h, G,
                                s, hook);
#pragma unroll
    for (int k = 0; k < KO; ++k) {
      const int oi = t + NTH * k;
      if (oi >= SL) break;
      const int g = oi / HD, d = oi % HD;
      float L = 0.0f, O = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float f = s.fw[w][g];
        L = fmaf(s.sl[w][g], f, L);
        O = fmaf(s.so[w][g][d], f, O);
      }
      const float mx = s.mg[g];
      if (ch == 0) {
        orun[k] = O;
        lrun[k] = L;
        mrun[k] = mx;
      } else {
        const float mn = fmaxf(mrun[k], mx);
        const float fa = expf(mrun[k] - mn), fb = expf(mx - mn);
        orun[k] = orun[k] * fa + O * fb;
        lrun[k] = lrun[k] * fa + L * fb;
        mrun[k] = mn;
      }
    }
    __syncthreads();  // s is reused by the next item
  }
  // the O projection's planes of this slice (a half-wave = one group of 32;
  // SL is a multiple of 128, so a half-wave is wholly in or out of range)
#pragma unroll
  for (int k = 0; k < KO; ++k) {
    const int oi = t + NTH * k;
    if (oi >= SL) break;
    const float v = nch > 0 ? orun[k] * (1.0f / lrun[k]) : 0.0f;
    quantize_group<1>(v, t & 31, oi >> 5, 0, 1, aq, am);
  }
  __syncthreads();
  if (nb < NB) {
    // lane (c, n): group 4 (q_first + i) + c of the input, row n of the
    // block; a group outside the slice adds exactly 0
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < KQM; ++i) {
      if (i >= KQS) break;
      const int gl = 4 * (q_first + i) + c - g_first;  // group within the slice
      const bool in = gl >= 0 && gl < SG;
      const int g = in ? gl : 0;
      const uint32_t wj[4] = {wq[i].x, wq[i].y, wq[i].z, wq[i].w};
      const int4 q0 = *(const int4 *)(aq + g * 32);
      const int4 q1 = *(const int4 *)(aq + g * 32 + 16);
      const int qa[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
      int T = 0;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        T = __builtin_amdgcn_sdot4((int)(wj[w] & 0x0F0F0F0Fu), qa[2 * w], T, false);
        T = __builtin_amdgcn_sdot4((int)((wj[w] >> 4) & 0x0F0F0F0Fu), qa[2 * w + 1], T, false);
      }
      const ActMeta mm = am[g];
      const float v = (float)(T - mm.corr);
      float tt = v * h2f(wsc[i]);
      tt = tt * mm.scale;
      acc += in ? tt : 0.0f;
    }
    acc = xor32_add(xor16_add(acc));
    // agent-scope store: written through to the level all XCDs read (see
    // the publication below)
    if (c == 0)
      __hip_atomic_store(a.parts + (size_t)h * a.N + nb * 16 + n_local, acc, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
  if (!a.y) return;
  // Cross-workgroup publication of the Hkv slices. In the HIP language model
  // this needs an agent-scope release on the counter increment and an
  // agent-scope acquire in the last arriver; on gfx950 those lower to a
  // write-back of the whole L2 and an L2 invalidate (measured +4.6 us per
  // launch). The merge instead rests on how the gfx942-family memory model
  // of the AMDGPU backend lowers agent-scope atomics, an ISA-level contract:
  //  (1) an agent-scope atomic store carries the device scope bits, so the
  //      XCD's L2 writes it through to the memory-side level every XCD
  //      reads; (2) a store counts in vmcnt until that write is
  //      acknowledged, so s_waitcnt vmcnt(0) returns only when every partial
  //      row of this wave is there; (3) an agent-scope atomic load carries
  //      the same scope bits and reads that level, never a stale L2 line.
  // The counter (an agent-scope read-modify-write, coherent across XCDs in
  // any lowering) is incremented only after every wave of the workgroup has
  // passed (2) (the barrier below), so the last arriver's loads (3) see all
  // Hkv slices. The built code shows the lowering: the slice stores and the
  // merge loads are global_store_dword / global_load_dword with sc1. Plain stores or loads of `parts`, or dropping the wait,
  // would break it; the workgroup-scope fences only keep the compiler from
  // moving the accesses across the barrier.
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __syncthreads();
  if (t == 0)
    last = __hip_atomic_fetch_add(a.counters + bg, 1u, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(Hkv - 1);
  __syncthreads();
  if (!last) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  float y = 0.0f;
  if (t < nrows) {
    const int n = r0 + t;
    float pv[kMaxAttnOHeads];  // every slice requested before the first add
#pragma unroll
    for (int h2 = 0; h2 < kMaxAttnOHeads; ++h2)
      pv[h2] = h2 < Hkv ? __hip_atomic_load(a.parts + (size_t)h2 * a.N + n, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT)
                        : 0.0f;
    float p = pv[0];
#pragma unroll
    for (int h2 = 1; h2 < kMaxAttnOHeads; ++h2)
      if (h2 < Hkv) p += pv[h2];
    y = resid + p;
    a.y[n] = y;
  }
  const float sq = wave_sum(y * y);
  if (l == 0) wsq[wv] = sq;
  __syncthreads();
  if (t == 0) {
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) tot += wsq[w];
    a.ss_out[bg] = tot;
    // ready for the next launch
    __hip_atomic_store(a.counters + bg, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Merge the chunk records of one (query head, row): every thread of the
// workgroup takes part in each step and issues all of its record loads of a
// step before using them, so the record count costs a few parallel memory
// round trips, not a serial chain.
static constexpr int kCombineThreads = 512;
template <int HD>
__global__ __launch_bounds__(kCombineThreads) void attn_combine2_kernel(
    const int32_t *ctx_len, int Hq, int chunk, int n_chunks_max, int max_ctx,
    const float *scratch, float *out, PlanesDst pd) {
  constexpr int NTH = kCombineThreads, NG = NTH / HD, U = 8, RPT = kMaxRecords / NTH;
  const int qh = blockIdx.x, m = blockIdx.y, t = threadIdx.x;
  const int ctx = min(ctx_len[m], max_ctx);
  const int nch = (ctx + chunk - 1) / chunk;
  if (nch <= 1) return;
  const float *rec0 = scratch + ((size_t)m * Hq + qh) * n_chunks_max * (2 + HD);
  __shared__ float f[kMaxRecords];
  __shared__ float redm[NTH / 64], redl[NTH / 64];
  __shared__ float part[NG][HD];
  float mc[RPT], lc[RPT];
  float mx = -INFINITY;
#pragma unroll
  for (int u = 0; u < RPT; ++u) {
    const int c = t + NTH * u;
    mc[u] = c < nch ? rec0[(size_t)c * (2 + HD)] : -INFINITY;
    lc[u] = c < nch ? rec0[(size_t)c * (2 + HD) + 1] : 0.0f;
    mx = fmaxf(mx, mc[u]);
  }
  mx = wave_max(mx);
  if ((t & 63) == 0) redm[t >> 6] = mx;
  __syncthreads();
  float M = redm[0];
#pragma unroll
  for (int w = 1; w < NTH / 64; ++w) M = fmaxf(M, redm[w]);
  float lp = 0.0f;
#pragma unroll
  for (int u = 0; u < RPT; ++u) {
    const int c = t + NTH * u;
    if (c < nch) {
      const float fc = expf(mc[u] - M);
      f[c] = fc;
      lp = fmaf(lc[u], fc, lp);
    }
  }
  lp = wave_sum(lp);
  if ((t & 63) == 0) redl[t >> 6] = lp;
  __syncthreads();
  float L = 0.0f;
#pragma unroll
  for (int w = 0; w < NTH / 64; ++w) L += redl[w];
  const int d = t % HD, g = t / HD;
  float o[U];
#pragma unroll
  for (int u = 0; u < U; ++u) o[u] = 0.0f;
  for (int c0 = g; c0 < nch; c0 += NG * U) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + NG * u;
      v[u] = c < nch ? rec0[(size_t)c * (2 + HD) + 2 + d] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + NG * u;
      if (c < nch) o[u] = fmaf(v[u], f[c], o[u]);
    }
  }
  float tot = 0.0f;
#pragma unroll
  for (int u = 0; u < U; ++u) tot += o[u];
  part[g][d] = tot;
  __syncthreads();
  if (g == 0) {
    float acc = part[0][d];
#pragma unroll
    for (int i = 1; i < NG; ++i) acc += part[i][d];
    const float v = acc * (1.0f / L);
    out[((size_t)m * Hq + qh) * HD + d] = v;
    emit_group(pd, v, t & 31, (qh * HD + d) >> 5, m, (int)gridDim.y);
  }
}

hipError_t launch_attention_f16(const float *q, const void *kv_pool, const int32_t *page_table,
                                int max_pages, const int32_t *lane_of_row, const int32_t *ctx_len,
                                int M, int layer, int num_layers, int num_heads, int num_kv_heads,
                                int head_dim, int max_ctx, float *scratch, float *out,
                                hipStream_t st, int wp, int nw, PlanesDst emit) {
  if (num_heads % num_kv_heads != 0 || num_heads / num_kv_heads > kMaxGroup || M < 1 || M > 64 ||
      max_ctx < 1)
    return hipErrorInvalidValue;
  const int chunk = wp * nw;
  if (chunk < kF16MinChunk || wp % 16) return hipErrorInvalidValue;
  const int nch = (max_ctx + chunk - 1) / chunk;  // record slots per (row, query head)
  if (nch > kMaxRecords) return hipErrorInvalidValue;
  // one workgroup per work item up to a cap; the rest loop over the list
  const long items = (long)nch * num_kv_heads * M;
  const unsigned grid = (unsigned)std::min<long>(items, kAttnMaxGrid);
  const __half *pool = (const __half *)kv_pool;
#define GK_F16(HD, NT, NW)                                                                   \
  hipLaunchKernelGGL((attn_f16_kernel<HD, NT, NW>), dim3(grid), dim3(64 * NW), 0, st, q, pool, \
                     page_table, max_pages, lane_of_row, ctx_len, M, layer, num_layers,      \
                     num_heads, num_kv_heads, nch, max_ctx, scratch, out, emit)
#define GK_F16_HD(NT, NW)                                        \
  do {                                                          \
    if (head_dim == 64) GK_F16(64, NT, NW);                     \
    else if (head_dim == 128) GK_F16(128, NT, NW);              \
    else return hipErrorInvalidValue;                           \
  } while (0)
  if (wp == 16 && nw == 4) GK_F16_HD(1, 4);
  else if (wp == 16 && nw == 8) GK_F16_HD(1, 8);
  else if (wp == 16 && nw == 16) GK_F16_HD(1, 16);
  else if (wp == 32 && nw == 4) GK_F16_HD(2, 4);
  else if (wp == 32 && nw == 8) GK_F16_HD(2, 8);
  else return hipErrorInvalidValue;
#undef GK_F16_HD
#undef GK_F16
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || nch <= 1) return e;
  if (head_dim == 64)
    hipLaunchKernelGGL((attn_combine2_kernel<64>), dim3(num_heads, M), dim3(kCombineThreads), 0,
                       st, ctx_len, num_heads, chunk, nch, max_ctx, scratch, out, emit);
  else
    hipLaunchKernelGGL((attn_combine2_kernel<128>), dim3(num_heads, M), dim3(kCombineThreads), 0,
                       st, ctx_len, num_heads, chunk, nch, max_ctx, scratch, out, emit);
  return hipGetLastError();
}

static constexpr int kAttnONT = 2, kAttnONW = 8;  // 256 positions per item

int attn_o_groups(int N) { return (N / 16 + kAttnONW - 1) / kAttnONW; }

bool attn_o_ok(const AttnOArgs &a) {
  const int hd = a.head_dim;
  if ((hd != 64 && hd != 128) || a.num_kv_heads < 1 || a.num_kv_heads > kMaxAttnOHeads ||
      a.num_heads % a.num_kv_heads)
    return false;
  const int G = a.num_heads / a.num_kv_heads;
  if (a.y && (!a.resid || !a.ss_out || !a.counters)) return false;
  // every slice is whole 32-column groups on at most the quads a workgroup
  // holds (kMaxGroup * hd / 128)
  const int SG = G * hd / 32;
  for (int h = 0; h < a.num_kv_heads; ++h)
    if ((h * SG + SG + 3) / 4 - (h * SG) / 4 > kMaxGroup * hd / 128) return false;
  return G <= kMaxGroup && (G * hd) % 32 == 0 && a.K == a.num_heads * hd && a.N > 0 &&
         a.N % 16 == 0 && a.max_ctx >= 1 && a.max_pages >= 1 && a.codes && a.scales && a.parts &&
         a.q && a.kv_pool && a.page_table && a.lane_of_row && a.ctx_len;
}

hipError_t launch_attn_o(const AttnOArgs &a, hipStream_t st) {
  if (!attn_o_ok(a)) return hipErrorInvalidValue;
  const unsigned grid = (unsigned)(attn_o_groups(a.N) * a.num_kv_heads);
#define GK_ATTN_O(HD, KV32) \
  hipLaunchKernelGGL((attn_o_kernel<HD, kAttnONT, kAttnONW, KV32>), dim3(grid), \
                     dim3(64 * kAttnONW), 0, st, a)
  if (a.head_dim == 64) {
    if (a.kv_f32) GK_ATTN_O(64, true); else GK_ATTN_O(64, false);
  } else {
    if (a.kv_f32) GK_ATTN_O(128, true); else GK_ATTN_O(128, false);
  }
#undef GK_ATTN_O
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// K3b: causal prefill attention over one lane's chunk of T consecutive
// positions pos0 .. pos0 + T - 1 (generate.zig:1511-1967 per row: softmax of
// q . k / sqrt(hd) over the row's positions 0 .. pos, then the weighted sum
// of v), fp16 KV pages.
//
// Workgroup = the G query heads of one KV head (one wave each) x 16 query
// rows; it walks the key pages 0 .. (last row's position) / 16, staging each
// page's K rows and V (transposed) in LDS, double buffered, one barrier per
// page, so the G waves share every K/V read. Per page and wave:
//   * S^T = K . Q^T as one 16 x 16 tile (keys x rows) with f16 MFMAs; Q is
//     split into f16 hi + lo parts (K is exact in f16), so the scores carry
//     f32 accuracy like the decode kernel's;
//   * online softmax per row (column of S^T: the 16 keys of row j sit in
//     lanes (c, j), c = 0..3, four per lane), causal mask on the diagonal;
//   * O += P . V with P split into f16 hi + lo (the tile's A operand is the
//     lane's own P registers) and V^T from LDS; O (16 rows x hd, f32) stays
//     in registers, rescaled by each row's exp(m_old - m_new).
// The last blocks (longest key ranges) are scheduled first. PPT: 16-byte
// K (and V) pieces each thread stages per page (16 * hd / 8 pieces over
// 64 * G threads).
template <int HD, int PPT>
__global__ __launch_bounds__(64 * kMaxGroup) void attn_prefill_kernel(
    const float *q, const __half *pool, const int32_t *ptab, int pos0, int T, int layer,
    int num_layers, int Hq, int Hkv, float *out) {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  typedef float f4 __attribute__((ext_vector_type(4)));
  constexpr int S = HD / 16;   // 16-wide steps over the head dim (scores)
  constexpr int NT = HD / 16;  // 16-wide output tiles over the head dim
  constexpr int KP = HD + 8;   // K row stride in halves (padded)
  constexpr int VP = 16 + 4;   // V^T row stride in halves (padded)
  constexpr int PIECES = 16 * HD / 8;  // 16-byte pieces of one page's K (or V)
  __shared__ __align__(16) _Float16 ks[2][16 * KP];
  __shared__ __align__(16) _Float16 vt[2][HD * VP];
  const int t = threadIdx.x, l = t & 63;
  const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
  const int c = l >> 4, j = l & 15;
  const int G = Hq / Hkv;
  const int nqb = (T + 15) / 16;
  const int i0 = (nqb - 1 - (int)blockIdx.x) * 16;  // longest blocks first
  const int h = blockIdx.y;
  const int qh = h * G + wv;
  const int kv_dim = Hkv * HD;
  const size_t lay = (size_t)num_layers;
  const int last_pos = pos0 + min(i0 + 15, T - 1);
  const int npages = last_pos / 16 + 1;
  const float scale = 1.0f / sqrtf((float)HD);

  // staging: thread t moves K and V pieces t + 64 G i (i < PPT) of a page;
  // key positions past the last row's are zeroed (their page slots may hold
  // anything, and a masked score still multiplies its V row)
  const int nthr = (int)blockDim.x;
  uint4 kreg[PPT], vreg[PPT];
  auto fetch = [&](int kp) {
    const size_t pbase = ((size_t)ptab[kp] * lay + layer) * 2;
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int pc = t + nthr * i, skey = pc / (HD / 8), spc = pc % (HD / 8);
      kreg[i] = vreg[i] = make_uint4(0, 0, 0, 0);
      if (pc < PIECES && 16 * kp + skey <= last_pos) {
        const size_t off = (pbase * 16 + skey) * kv_dim + (size_t)h * HD + 8 * spc;
        kreg[i] = *(const uint4 *)(pool + off);
        vreg[i] = *(const uint4 *)(pool + off + 16 * (size_t)kv_dim);
      }
    }
  };
  auto stage = [&](int b) {
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int pc = t + nthr * i, skey = pc / (HD / 8), spc = pc % (HD / 8);
      if (pc >= PIECES) continue;
      *(uint4 *)&ks[b][skey * KP + 8 * spc] = kreg[i];
      const _Float16 *vh = (const _Float16 *)&vreg[i];
#pragma unroll
      for (int e = 0; e < 8; ++e) vt[b][(8 * spc + e) * VP + skey] = vh[e];
    }
  };
  fetch(0);
  stage(0);

  // Q^T as the B operand: lane (c, j) = row i0 + j, dims 16 st + 4c .. + 3
  h4 qhi[S], qlo[S];
  {
    const float *qrow = q + ((size_t)min(i0 + j, T - 1) * Hq + qh) * HD;
#pragma unroll
    for (int st = 0; st < S; ++st) {
      const float4 qv = *(const float4 *)(qrow + 16 * st + 4 * c);
      const float qa[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const _Float16 hv = (_Float16)qa[e];
        qhi[st][e] = hv;
        qlo[st][e] = (_Float16)(qa[e] - (float)hv);
      }
    }
  }
  const int qpos = pos0 + i0 + j;  // position of this lane's score column
  f4 o[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) o[nt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  float mx = -INFINITY, sum = 0.0f;
  __syncthreads();

  for (int kp = 0; kp < npages; ++kp) {
    const int b = kp & 1;
    if (kp + 1 < npages) fetch(kp + 1);  // next page in flight
    // scores S^T[key 4c + r][row j]; every K fragment is read from LDS
    // before the first MFMA (one LDS round trip a page, not one a step)
    h4 kf[S];
#pragma unroll
    for (int st = 0; st < S; ++st) kf[st] = *(const h4 *)&ks[b][j * KP + 16 * st + 4 * c];
    __builtin_amdgcn_sched_barrier(0);  // (the scheduler would sink them again)
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int st = 0; st < S; ++st) {
      acc = __builtin_amdgcn_mfma_f32_16x16x16f16(kf[st], qhi[st], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x16f16(kf[st], qlo[st], acc, 0, 0, 0);
    }
    // the V fragments do not depend on the softmax: requested before it
    __builtin_amdgcn_sched_barrier(0);
    h4 vf[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) vf[nt] = *(const h4 *)&vt[b][(16 * nt + j) * VP + 4 * c];
    __builtin_amdgcn_sched_barrier(0);
    float sv[4], pm = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int kpos = 16 * kp + 4 * c + r;
      sv[r] = kpos <= qpos ? acc[r] * scale : -INFINITY;
      pm = fmaxf(pm, sv[r]);
    }
    pm = xor32_max(xor16_max(pm));
    const float mnew = fmaxf(mx, pm);  // finite: key 0 is in every row's range
    const float alpha = expf(mx - mnew);
    h4 phi, plo;
    float ps = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float pv = expf(sv[r] - mnew);
      ps += pv;
      const _Float16 hv = (_Float16)pv;
      phi[r] = hv;
      plo[r] = (_Float16)(pv - (float)hv);
    }
    ps = xor32_add(xor16_add(ps));
    sum = sum * alpha + ps;
    mx = mnew;
    // O rows are rows 4c + r: their factors live in lanes 4c + r
    float ar[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) ar[r] = __shfl(alpha, 4 * c + r);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
      for (int r = 0; r < 4; ++r) o[nt][r] *= ar[r];
      o[nt] = __builtin_amdgcn_mfma_f32_16x16x16f16(phi, vf[nt], o[nt], 0, 0, 0);
      o[nt] = __builtin_amdgcn_mfma_f32_16x16x16f16(plo, vf[nt], o[nt], 0, 0, 0);
    }
    // publish the next page (the other buffer was last read before the
    // previous barrier)
    if (kp + 1 < npages) stage(b ^ 1);
    __syncthreads();
  }
  // lane (c, j): O[row 4c + r][dim 16 nt + j]
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = i0 + 4 * c + r;
    const float lr = __shfl(sum, 4 * c + r);
    if (row < T) {
      float *orow = out + ((size_t)row * Hq + qh) * HD;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) orow[16 * nt + j] = o[nt][r] / lr;
    }
  }
}

hipError_t launch_attention_prefill(const float *q, const void *kv_pool, const int32_t *page_table,
                                    int max_pages, int lane, int pos0, int T, int layer,
                                    int num_layers, int num_heads, int num_kv_heads, int head_dim,
                                    float *out, hipStream_t st) {
  if (T < 1 || lane < 0 || pos0 < 0 || num_heads % num_kv_heads != 0 ||
      num_heads / num_kv_heads > kMaxGroup || (pos0 + T + 15) / 16 > max_pages)
    return hipErrorInvalidValue;
  const int G = num_heads / num_kv_heads;
  if (head_dim != 64 && head_dim != 128) return hipErrorInvalidValue;
  const dim3 grid((T + 15) / 16, num_kv_heads), block(64 * G);
  const int32_t *ptab = page_table + (size_t)lane * max_pages;
  const __half *pool = (const __half *)kv_pool;
  const int ppt = (16 * head_dim / 8 + 64 * G - 1) / (64 * G);
#define GK_PF(HD, P)                                                                              hipLaunchKernelGGL((attn_prefill_kernel<HD, P>), grid, block, 0, st, q, pool, ptab, pos0, T,                      layer, num_layers, num_heads, num_kv_heads, out)
  if (head_dim == 64) {
    if (ppt <= 1) GK_PF(64, 1); else GK_PF(64, 2);
  } else {
    if (ppt <= 1) GK_PF(128, 1); else if (ppt == 2) GK_PF(128, 2); else GK_PF(128, 4);
  }
#undef GK_PF
  return hipGetLastError();
}

hipError_t launch_attention(const float *q, const void *kv_pool, int kv_f16,
                            const int32_t *page_table, int max_pages, const int32_t *lane_of_row,
                            const int32_t *ctx_len, int M, int layer, int num_layers,
                            int num_heads, int num_kv_heads, int head_dim, int max_ctx,
                            float *scratch, float *out, hipStream_t st, PlanesDst emit) {
  if (num_heads % num_kv_heads != 0 || num_heads / num_kv_heads > kMaxGroup)
    return hipErrorInvalidValue;
  if (kv_f16) {
    // contexts up to 256 positions: one work item per (row, KV head) of 8
    // waves x 2 pages, no combine launch; longer ones: 64-position items of
    // 4 waves x 1 page for few (row, KV head) pairs (batch-1 decode), else
    // 128-position items of 4 waves x 2 pages (measured at 1-32 rows,
    // contexts 16-8192)
    int wp = 32, nw = 8;
    if (max_ctx > 256) {
      wp = M * num_kv_heads < 16 ? 16 : 32;
      nw = 4;
    }
    return launch_attention_f16(q, kv_pool, page_table, max_pages, lane_of_row, ctx_len, M, layer,
                                num_layers, num_heads, num_kv_heads, head_dim, max_ctx, scratch,
                                out, st, wp, nw, emit);
  }
  const int chunk = attention_chunk(max_ctx, num_kv_heads, M);
  if ((max_ctx + chunk - 1) / chunk > kMaxRecords) return hipErrorInvalidValue;
  const int nch = (max_ctx + chunk - 1) / chunk;
  // few workgroups (batch-1 decode, f32 KV): one query head each; fp16 KV
  // always groups the query heads of a KV head (MFMA scores)
  const bool per_head = !kv_f16 && nch * num_kv_heads * M < 64;
  dim3 grid(nch, per_head ? num_heads : num_kv_heads, M);
#define GK_ATT(HD, F)                                                                           \
  do {                                                                                          \
    if (per_head)                                                                               \
      hipLaunchKernelGGL((attn_decode_kernel<HD, F, 1>), grid, dim3(256), 0, st, q, kv_pool,    \
                         page_table, max_pages, lane_of_row, ctx_len, layer, num_layers,        \
                         num_heads, num_kv_heads, chunk, nch, max_ctx, scratch, out, emit);     \
    else                                                                                        \
      hipLaunchKernelGGL((attn_decode_kernel<HD, F, kMaxGroup>), grid, dim3(256), 0, st, q,     \
                         kv_pool, page_table, max_pages, lane_of_row, ctx_len, layer,           \
                         num_layers, num_heads, num_kv_heads, chunk, nch, max_ctx, scratch, out, \
                         emit);                                                                 \
  } while (0)
  if (head_dim == 64) {
    if (kv_f16) GK_ATT(64, 1); else GK_ATT(64, 0);
  } else if (head_dim == 128) {
    if (kv_f16) GK_ATT(128, 1); else GK_ATT(128, 0);
  } else {
    return hipErrorInvalidValue;
  }
#undef GK_ATT
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || nch <= 1) return e;
  if (head_dim == 64)
    hipLaunchKernelGGL((attn_combine2_kernel<64>), dim3(num_heads, M), dim3(kCombineThreads), 0, st, ctx_len,
                       num_heads, chunk, nch, max_ctx, scratch, out, emit);
  else
    hipLaunchKernelGGL((attn_combine2_kernel<128>), dim3(num_heads, M), dim3(kCombineThreads), 0, st,
                       ctx_len, num_heads, chunk, nch, max_ctx, scratch, out, emit);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// K5: argmax / eligible argmax
// ---------------------------------------------------------------------------
// Candidate order and merge: arg_better / arg_merge (epilogue.h). A block
// owns 8192 logits of one row; each thread issues all 32 of its loads (and
// the block's 128 mask words go to LDS) before comparing, so a block costs
// one memory round trip. The last block of a row (atomic counter, which it
// resets) merges the row's partials and writes the result.
static constexpr int kArgBlock = 256;
static constexpr int kArgPerBlock = 8192;  // 128 mask words per block

size_t argmax_scratch_bytes(int rows, long n) {
  const long blocks = (n + kArgPerBlock - 1) / kArgPerBlock;
  return (size_t)rows * blocks * sizeof(ArgPartial);
}

static __device__ __forceinline__ ArgPartial arg_none() {
  ArgPartial p;
  p.v = 0.0f;
  p.i = -1;
  p.nan_flag = 0;
  p.rows = 0;
  p.bad_mask = 0;
  p.nan0 = 0;
  return p;
}

// Reduce one partial per thread over a 256-thread block; thread 0 gets it.
static __device__ ArgPartial arg_block_reduce(ArgPartial p) {
  __shared__ ArgPartial wpart[kArgBlock / 64];
  const int t = threadIdx.x;
  for (int o = 32; o > 0; o >>= 1) arg_merge(p, arg_shfl_xor(p, o));
  __syncthreads();  // wpart may still be read by a previous call
  if ((t & 63) == 0) wpart[t >> 6] = p;
  __syncthreads();
  ArgPartial r = wpart[0];
  for (int w = 1; w < kArgBlock / 64; ++w) arg_merge(r, wpart[w]);
  return r;
}

static __device__ void arg_write_result(const ArgPartial &r, bool masked, long n,
                                        ArgmaxResult *res_out) {
  ArgmaxResult res;
  res.pad = 0;
  if (masked) {
    res.eligible_rows = r.rows;
    if (r.bad_mask || r.rows == 0 || r.rows > (unsigned long long)n) {
      res.status = 6;  // GLACIER_HIP_INVALID_MASK
      res.index = 0;
    } else if (r.nan_flag) {
      res.status = 7;  // GLACIER_HIP_ELIGIBLE_NAN
      res.index = 0;
    } else {
      res.status = 0;
      res.index = (uint64_t)r.i;
    }
  } else {
    res.eligible_rows = (uint64_t)n;
    res.status = 0;
    // a NaN at index 0 is the initial best and is never displaced
    res.index = (r.nan0 || r.i < 0) ? 0 : (uint64_t)r.i;
  }
  *res_out = res;
}

__global__ __launch_bounds__(kArgBlock) void argmax_kernel(const float *logits, long n,
                                                           const uint64_t *words,
                                                           long word_count,
                                                           ArgPartial *parts,
                                                           uint32_t *counters,
                                                           ArgmaxResult *result) {
  constexpr int PER = kArgPerBlock / kArgBlock;
  const int row = blockIdx.y, blk = blockIdx.x, t = threadIdx.x;
  const long nblocks = gridDim.x;
  const float *lr = logits + (size_t)row * n;
  const uint64_t *wr = words ? words + (size_t)row * word_count : nullptr;
  const long e0 = (long)blk * kArgPerBlock, e1 = min(n, e0 + kArgPerBlock);
  __shared__ uint64_t sw[kArgPerBlock / 64];
  __shared__ int last;
  uint64_t myword = 0;
  if (wr && t < kArgPerBlock / 64) {
    const long wi = (e0 >> 6) + t;
    myword = wi < word_count ? wr[wi] : 0ull;
  }
  float v[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const long e = e0 + t + (long)kArgBlock * u;
    v[u] = e < e1 ? lr[e] : 0.0f;
  }
  if (wr && t < kArgPerBlock / 64) sw[t] = myword;
  __syncthreads();
  ArgPartial p = arg_none();
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const long e = e0 + t + (long)kArgBlock * u;
    if (e >= e1) break;
    if (wr && !((sw[(e - e0) >> 6] >> (e & 63)) & 1ull)) continue;
    if (isnan(v[u])) p.nan_flag = 1;
    if (arg_better(v[u], e, p.v, p.i)) {
      p.v = v[u];
      p.i = e;
    }
  }
  if (blk == 0 && t == 0 && isnan(v[0])) p.nan0 = 1;
  if (wr && t < kArgPerBlock / 64) {
    const long wi = (e0 >> 6) + t, w1 = (e1 + 63) >> 6;
    if (wi < w1) p.rows = __popcll(myword);
    if (wi == word_count - 1 && (n & 63) && (myword & ~((1ull << (n & 63)) - 1ull)))
      p.bad_mask = 1;
  }
  const ArgPartial bp = arg_block_reduce(p);
  if (t == 0) {
    parts[(size_t)row * nblocks + blk] = bp;
    __threadfence();
    last = atomicAdd(&counters[row], 1u) == (unsigned)(nblocks - 1);
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  ArgPartial q = arg_none();
  for (long b = t; b < nblocks; b += kArgBlock) arg_merge(q, parts[(size_t)row * nblocks + b]);
  const ArgPartial r = arg_block_reduce(q);
  if (t == 0) {
    counters[row] = 0u;
    arg_write_result(r, wr != nullptr, n, &result[row]);
  }
}

hipError_t launch_argmax(const float *logits, long n, int rows, const uint64_t *words,
                         long word_count, void *scratch, uint32_t *counters,
                         ArgmaxResult *result, hipStream_t st) {
  const long blocks = (n + kArgPerBlock - 1) / kArgPerBlock;
  hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)blocks, rows), dim3(kArgBlock), 0, st,
                     logits, n, words, word_count, (ArgPartial *)scratch, counters, result);
  return hipGetLastError();
}

// Fused-head finisher: one block per row merges the candidates the head
// GEMV wrote and, for the eligible variant, counts the mask bits and checks
// those beyond n; all loads of a pass are issued before they are used.
__global__ __launch_bounds__(kArgBlock) void argmax_parts_kernel(const ArgPartial *parts,
                                                                 int nparts, long n,
                                                                 const uint64_t *words,
                                                                 long word_count,
                                                                 ArgmaxResult *result) {
  constexpr int U = 8;
  const int row = blockIdx.x, t = threadIdx.x;
  const ArgPartial *pr = parts + (size_t)row * nparts;
  const uint64_t *wr = words ? words + (size_t)row * word_count : nullptr;
  ArgPartial p = arg_none();
  for (int base = 0; base < nparts; base += kArgBlock * U) {
    ArgPartial q[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = base + t + kArgBlock * u;
      q[u] = i < nparts ? pr[i] : arg_none();
    }
#pragma unroll
    for (int u = 0; u < U; ++u) arg_merge(p, q[u]);
  }
  if (wr) {
    for (long base = 0; base < word_count; base += (long)kArgBlock * U) {
      uint64_t w[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const long i = base + t + (long)kArgBlock * u;
        w[u] = i < word_count ? wr[i] : 0ull;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const long i = base + t + (long)kArgBlock * u;
        if (i < (n + 63) / 64) p.rows += __popcll(w[u]);
        if (i == word_count - 1 && (n & 63) && (w[u] & ~((1ull << (n & 63)) - 1ull)))
          p.bad_mask = 1;
      }
    }
  }
  const ArgPartial r = arg_block_reduce(p);
  if (t == 0) arg_write_result(r, wr != nullptr, n, &result[row]);
}

int gemv_argmax_parts(int N, int K, int M, int D) {
  // the grid of the fused-head launch itself (gemv_shape adjusts the plain
  // plan per path); the shape only tests these pointers for null
  static int8_t q_tag;
  static ActMeta meta_tag;
  static float y_tag;
  static ArgPartial part_tag;
  GemvArgs a{};
  a.N = N;
  a.K = K;
  a.M = M;
  a.D = D;
  a.epi = EPI_PLAIN;
  a.act_q = &q_tag;
  a.act_meta = &meta_tag;
  a.y = &y_tag;
  a.arg_parts = &part_tag;
  GemvShape p;
  return gemv_shape(a, p) ? p.grid : -1;
}

hipError_t launch_argmax_parts(const ArgPartial *parts, int nparts, long n, int rows,
                               const uint64_t *words, long word_count, ArgmaxResult *result,
                               hipStream_t st) {
  if (rows <= 0 || nparts <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(argmax_parts_kernel, dim3(rows), dim3(kArgBlock), 0, st, parts, nparts, n,
                     words, word_count, result);
  return hipGetLastError();
}

}  // namespace gk
