// kernels.hip — hand-written gfx950 kernels for Glacier's text token loop.
//
//  K1  gemv_kernel     INT4 x (Q8 | f32-as-3-digit) GEMV on v_mfma_i32_16x16x32_i8,
//                      split-K with a deterministic last-arriving finisher and
//                      fused epilogues (residual, SwiGLU, RoPE + paged KV write).
//  K4  prep_act_kernel RMSNorm (kernels.zig:141-220) fused with the activation
//                      quantiser (int4_matmul.zig:380-398).
//  K3  attn_*          paged-KV GQA decode attention (split over context chunks).
//  K5  argmax_*        wavefront masked argmax (sampling.zig:55-105, :194-206).
//
// Compiled with -ffp-contract=off so that the element-wise f32 arithmetic
// rounds where the reference rounds; explicit fmaf() marks the places where a
// fused multiply-add is intended.
#include "kernels.h"

#include <hip/hip_fp16.h>
#include <math.h>

namespace gk {

typedef int v4i __attribute__((ext_vector_type(4)));

static __device__ __forceinline__ float h2f(uint32_t bits16) {
  return __half2float(__ushort_as_half((unsigned short)bits16));
}

// Eight 4-bit codes of one u32 -> eight int8 lanes k0..k7 (low nibbles are
// k0..k3, high nibbles k4..k7 in the device tile layout).
static __device__ __forceinline__ long unpack_codes(uint32_t w) {
  uint32_t lo = w & 0x0F0F0F0Fu;
  uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;
  return (long)(((uint64_t)hi << 32) | (uint64_t)lo);
}

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

template <int D>
__global__ __launch_bounds__(256) void prep_act_kernel(const void *x, int x_bf16,
                                                       const float *norm_w, float eps, int M,
                                                       int K, int8_t *act_q, ActMeta *meta,
                                                       float *normed_out) {
  const int m = blockIdx.x;
  const int t = threadIdx.x;
  const size_t row = (size_t)m * K;
  __shared__ float red[8];
  float inv = 1.0f;
  if (norm_w) {
    float ss = 0.0f;
    for (int i = t; i < K; i += 256) {
      float v = load_x(x, x_bf16, row + i);
      ss = fmaf(v, v, ss);
    }
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
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
  for (int g = half; g < G; g += 8) {
    const int k = (g << 5) + hl;
    float v = load_x(x, x_bf16, row + k);
    if (norm_w) {
      float tt = v * inv;
      v = tt * norm_w[k];
    }
    if (normed_out) normed_out[row + k] = v;
    float amax = fabsf(v);
    for (int o = 16; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 32));
    const float scale = amax / 127.0f;
    const float inv_s = scale == 0.0f ? 0.0f : 1.0f / scale;
    const float y = v * inv_s;
    float q0f = roundf(y);
    q0f = fminf(fmaxf(q0f, -127.0f), 127.0f);
    int q0 = (int)q0f;
    int qd[3] = {q0, 0, 0};
    if (D == 3) {
      float r1 = (y - q0f) * 128.0f;
      float q1f = roundf(r1);
      float r2 = (r1 - q1f) * 128.0f;
      float q2f = roundf(r2);
      qd[1] = (int)q1f;
      qd[2] = (int)q2f;
    }
    int sum = 0;
#pragma unroll
    for (int d = 0; d < D; ++d) {
      act_q[(((size_t)g * D + d) * M + m) * 32 + hl] = (int8_t)qd[d];
      int sd = qd[d];
      for (int o = 16; o > 0; o >>= 1) sd += __shfl_xor(sd, o, 32);
      sum = sum * 128 + sd;
    }
    if (hl == 0) {
      ActMeta mm;
      mm.scale = D == 3 ? scale * (1.0f / 16384.0f) : scale;
      mm.corr = 7 * sum;
      meta[(size_t)g * M + m] = mm;
    }
  }
}

hipError_t launch_prep_act(const void *x, int x_bf16, const float *norm_w, float eps, int M,
                           int K, int D, int8_t *act_q, ActMeta *meta, float *normed_out,
                           hipStream_t st) {
  if (D == 1)
    hipLaunchKernelGGL(prep_act_kernel<1>, dim3(M), dim3(256), 0, st, x, x_bf16, norm_w, eps,
                       M, K, act_q, meta, normed_out);
  else
    hipLaunchKernelGGL(prep_act_kernel<3>, dim3(M), dim3(256), 0, st, x, x_bf16, norm_w, eps,
                       M, K, act_q, meta, normed_out);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// K1: INT4 GEMV on i8 MFMA
// ---------------------------------------------------------------------------
static constexpr int kLdsBudget = 40 * 1024;

static size_t act_slice_bytes(int quads, int M, int D) {
  return (size_t)quads * 4 * ((size_t)D * M * 32 + (size_t)M * sizeof(ActMeta));
}

int choose_splits(int NB, int KQ, int M) {
  // Enough waves to cover 256 CUs x 8, at least two quads per split, and
  // an activation slice that fits the LDS budget.
  int S = (2048 + NB - 1) / NB;
  int max_s = KQ >= 4 ? KQ / 2 : 1;
  if (S > max_s) S = max_s;
  if (S < 1) S = 1;
  while (S < KQ && act_slice_bytes((KQ + S - 1) / S, M, 3) > (size_t)kLdsBudget) ++S;
  return S;
}

static __device__ __forceinline__ float silu_mul(float g, float u) {
  // kernels.zig:465-520: g * (1 / (1 + exp(-g))) * u
  float sig = 1.0f / (1.0f + expf(-g));
  float t = g * sig;
  return t * u;
}

template <int D, int MT>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int NB = a.N >> 4, KQ = a.K >> 7;
  const int s = blockIdx.y;
  const int kq0 = (s * KQ) / a.S, kq1 = ((s + 1) * KQ) / a.S;
  const int nq = kq1 - kq0;
  const int M = a.M;

  // Stage this split's activation slice in LDS.
  const size_t qbytes = (size_t)nq * 4 * D * M * 32;
  const size_t mbytes = (size_t)nq * 4 * M * sizeof(ActMeta);
  {
    const uint4 *src = (const uint4 *)(a.act_q + (size_t)kq0 * 4 * D * M * 32);
    uint4 *dst = (uint4 *)smem;
    for (size_t i = threadIdx.x; i < qbytes / 16; i += 256) dst[i] = src[i];
    const uint2 *msrc = (const uint2 *)(a.act_meta + (size_t)kq0 * 4 * M);
    uint2 *mdst = (uint2 *)(smem + qbytes);
    for (size_t i = threadIdx.x; i < mbytes / 8; i += 256) mdst[i] = msrc[i];
  }
  __syncthreads();
  const int8_t *sq = (const int8_t *)smem;
  const ActMeta *sm = (const ActMeta *)(smem + qbytes);

  const int nb = blockIdx.x * 4 + wave;
  if (nb >= NB) return;
  const int n_local = lane & 15, c = lane >> 4;

  float acc[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[mt][r] = 0.0f;

  const uint4 *cp = a.codes + ((size_t)nb * KQ + kq0) * 64 + lane;
  const uint2 *sp = a.scales + ((size_t)nb * KQ + kq0) * 16 + n_local;
  constexpr int U = 4;
  uint4 wb[U];
  uint2 sb[U];
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (u < nq) {
      wb[u] = cp[(size_t)u * 64];
      sb[u] = sp[(size_t)u * 16];
    }
  const v4i zero = {0, 0, 0, 0};
  for (int q = 0; q < nq; q += U) {
    uint4 wc[U];
    uint2 sc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      wc[u] = wb[u];
      sc[u] = sb[u];
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (q + U + u < nq) {
        wb[u] = cp[(size_t)(q + U + u) * 64];
        sb[u] = sp[(size_t)(q + U + u) * 16];
      }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (q + u >= nq) break;
      const uint32_t wj[4] = {wc[u].x, wc[u].y, wc[u].z, wc[u].w};
      const float wsj[4] = {h2f(sc[u].x & 0xFFFFu), h2f(sc[u].x >> 16), h2f(sc[u].y & 0xFFFFu),
                            h2f(sc[u].y >> 16)};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int gl = (q + u) * 4 + j;  // group index within the slice
        const long b = unpack_codes(wj[j]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int ma = mt * 16 + n_local;
          v4i dd[D];
#pragma unroll
          for (int d = 0; d < D; ++d) {
            long av = 0;
            if (ma < M) av = *(const long *)(sq + (((size_t)gl * D + d) * M + ma) * 32 + c * 8);
            dd[d] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, b, zero, 0, 0, 0);
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = mt * 16 + c * 4 + r;
            if (m < M) {
              int T = dd[0][r];
              if (D == 3) T = dd[0][r] * 16384 + dd[1][r] * 128 + dd[2][r];
              const ActMeta mm = sm[(size_t)gl * M + m];
              const float v = (float)(T - mm.corr);
              float tt = v * wsj[j];
              tt = tt * mm.scale;
              acc[mt][r] += tt;
            }
          }
        }
      }
    }
  }

  // ---- split-K: deterministic last-arriving finisher ----
  const int N = a.N;
  const int n = nb * 16 + n_local;
  if (a.S > 1) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = mt * 16 + c * 4 + r;
        if (m < M) a.partial[((size_t)s * M + m) * N + n] = acc[mt][r];
      }
    __threadfence();
    int last = 0;
    if (lane == 0) last = (atomicAdd(&a.counters[nb], 1u) == (unsigned)(a.S - 1));
    last = __shfl(last, 0);
    if (!last) return;
    __threadfence();
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = mt * 16 + c * 4 + r;
        float tot = 0.0f;
        if (m < M)
          for (int ss = 0; ss < a.S; ++ss) tot += __builtin_nontemporal_load(&a.partial[((size_t)ss * M + m) * N + n]);
        acc[mt][r] = tot;
      }
    if (lane == 0) a.counters[nb] = 0u;
  }

  // ---- fused epilogues ----
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = mt * 16 + c * 4 + r;
      const float tot = acc[mt][r];
      if (a.epi == EPI_SWIGLU || a.epi == EPI_QKV) {
        // partner row (n_local ^ 8) lives in lane ^ 8 with the same (c, r)
        const float partner = __shfl_xor(tot, 8);
        if (m >= M) continue;
        if (a.epi == EPI_SWIGLU) {
          if (n_local < 8) {
            const int j = nb * 8 + n_local;
            a.y[(size_t)m * (N / 2) + j] = silu_mul(tot, partner);
          }
          continue;
        }
        const QkvArgs &Q = a.qkv;
        const int hd = Q.head_dim;
        const int nbq = Q.num_heads * hd / 16, nbk = Q.num_kv_heads * hd / 16;
        const int kv_dim = Q.num_kv_heads * hd;
        const int pos = Q.pos_of_row[m];
        const int lane_id = Q.lane_of_row[m];
        const int page = Q.page_table[(size_t)lane_id * Q.max_pages + pos / 16];
        const size_t page_base =
            (((size_t)page * Q.num_layers + Q.layer) * 2) * 16 * (size_t)kv_dim;
        const size_t krow = page_base + (size_t)(pos % 16) * kv_dim;
        const size_t vrow = page_base + (size_t)(16 + pos % 16) * kv_dim;
        if (nb < nbq + nbk) {
          if (n_local >= 8) continue;
          const bool is_q = nb < nbq;
          const int rel = is_q ? nb : nb - nbq;
          const int bph = hd / 16;  // row blocks per head
          const int head = rel / bph, p = (rel % bph) * 8 + n_local;
          const int i0 = head * hd + p, i1 = i0 + hd / 2;
          float x0 = tot, x1 = partner;
          if (a.bias) {
            const int off = is_q ? 0 : Q.num_heads * hd;
            x0 = a.bias[off + i0] + x0;
            x1 = a.bias[off + i1] + x1;
          }
          // RopeTable.apply (generate.zig:813-830)
          const float cs = Q.rope_cos[(size_t)pos * (hd / 2) + p];
          const float sn = Q.rope_sin[(size_t)pos * (hd / 2) + p];
          const float a0 = x0 * cs, b0 = x1 * sn, a1 = x0 * sn, b1 = x1 * cs;
          const float y0 = a0 - b0, y1 = a1 + b1;
          if (is_q) {
            float *qo = Q.q_out + (size_t)m * Q.num_heads * hd;
            qo[i0] = y0;
            qo[i1] = y1;
          } else if (Q.kv_f16) {
            __half *kp = (__half *)Q.kv_pool;
            kp[krow + i0] = __float2half_rn(y0);
            kp[krow + i1] = __float2half_rn(y1);
          } else {
            float *kp = (float *)Q.kv_pool;
            kp[krow + i0] = y0;
            kp[krow + i1] = y1;
          }
        } else {
          const int idx = (nb - nbq - nbk) * 16 + n_local;
          float v = tot;
          if (a.bias) v = a.bias[Q.num_heads * hd + kv_dim + idx] + v;
          if (Q.kv_f16)
            ((__half *)Q.kv_pool)[vrow + idx] = __float2half_rn(v);
          else
            ((float *)Q.kv_pool)[vrow + idx] = v;
        }
        continue;
      }
      if (m >= M) continue;
      if (a.epi == EPI_RESID) {
        a.y[(size_t)m * N + n] = a.resid[(size_t)m * N + n] + tot;
      } else {
        a.y[(size_t)m * N + n] = a.bias ? a.bias[n] + tot : tot;
      }
    }
}

hipError_t launch_gemv(const GemvArgs &a, hipStream_t st) {
  const int NB = a.N / 16, KQ = a.K / 128;
  const int maxq = (KQ + a.S - 1) / a.S;
  const size_t lds = act_slice_bytes(maxq, a.M, a.D);
  dim3 grid((NB + 3) / 4, a.S);
  const int MT = (a.M + 15) / 16;
  if (MT > 2) return hipErrorInvalidValue;
#define GK_LAUNCH(DD, MM) \
  hipLaunchKernelGGL((gemv_kernel<DD, MM>), grid, dim3(256), lds, st, a)
  if (a.D == 1) {
    if (MT == 1) GK_LAUNCH(1, 1); else GK_LAUNCH(1, 2);
  } else {
    if (MT == 1) GK_LAUNCH(3, 1); else GK_LAUNCH(3, 2);
  }
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
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
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

__global__ void gather_rows_kernel(const float *table, const int32_t *ids, int dim, float *out) {
  const int m = blockIdx.y;
  const size_t src = (size_t)ids[m] * dim;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < dim; i += gridDim.x * blockDim.x)
    out[(size_t)m * dim + i] = table[src + i];
}

hipError_t launch_gather_rows(const float *table, const int32_t *ids, int M, int dim,
                              float *out, hipStream_t st) {
  hipLaunchKernelGGL(gather_rows_kernel, dim3((dim + 255) / 256, M), dim3(256), 0, st, table,
                     ids, dim, out);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// K3: paged GQA decode attention
// ---------------------------------------------------------------------------
static constexpr int kChunk = 256;
static constexpr int kMaxGroup = 8;

size_t attention_scratch_floats(int M, int num_heads, int head_dim, int max_ctx) {
  const int nch = (max_ctx + kChunk - 1) / kChunk;
  return (size_t)M * num_heads * nch * (2 + head_dim);
}

template <int HD, int F16>
__global__ __launch_bounds__(256) void attn_chunk_kernel(
    const float *q, const void *kv_pool, const int32_t *page_table, int max_pages,
    const int32_t *lane_of_row, const int32_t *ctx_len, int layer, int num_layers, int Hq,
    int Hkv, int n_chunks_max, int max_ctx, float *scratch, float *out) {
  const int ch = blockIdx.x, h = blockIdx.y, m = blockIdx.z, t = threadIdx.x;
  // lengths beyond the launch's capacity are clamped, never read past it
  const int ctx = min(ctx_len[m], max_ctx);
  const int j0 = ch * kChunk;
  if (j0 >= ctx) return;
  const int nvalid = min(kChunk, ctx - j0);
  const int nchunks = (ctx + kChunk - 1) / kChunk;
  const int G = Hq / Hkv;
  const int kv_dim = Hkv * HD;
  const int lane_id = lane_of_row[m];
  __shared__ float sq[kMaxGroup][HD];
  __shared__ float sp[kMaxGroup][kChunk];
  __shared__ float smax[kMaxGroup], ssum[kMaxGroup];
  __shared__ int spage[kChunk / 16];
  for (int i = t; i < G * HD; i += 256)
    sq[i / HD][i % HD] = q[(size_t)m * Hq * HD + (size_t)(h * G) * HD + i];
  if (t < (nvalid + 15) / 16) spage[t] = page_table[(size_t)lane_id * max_pages + (j0 / 16) + t];
  __syncthreads();

  const float scale = 1.0f / sqrtf((float)HD);
  if (t < nvalid) {
    const int j = j0 + t;
    const size_t base =
        ((((size_t)spage[t >> 4] * num_layers + layer) * 2 + 0) * 16 + (j & 15)) * kv_dim +
        (size_t)h * HD;
    float dot[kMaxGroup];
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) dot[g] = 0.0f;
    for (int d = 0; d < HD; d += 8) {
      float kv[8];
      if (F16) {
        const uint4 raw = *(const uint4 *)((const __half *)kv_pool + base + d);
        const __half *hp = (const __half *)&raw;
#pragma unroll
        for (int e = 0; e < 8; ++e) kv[e] = __half2float(hp[e]);
      } else {
        const float4 r0 = *(const float4 *)((const float *)kv_pool + base + d);
        const float4 r1 = *(const float4 *)((const float *)kv_pool + base + d + 4);
        kv[0] = r0.x; kv[1] = r0.y; kv[2] = r0.z; kv[3] = r0.w;
        kv[4] = r1.x; kv[5] = r1.y; kv[6] = r1.z; kv[7] = r1.w;
      }
#pragma unroll
      for (int g = 0; g < kMaxGroup; ++g)
        if (g < G)
#pragma unroll
          for (int e = 0; e < 8; ++e) dot[g] = fmaf(sq[g][d + e], kv[e], dot[g]);
    }
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g)
      if (g < G) sp[g][t] = dot[g] * scale;
  } else {
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g)
      if (g < G) sp[g][t] = -INFINITY;
  }
  __syncthreads();
  // softmax statistics per query head: wave w handles heads w, w + 4
  {
    const int w = t >> 6, l = t & 63;
    for (int g = w; g < G; g += 4) {
      float mx = -INFINITY;
      for (int i = l; i < kChunk; i += 64) mx = fmaxf(mx, sp[g][i]);
      for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
      float sum = 0.0f;
      for (int i = l; i < kChunk; i += 64) {
        const float e = i < nvalid ? expf(sp[g][i] - mx) : 0.0f;
        sp[g][i] = e;
        sum += e;
      }
      for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
      if (l == 0) {
        smax[g] = mx;
        ssum[g] = sum;
      }
    }
  }
  __syncthreads();
  if (nchunks == 1) {
    // single chunk: normalise the weights first, as forward.zig:515-528 does
    for (int i = t; i < G * kChunk; i += 256) {
      const int g = i / kChunk, jj = i % kChunk;
      sp[g][jj] = sp[g][jj] * (1.0f / ssum[g]);
    }
    __syncthreads();
  }
  // P.V: thread -> (d, part)
  constexpr int PARTS = 256 / HD;
  const int d = t % HD, part = t / HD;
  float o[kMaxGroup];
#pragma unroll
  for (int g = 0; g < kMaxGroup; ++g) o[g] = 0.0f;
  for (int i = part; i < nvalid; i += PARTS) {
    const int j = j0 + i;
    const size_t vidx =
        ((((size_t)spage[i >> 4] * num_layers + layer) * 2 + 1) * 16 + (j & 15)) * kv_dim +
        (size_t)h * HD + d;
    const float v = F16 ? __half2float(((const __half *)kv_pool)[vidx]) : ((const float *)kv_pool)[vidx];
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g)
      if (g < G) o[g] = fmaf(sp[g][i], v, o[g]);
  }
  __syncthreads();  // sp reused below as the part-reduction buffer
  float *red = &sp[0][0];
#pragma unroll
  for (int g = 0; g < kMaxGroup; ++g)
    if (g < G) red[(part * kMaxGroup + g) * HD + d] = o[g];
  __syncthreads();
  if (part == 0) {
    for (int g = 0; g < G; ++g) {
      float acc = red[g * HD + d];
      for (int p = 1; p < PARTS; ++p) acc += red[(p * kMaxGroup + g) * HD + d];
      const int qh = h * G + g;
      if (nchunks == 1) {
        out[((size_t)m * Hq + qh) * HD + d] = acc;
      } else {
        float *rec = scratch + (((size_t)m * Hq + qh) * n_chunks_max + ch) * (2 + HD);
        if (d == 0) {
          rec[0] = smax[g];
          rec[1] = ssum[g];
        }
        rec[2 + d] = acc;
      }
    }
  }
}

template <int HD>
__global__ __launch_bounds__(HD) void attn_combine_kernel(const int32_t *ctx_len, int Hq,
                                                          int n_chunks_max, int max_ctx,
                                                          const float *scratch, float *out) {
  const int qh = blockIdx.x, m = blockIdx.y, d = threadIdx.x;
  const int ctx = min(ctx_len[m], max_ctx);
  const int nch = (ctx + kChunk - 1) / kChunk;
  if (nch <= 1) return;
  const float *rec0 = scratch + ((size_t)m * Hq + qh) * n_chunks_max * (2 + HD);
  float mx = -INFINITY;
  for (int c = 0; c < nch; ++c) mx = fmaxf(mx, rec0[(size_t)c * (2 + HD)]);
  float l = 0.0f, o = 0.0f;
  for (int c = 0; c < nch; ++c) {
    const float *rec = rec0 + (size_t)c * (2 + HD);
    const float f = expf(rec[0] - mx);
    l = fmaf(rec[1], f, l);
    o = fmaf(rec[2 + d], f, o);
  }
  out[((size_t)m * Hq + qh) * HD + d] = o * (1.0f / l);
}

hipError_t launch_attention(const float *q, const void *kv_pool, int kv_f16,
                            const int32_t *page_table, int max_pages, const int32_t *lane_of_row,
                            const int32_t *ctx_len, int M, int layer, int num_layers,
                            int num_heads, int num_kv_heads, int head_dim, int max_ctx,
                            float *scratch, float *out, hipStream_t st) {
  if (num_heads % num_kv_heads != 0 || num_heads / num_kv_heads > kMaxGroup)
    return hipErrorInvalidValue;
  const int nch = (max_ctx + kChunk - 1) / kChunk;
  dim3 grid(nch, num_kv_heads, M);
#define GK_ATT(HD, F)                                                                        \
  hipLaunchKernelGGL((attn_chunk_kernel<HD, F>), grid, dim3(256), 0, st, q, kv_pool,          \
                     page_table, max_pages, lane_of_row, ctx_len, layer, num_layers,          \
                     num_heads, num_kv_heads, nch, max_ctx, scratch, out)
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
    hipLaunchKernelGGL((attn_combine_kernel<64>), dim3(num_heads, M), dim3(64), 0, st, ctx_len,
                       num_heads, nch, max_ctx, scratch, out);
  else
    hipLaunchKernelGGL((attn_combine_kernel<128>), dim3(num_heads, M), dim3(128), 0, st,
                       ctx_len, num_heads, nch, max_ctx, scratch, out);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// K5: argmax / eligible argmax
// ---------------------------------------------------------------------------
// Candidate order: larger value wins; equal values -> lower index. NaN
// candidates never win (sampling.zig:194-206 strict '>' scan); index 0's NaN
// case is settled by the finisher.
struct Cand {
  float v;
  long i;
};
static __device__ __forceinline__ bool better(float v, long i, float bv, long bi) {
  if (isnan(v)) return false;
  if (bi < 0) return true;
  return v > bv || (v == bv && i < bi);
}

static constexpr int kArgBlock = 256;
static constexpr int kArgPerBlock = 8192;  // 128 mask words per block

size_t argmax_scratch_bytes(int rows, long n) {
  const long blocks = (n + kArgPerBlock - 1) / kArgPerBlock;
  return (size_t)rows * blocks * 32;
}

struct ArgPartial {
  float v;
  int nan_flag;
  long i;
  unsigned long long rows;
  int bad_mask;
  int pad;
};

__global__ __launch_bounds__(kArgBlock) void argmax_kernel(const float *logits, long n,
                                                           const uint64_t *words,
                                                           long word_count,
                                                           ArgPartial *parts,
                                                           uint32_t *counters,
                                                           ArgmaxResult *result) {
  const int row = blockIdx.y, blk = blockIdx.x, t = threadIdx.x;
  const long nblocks = gridDim.x;
  const float *lr = logits + (size_t)row * n;
  const uint64_t *wr = words ? words + (size_t)row * word_count : nullptr;
  const long e0 = (long)blk * kArgPerBlock, e1 = min(n, e0 + kArgPerBlock);
  float bv = 0.0f;
  long bi = -1;
  int nan_flag = 0;
  for (long e = e0 + t; e < e1; e += kArgBlock) {
    if (wr && !((wr[e >> 6] >> (e & 63)) & 1ull)) continue;
    const float v = lr[e];
    if (isnan(v)) nan_flag = 1;
    if (better(v, e, bv, bi)) {
      bv = v;
      bi = e;
    }
  }
  unsigned long long cnt = 0;
  int bad = 0;
  if (wr) {
    const long w0 = e0 >> 6, w1 = (e1 + 63) >> 6;
    for (long w = w0 + t; w < w1; w += kArgBlock) cnt += __popcll(wr[w]);
    if (blk == nblocks - 1 && t == 0 && (n & 63)) {
      const uint64_t tail = (1ull << (n & 63)) - 1ull;
      if (wr[word_count - 1] & ~tail) bad = 1;
    }
  }
  // wave reduction
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const long oi = __shfl_xor(bi, o);
    if (oi >= 0 && better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
    nan_flag |= __shfl_xor(nan_flag, o);
    cnt += __shfl_xor(cnt, o);
    bad |= __shfl_xor(bad, o);
  }
  __shared__ ArgPartial wp[kArgBlock / 64];
  if ((t & 63) == 0) wp[t >> 6] = ArgPartial{bv, nan_flag, bi, cnt, bad, 0};
  __syncthreads();
  if (t != 0) return;
  ArgPartial p = wp[0];
  for (int w = 1; w < kArgBlock / 64; ++w) {
    const ArgPartial q = wp[w];
    if (q.i >= 0 && better(q.v, q.i, p.v, p.i)) {
      p.v = q.v;
      p.i = q.i;
    }
    p.nan_flag |= q.nan_flag;
    p.rows += q.rows;
    p.bad_mask |= q.bad_mask;
  }
  parts[(size_t)row * nblocks + blk] = p;
  __threadfence();
  if (atomicAdd(&counters[row], 1u) != (unsigned)(nblocks - 1)) return;
  __threadfence();
  ArgPartial r = parts[(size_t)row * nblocks];
  for (long b = 1; b < nblocks; ++b) {
    const ArgPartial q = parts[(size_t)row * nblocks + b];
    if (q.i >= 0 && better(q.v, q.i, r.v, r.i)) {
      r.v = q.v;
      r.i = q.i;
    }
    r.nan_flag |= q.nan_flag;
    r.rows += q.rows;
    r.bad_mask |= q.bad_mask;
  }
  counters[row] = 0u;
  ArgmaxResult res;
  res.pad = 0;
  if (wr) {
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
    res.index = (isnan(lr[0]) || r.i < 0) ? 0 : (uint64_t)r.i;
  }
  result[row] = res;
}

hipError_t launch_argmax(const float *logits, long n, int rows, const uint64_t *words,
                         long word_count, void *scratch, uint32_t *counters,
                         ArgmaxResult *result, hipStream_t st) {
  const long blocks = (n + kArgPerBlock - 1) / kArgPerBlock;
  hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)blocks, rows), dim3(kArgBlock), 0, st,
                     logits, n, words, word_count, (ArgPartial *)scratch, counters, result);
  return hipGetLastError();
}

}  // namespace gk
