// epilogue.h — the fused output stage shared by the decode GEMV (K1) and the
// prefill GEMM (K2).
//
// Both kernels finish with the same register layout: a lane owns output
// column n = 16 * nb + n_local of weight row block nb for some activation
// rows m, and the partner row n_local ^ 8 of the same block lives in lane ^ 8
// with the same m. The device weight layout pairs rows so that the SwiGLU and
// RoPE partners sit 8 rows apart inside a 16-row block:
//   * gate/up (EPI_SWIGLU): rows 0..7 of block b are gate rows 8b..8b+7,
//     rows 8..15 the matching up rows;
//   * QKV (EPI_QKV): q and k heads in blocks of 8 RoPE pairs (p, p + hd/2),
//     then the v rows in plain order.
#pragma once
#include <hip/hip_fp16.h>
#include <math.h>

#include "int4_ops.h"
#include "kernels.h"

namespace gk {

// Greedy candidate order (sampling.zig:194-206): a larger value wins, equal
// values go to the lower index, a NaN never wins; bi < 0 means "none yet".
static __device__ __forceinline__ bool arg_better(float v, long i, float bv, long bi) {
  if (isnan(v)) return false;
  if (bi < 0) return true;
  return v > bv || (v == bv && i < bi);
}

static __device__ __forceinline__ void arg_merge(ArgPartial &p, const ArgPartial &q) {
  if (q.i >= 0 && arg_better(q.v, q.i, p.v, p.i)) {
    p.v = q.v;
    p.i = q.i;
  }
  p.nan_flag |= q.nan_flag;
  p.rows += q.rows;
  p.bad_mask |= q.bad_mask;
  p.nan0 |= q.nan0;
}

static __device__ __forceinline__ ArgPartial arg_shfl_xor(const ArgPartial &p, int o) {
  ArgPartial q;
  q.v = __shfl_xor(p.v, o);
  q.i = __shfl_xor(p.i, o);
  q.nan_flag = __shfl_xor(p.nan_flag, o);
  q.rows = __shfl_xor(p.rows, o);
  q.bad_mask = __shfl_xor(p.bad_mask, o);
  q.nan0 = __shfl_xor(p.nan0, o);
  return q;
}

// Converts the 32-element group held by a 32-lane half-wave (one value per
// lane, hl = lane within the half-wave) into D digit bytes per lane and the
// group's meta. q layout [G][D][M][32], meta [G][M].
template <int D>
static __device__ __forceinline__ void quantize_group(float v, int hl, int g, int m, int M,
                                                      int8_t *act_q, ActMeta *meta) {
  const float amax = half_wave_max(fabsf(v));
  const float scale = amax / 127.0f;
  const float inv_s = scale == 0.0f ? 0.0f : 1.0f / scale;
  const float y = v * inv_s;
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
  int comb = 0;  // 128-adic combination of the digits; one reduction gives sum_d 128^(D-1-d) sum q_d
#pragma unroll
  for (int d = 0; d < D; ++d) {
    act_q[(((size_t)g * D + d) * M + m) * 32 + hl] = (int8_t)qd[d];
    comb = comb * 128 + qd[d];
  }
  const int sum = half_wave_sum(comb);
  if (hl == 0) {
    ActMeta mm;
    mm.scale = D == 3 ? scale * (1.0f / 16384.0f) : scale;
    mm.corr = 7 * sum;
    meta[(size_t)g * M + m] = mm;
  }
}

static __device__ __forceinline__ float silu_mul(float g, float u) {
  // kernels.zig:465-520: g * (1 / (1 + exp(-g))) * u
  float sig = 1.0f / (1.0f + expf(-g));
  float t = g * sig;
  return t * u;
}

// Inputs the epilogue reads besides the dot product, for one output (row m,
// weight row block nb, row n_local): the residual, bias values, the RoPE
// factors and the KV page slot of the row's position. Loading them is
// separate from storing so the decode GEMV can request them early: the
// first level (epi_load1) has no dependence on other loads, the second
// (epi_load2: page id and RoPE factors of the row's position) needs pos and
// lane_id from the first.
struct EpiIn {
  float resid, b0, b1, cs, sn;
  int pos, lane_id, page;
};

static __device__ __forceinline__ void epi_load1(EpiIn &e, const GemvArgs &a, int epi, int nb,
                                                 int n_local, int m) {
  e.resid = e.b0 = e.b1 = e.cs = e.sn = 0.0f;
  e.pos = e.lane_id = e.page = 0;
  const int n = nb * 16 + n_local;
  if (epi == EPI_QKV) {
    // every lane of a row block loads (RoPE partner rows n_local >= 8 read
    // their pair's entries and ignore them), so no branch splits the wave
    const QkvArgs &Q = a.qkv;
    const int hd = Q.head_dim;
    const int nbq = Q.num_heads * hd / 16, nbk = Q.num_kv_heads * hd / 16;
    const int kv_dim = Q.num_kv_heads * hd;
    e.pos = Q.pos_of_row[m];
    e.lane_id = Q.lane_of_row[m];
    if (a.bias) {
      if (nb < nbq + nbk) {
        const bool is_q = nb < nbq;
        const int rel = is_q ? nb : nb - nbq;
        const int bph = hd / 16;  // row blocks per head
        const int head = rel / bph, p = (rel % bph) * 8 + (n_local & 7);
        const int i0 = head * hd + p, i1 = i0 + hd / 2;
        const int off = is_q ? 0 : Q.num_heads * hd;
        e.b0 = a.bias[off + i0];
        e.b1 = a.bias[off + i1];
      } else {
        e.b0 = a.bias[Q.num_heads * hd + kv_dim + (nb - nbq - nbk) * 16 + n_local];
      }
    }
  } else if (epi == EPI_RESID) {
    e.resid = a.resid[(size_t)m * a.N + n];
  } else if (epi == EPI_PLAIN) {
    if (a.bias) e.b0 = a.bias[n];
  }
}

static __device__ __forceinline__ void epi_load2(EpiIn &e, const GemvArgs &a, int epi, int nb,
                                                 int n_local) {
  if (epi != EPI_QKV) return;
  const QkvArgs &Q = a.qkv;
  const int hd = Q.head_dim;
  const int nbq = Q.num_heads * hd / 16, nbk = Q.num_kv_heads * hd / 16;
  e.page = Q.page_table[(size_t)e.lane_id * Q.max_pages + e.pos / 16];
  if (nb < nbq + nbk) {
    const int rel = nb < nbq ? nb : nb - nbq;
    const int p = (rel % (hd / 16)) * 8 + (n_local & 7);
    e.cs = Q.rope_cos[(size_t)e.pos * (hd / 2) + p];
    e.sn = Q.rope_sin[(size_t)e.pos * (hd / 2) + p];
  }
}

static __device__ __forceinline__ EpiIn epi_load(const GemvArgs &a, int epi, int nb, int n_local,
                                                 int m) {
  EpiIn e;
  epi_load1(e, a, epi, nb, n_local, m);
  epi_load2(e, a, epi, nb, n_local);
  return e;
}

// Stores one output value `tot` of activation row m, weight row block nb,
// row n_local with epilogue type epi; `partner` is the value of row
// n_local ^ 8 (only read by the SwiGLU and QKV epilogues), e its epi_load
// inputs. Rows m >= M are never passed in.
static __device__ __forceinline__ void store_output(const GemvArgs &a, int epi, int nb,
                                                    int n_local, int m, float tot, float partner,
                                                    const EpiIn &e) {
  const int N = a.N;
  if (epi == EPI_SWIGLU) {
    if (n_local < 8) a.y[(size_t)m * (N / 2) + nb * 8 + n_local] = silu_mul(tot, partner);
    return;
  }
  if (epi == EPI_QKV) {
    const QkvArgs &Q = a.qkv;
    const int hd = Q.head_dim;
    const int nbq = Q.num_heads * hd / 16, nbk = Q.num_kv_heads * hd / 16;
    const int kv_dim = Q.num_kv_heads * hd;
    const size_t page_base = (((size_t)e.page * Q.num_layers + Q.layer) * 2) * 16 * (size_t)kv_dim;
    const size_t krow = page_base + (size_t)(e.pos % 16) * kv_dim;
    const size_t vrow = page_base + (size_t)(16 + e.pos % 16) * kv_dim;
    if (nb < nbq + nbk) {
      if (n_local >= 8) return;
      const bool is_q = nb < nbq;
      const int rel = is_q ? nb : nb - nbq;
      const int bph = hd / 16;  // row blocks per head
      const int head = rel / bph, p = (rel % bph) * 8 + n_local;
      const int i0 = head * hd + p, i1 = i0 + hd / 2;
      float x0 = tot, x1 = partner;
      if (a.bias) {
        x0 = e.b0 + x0;
        x1 = e.b1 + x1;
      }
      // RopeTable.apply (generate.zig:813-830)
      const float a0 = x0 * e.cs, b0 = x1 * e.sn, a1 = x0 * e.sn, b1 = x1 * e.cs;
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
      if (a.bias) v = e.b0 + v;
      if (Q.kv_f16)
        ((__half *)Q.kv_pool)[vrow + idx] = __float2half_rn(v);
      else
        ((float *)Q.kv_pool)[vrow + idx] = v;
    }
    return;
  }
  const int n = nb * 16 + n_local;
  if (epi == EPI_RESID)
    a.y[(size_t)m * N + n] = e.resid + tot;
  else
    a.y[(size_t)m * N + n] = a.bias ? e.b0 + tot : tot;
}

}  // namespace gk
