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

static __device__ __forceinline__ float silu_mul(float g, float u) {
  // kernels.zig:465-520: g * (1 / (1 + exp(-g))) * u
  float sig = 1.0f / (1.0f + expf(-g));
  float t = g * sig;
  return t * u;
}

// Stores one output value `tot` of activation row m, weight row block nb,
// row n_local; `partner` is the value of row n_local ^ 8 (only read by the
// SwiGLU and QKV epilogues). Rows m >= M are never passed in.
static __device__ __forceinline__ void store_output(const GemvArgs &a, int nb, int n_local, int m,
                                                    float tot, float partner) {
  const int N = a.N;
  if (a.epi == EPI_SWIGLU) {
    if (n_local < 8) a.y[(size_t)m * (N / 2) + nb * 8 + n_local] = silu_mul(tot, partner);
    return;
  }
  if (a.epi == EPI_QKV) {
    const QkvArgs &Q = a.qkv;
    const int hd = Q.head_dim;
    const int nbq = Q.num_heads * hd / 16, nbk = Q.num_kv_heads * hd / 16;
    const int kv_dim = Q.num_kv_heads * hd;
    const int pos = Q.pos_of_row[m];
    const int lane_id = Q.lane_of_row[m];
    const int page = Q.page_table[(size_t)lane_id * Q.max_pages + pos / 16];
    const size_t page_base = (((size_t)page * Q.num_layers + Q.layer) * 2) * 16 * (size_t)kv_dim;
    const size_t krow = page_base + (size_t)(pos % 16) * kv_dim;
    const size_t vrow = page_base + (size_t)(16 + pos % 16) * kv_dim;
    if (nb < nbq + nbk) {
      if (n_local >= 8) return;
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
    return;
  }
  const int n = nb * 16 + n_local;
  if (a.epi == EPI_RESID)
    a.y[(size_t)m * N + n] = a.resid[(size_t)m * N + n] + tot;
  else
    a.y[(size_t)m * N + n] = a.bias ? a.bias[n] + tot : tot;
}

}  // namespace gk
