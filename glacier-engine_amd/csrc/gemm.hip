// gemm.hip — K2: INT4 x int8-digit GEMM on gfx950 MFMA.
//
// y[M][N] = planes(x)[M][K] . W^T past the decode GEMV's rows (decode
// batches of 6 or more lanes, prompt chunks), with the
// same digit planes, tile layout and fused epilogues as the decode GEMV (K1):
// the per-group arithmetic is the reference's Q8 dot
// (int4_matmul.zig:365-418): an exact integer dot per 32-element group,
// scaled by the weight and activation group scales and summed in f32.
//
// One v_mfma_i32_16x16x32_i8 covers exactly one group of a 16x16 output tile.
// The weight codes are made signed (u - 7) in registers, so the MFMA result
// is the group dot T itself; with one digit the accumulator starts at the
// bits of 1.5 * 2^23 and fma(that as f32, ws, -12582912 * ws) = RN(T * ws)
// (int4_ops.h), then one fma applies the activation scale into the running
// sum. Three-digit (f32 activation) planes run three independent MFMAs and
// combine them as the exact 128-adic integer.
//
// The per-group scaling (two fmas per output and group against one MFMA per
// 16 x 16 x 32 group tile) bounds this kernel by VALU issue, not by the
// matrix cores; the layout keeps everything else off that path:
//   * workgroup = 4 waves over a BM-row (32 or 64) x 64 kRB-column output
//     tile; each wave owns kRB (1, 2 or 4) weight row blocks x the BM / 16
//     activation row tiles;
//   * weights: each lane loads its own 16-byte tile slot per row block and
//     quad (1 KB per wave, fully coalesced), two quads in flight; the words
//     are transposed across lanes into MFMA operands (quad_transpose) and
//     the lane-ordered fp16 scales gathered per column (column_gather);
//   * activations: the workgroup stages each quad's digit planes (64 rows x
//     128 columns x D) and their scales in LDS, double buffered, one barrier
//     per quad; every wave reads its operands from there;
//   * block ids are remapped so that the row tiles of one weight column tile
//     run on one XCD (hardware places block b on XCD b % 8), which keeps the
//     tile's weights in that XCD's L2 for every row tile that reads them;
//   * small grids (few row tiles x few column tiles, e.g. 32 decode rows of a
//     3584-wide projection) split K over workgroups: each split writes its
//     partial sums and splitk_reduce_kernel adds the splits in a fixed order
//     and runs the epilogue (deterministic, no atomics).
#include "epilogue.h"
#include "int4_ops.h"
#include "kernels.h"

#include <algorithm>

namespace gk {

namespace {

constexpr int kWaves = 4;            // waves per workgroup, side by side in N
constexpr int kU = 2;                // weight quads in flight per wave
constexpr int kFoldSplits = 4;       // K splits a folded tile adds at most

// Per-quad activation staging of a BM-row tile: digit planes
// [4 groups][D][BM rows][32] then the scales [4][BM].
template <int D, int BM>
struct ActStage {
  static constexpr int kActBytes = 4 * D * BM * 32;
  static constexpr int kBufBytes = kActBytes + 4 * BM * 4;
  static constexpr int kUnitCount = kActBytes / 16;            // 16-byte units
  static constexpr int kUnits = (kUnitCount + 255) / 256;      // per thread
};

// One thread's share of a quad's activation staging: up to six 16-byte
// units (3-digit planes, 64 rows) as named members, read and written through
// at() with indices that are constants once the loops are unrolled. (An
// array member of six units was kept in scratch memory, whose stores waited
// for the loads as soon as they were issued.)
template <int D, int BM>
struct ActRegs {
  static_assert(ActStage<D, BM>::kUnits <= 6, "six units per thread at most");
  uint4 v0, v1, v2, v3, v4, v5;
  float sc;
  __device__ __forceinline__ uint4 &at(int i) {
    switch (i) {
      case 0: return v0;
      case 1: return v1;
      case 2: return v2;
      case 3: return v3;
      case 4: return v4;
      default: return v5;
    }
  }
  __device__ __forceinline__ const uint4 &at(int i) const {
    return const_cast<ActRegs *>(this)->at(i);
  }
};

// Loads quad kq's activation planes (rows m0 .. m0 + BM - 1, clamped to
// M - 1) and scales into registers; one 16-byte unit per thread and pass
// (16-row tiles have fewer units than threads: the extra threads repeat the
// last unit, branch-free).
template <int D, int BM>
__device__ __forceinline__ ActRegs<D, BM> act_load(const GemvArgs &p, int kq, int m0) {
  ActRegs<D, BM> r;
  const int M = p.M, t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < ActStage<D, BM>::kUnits; ++i) {
    const int u = min(t + 256 * i, ActStage<D, BM>::kUnitCount - 1);  // ((j * D + d) * BM + row) * 2 + half
    const int half = u & 1, row = (u >> 1) % BM, jd = (u >> 1) / BM;
    const int m = min(m0 + row, M - 1);
    const size_t src = ((size_t)(4 * kq) * D + jd) * M + m;  // group 4kq + j, digit d
    r.at(i) = *(const uint4 *)(p.act_q + src * 32 + 16 * half);
  }
  const int ts = t % (4 * BM);  // threads past 4 BM repeat another's scale
  const int j = ts / BM, row = ts % BM;
  r.sc = p.act_meta[(size_t)(4 * kq + j) * M + min(m0 + row, M - 1)].scale;
  return r;
}

template <int D, int BM>
__device__ __forceinline__ void act_store(unsigned char *buf, const ActRegs<D, BM> &r) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < ActStage<D, BM>::kUnits; ++i)
    ((uint4 *)buf)[min(t + 256 * i, ActStage<D, BM>::kUnitCount - 1)] = r.at(i);
  // (duplicates store the same value to the same slot: no branch)
  ((float *)(buf + ActStage<D, BM>::kActBytes))[t % (4 * BM)] = r.sc;
}

// kRB: 16-row weight blocks per wave (1, 2 or 4; the workgroup covers 4 kRB);
// BM: activation rows per workgroup (16, 32 or 64). The K quads are split over
// blockIdx.y (ks_count splits); with part set each split writes its partial
// sums to part [ks_count][M][N] (no epilogue; a finishing kernel runs it),
// unless fold: then the splits of a tile meet at p.splitk_counters and the
// last to arrive runs the epilogue (the SwiGLU plane emission included).
template <int D, int kRB, int BM>
__global__ __launch_bounds__(256, kRB == 4 ? 2 : kRB == 2 ? 4 : 5) void gemm_kernel(GemvArgs p, int m_tiles,
                                                                     int ks_count, float *part,
                                                                     int fold) {
  using S = ActStage<D, BM>;
  constexpr int MT = BM / 16;         // 16-row activation tiles per wave
  constexpr int kNBW = kWaves * kRB;  // weight row blocks per workgroup
  __shared__ __align__(16) unsigned char lds[2 * S::kBufBytes];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform
  const int n_local = lane & 15, c = lane >> 4;
  const int NB = p.N >> 4, KQ = p.K >> 7;
  // XCD-aware block order: XCD x runs logical blocks [first_x, first_x + cnt_x)
  const int nblk = gridDim.x, b = blockIdx.x;
  const int xcd = b & 7, idx = b >> 3;
  const int logical = xcd * (nblk >> 3) + min(xcd, nblk & 7) + idx;
  const int n_tile = logical / m_tiles, m_tile = logical % m_tiles;
  const int m0 = m_tile * BM;
  const int nb0 = n_tile * kNBW + wave * kRB;  // this wave's first row block
  // this split's quads kq0 .. kq0 + nq - 1
  const int kq0 = (int)(((long)blockIdx.y * KQ) / ks_count);
  const int nq = (int)(((long)(blockIdx.y + 1) * KQ) / ks_count) - kq0;

  // weight slots of this wave's row blocks: one per-lane base pointer plus
  // uniform tile offsets (row blocks past NB are clamped into range, compute
  // on a copy and are never stored)
  const uint4 *cp = p.codes + lane;
  const uint16_t *spp = (const uint16_t *)p.scales + lane;
  size_t toff[kRB];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) toff[rb] = ((size_t)min(nb0 + rb, NB - 1) * KQ + kq0) * 64;
  uint4 wb[kU][kRB];
  uint32_t sb[kU][kRB];
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const int q = min(u, nq - 1);
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) {
      wb[u][rb] = load_stream(cp + toff[rb] + (size_t)q * 64);
      sb[u][rb] = spp[toff[rb] + (size_t)q * 64];
    }
  }
  act_store<D, BM>(lds, act_load<D, BM>(p, kq0, m0));
  __syncthreads();

  float acc[kRB][MT][4];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[rb][mt][r] = 0.0f;
  const v4i magic = {kMagic, kMagic, kMagic, kMagic};
  const v4i zero = {0, 0, 0, 0};

  for (int q0 = 0; q0 < nq; q0 += kU) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int q = q0 + u;  // local quad index (absolute kq0 + q)
      if (q >= nq) break;
      // this quad's weights; the slot is refilled with quad q + kU
      uint4 wc[kRB];
      uint32_t sc[kRB];
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) {
        wc[rb] = wb[u][rb];
        sc[rb] = sb[u][rb];
      }
      // (branch-free: past the end the last quad is loaded again and never
      // used, so the quad's work stays one block for the scheduler)
      const int qn = min(q + kU, nq - 1);
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) {
        wb[u][rb] = load_stream(cp + toff[rb] + (size_t)qn * 64);
        sb[u][rb] = spp[toff[rb] + (size_t)qn * 64];
      }
      // the next quad's activations, in flight while this one computes
      // (the last quad stages a copy of itself into the idle buffer)
      const ActRegs<D, BM> nxt = act_load<D, BM>(p, kq0 + min(q + 1, nq - 1), m0);

      // q0 is even, so this quad's buffer is u: constant LDS offsets
      const unsigned char *buf = lds + u * S::kBufBytes;
      uint4 wt[kRB];
      float ws[kRB][4];  // [row block][group]: scale of this lane's column
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) wt[rb] = quad_transpose(wc[rb]);
#pragma unroll
      for (int h = 0; h < (kRB + 1) / 2; ++h) {
        // two row blocks' u16 scales per register, all four groups' rows
        uint32_t g4[4];
        const uint32_t hi = 2 * h + 1 < kRB ? sc[min(2 * h + 1, kRB - 1)] << 16 : 0u;
        column_gather((sc[2 * h] & 0xFFFFu) | hi, g4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          ws[2 * h][j] = h2f(g4[j] & 0xFFFFu);
          if (2 * h + 1 < kRB) ws[min(2 * h + 1, kRB - 1)][j] = h2f(g4[j] >> 16);
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        long bw[kRB];
#pragma unroll
        for (int rb = 0; rb < kRB; ++rb) {
          const uint32_t w = j == 0 ? wt[rb].x : j == 1 ? wt[rb].y : j == 2 ? wt[rb].z : wt[rb].w;
          bw[rb] = signed_codes(w);
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          long av[D];
#pragma unroll
          for (int d = 0; d < D; ++d)
            av[d] = *(const long *)(buf + (((j * D + d) * BM + mt * 16 + n_local) * 32 + 8 * c));
          const float4 as4 = *(const float4 *)(buf + S::kActBytes + (j * BM + mt * 16 + 4 * c) * 4);
          const float as[4] = {as4.x, as4.y, as4.z, as4.w};
#pragma unroll
          for (int rb = 0; rb < kRB; ++rb) {
            if constexpr (D == 1) {
              const v4i dd = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[0], bw[rb], magic, 0, 0, 0);
              const float wcorr = -kMagicF * ws[rb][j];
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const float t = fmaf(__int_as_float(dd[r]), ws[rb][j], wcorr);
                acc[rb][mt][r] = fmaf(t, as[r], acc[rb][mt][r]);
              }
            } else {
              v4i dd[D];
#pragma unroll
              for (int d = 0; d < D; ++d)
                dd[d] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[d], bw[rb], zero, 0, 0, 0);
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                int T = dd[0][r];
#pragma unroll
                for (int d = 1; d < D; ++d) T = (T << 7) + dd[d][r];
                acc[rb][mt][r] = fmaf((float)T * ws[rb][j], as[r], acc[rb][mt][r]);
              }
            }
          }
          // one activation tile's MFMAs at a time: their results are
          // consumed before the next tile's are issued (register budget)
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      // publish the next quad's activations (the other buffer was last read
      // before the previous barrier)
      act_store<D, BM>(lds + (u ^ 1) * S::kBufBytes, nxt);
      __syncthreads();
    }
  }

  // Lane (c, n) holds rows m0 + 16 mt + 4c + r of column 16 nb + n.
  // (the fold's publication is compiled into tiles of up to 32 rows only: in
  // the 64-row prompt-chunk tiles its registers would spill the whole
  // kernel; those fold only without a K split, where the sums are complete)
  if (fold) {
    if (BM <= 32 && ks_count > 1) {
      // Publish this split's partial sums; the tile's last split to arrive
      // adds every split's in split order (the finishing kernel's order, so
      // the sums are the same) and runs the epilogue. The publication is the
      // cross-workgroup contract attn_o_kernel's merge documents:
      // agent-scope stores written through to the level every XCD reads,
      // waited for (s_waitcnt covers stores), then an agent-scope counter
      // increment; the last arriver reads with agent-scope loads.
      const size_t MN = (size_t)p.M * p.N;
      float *dst = part + (size_t)blockIdx.y * MN;
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = m0 + 16 * mt + 4 * c + r, nb = nb0 + rb;
            if (m < p.M && nb < NB)
              __hip_atomic_store(dst + (size_t)m * p.N + nb * 16 + n_local, acc[rb][mt][r],
                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
      __builtin_amdgcn_s_waitcnt(0);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      __syncthreads();
      __shared__ int tile_last;
      if (threadIdx.x == 0)
        tile_last = __hip_atomic_fetch_add(p.splitk_counters + blockIdx.x, 1u, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(ks_count - 1);
      __syncthreads();
      if (!tile_last) return;
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
      // one (row block, row tile) at a time: its up to kFoldSplits splits'
      // loads issued together, then added in split order
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          float v[kFoldSplits][4];
#pragma unroll
          for (int sp = 0; sp < kFoldSplits; ++sp)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int m = m0 + 16 * mt + 4 * c + r, nb = nb0 + rb;
              const size_t idx = m < p.M && nb < NB ? (size_t)m * p.N + nb * 16 + n_local : 0;
              v[sp][r] = sp < ks_count ? __hip_atomic_load(part + sp * MN + idx, __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT)
                                       : 0.0f;
            }
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float tot = v[0][r];
#pragma unroll
            for (int sp = 1; sp < kFoldSplits; ++sp)
              if (sp < ks_count) tot += v[sp][r];
            acc[rb][mt][r] = tot;
          }
        }
      if (threadIdx.x == 0)
        __hip_atomic_store(p.splitk_counters + blockIdx.x, 0u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    if constexpr (BM * 32 * kRB * 4 <= 2 * S::kBufBytes) {
      if (p.epi == EPI_SWIGLU && p.out_q) {
        // The SwiGLU plane emission of splitk_swiglu_emit_kernel for this
        // tile: its 4 kRB row blocks hold 32 kRB SwiGLU outputs (kRB whole
        // quantisation groups) of each activation row; silu(g) * u into LDS
        // [BM][32 kRB], then a half-wave quantises each (row, group).
        constexpr int NO = 32 * kRB;
        float *stage = (float *)lds;
        __syncthreads();  // the staging buffers were last read before the loop's end
#pragma unroll
        for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float tot = acc[rb][mt][r];
              const float partner = row_xor8(tot);
              if (n_local < 8)
                stage[(16 * mt + 4 * c + r) * NO + (wave * kRB + rb) * 8 + n_local] =
                    silu_mul(tot, partner);
            }
        __syncthreads();
        const int No = p.N >> 1;
        const int half = threadIdx.x >> 5, hl = threadIdx.x & 31;
        for (int it = half; it < BM * kRB; it += 8) {
          const int row = it / kRB, gl = it % kRB, m = m0 + row;
          const int o = (n_tile * kNBW) * 8 + gl * 32 + hl;  // SwiGLU output index
          if (m >= p.M || o >= No) continue;  // whole half-waves: No is a multiple of 32
          const float v = stage[row * NO + gl * 32 + hl];
          if (p.y) p.y[(size_t)m * No + o] = v;
          if (p.out_D == 1)
            quantize_group<1>(v, hl, o >> 5, m, p.M, p.out_q, p.out_meta);
          else
            quantize_group<3>(v, hl, o >> 5, m, p.M, p.out_q, p.out_meta);
        }
        return;
      }
    }
  } else if (part) {
    // split K (or a finishing pass that emits planes): this split's partial
    // sums, part[split][m][n]
    float *dst = part + (size_t)blockIdx.y * p.M * p.N;
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + 16 * mt + 4 * c + r, nb = nb0 + rb;
          if (m < p.M && nb < NB) dst[(size_t)m * p.N + nb * 16 + n_local] = acc[rb][mt][r];
        }
    return;
  }
  // The SwiGLU / RoPE partner row n ^ 8 lives in lane ^ 8. The epilogue runs
  // as a loop over each row block's values parked in this thread's own LDS
  // column (the staging buffers are free after the last barrier): unrolled
  // over the large inlined epilogue it would index the accumulators
  // dynamically and push them to scratch.
  static_assert(MT * 4 * 256 * 4 <= 2 * S::kBufBytes, "parking area");
  const bool paired = p.epi == EPI_SWIGLU || p.epi == EPI_QKV;
  float *park = (float *)lds + threadIdx.x;
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) park[(mt * 4 + r) * 256] = acc[rb][mt][r];
    const int nb = nb0 + rb;
#pragma unroll 1
    for (int i = 0; i < MT * 4; ++i) {
      const float tot = park[i * 256];
      const float partner = paired ? row_xor8(tot) : 0.0f;
      const int m = m0 + 16 * (i >> 2) + 4 * c + (i & 3);
      if (m < p.M && nb < NB)
        store_output(p, p.epi, nb, n_local, m, tot, partner, epi_load(p, p.epi, nb, n_local, m));
    }
  }
}

// Split-K finish: y = the fixed-order sum over splits of part[s][m][n],
// through the same epilogue as the one-split kernel. One thread per output
// (m, n); the SwiGLU / RoPE partner n ^ 8 is summed by the same thread.
// KS > 0: that many splits, every load issued before the first add; KS = 0:
// ks_count splits in a loop.
template <int KS>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemvArgs p, int ks_count,
                                                            const float *part) {
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t MN = (size_t)p.M * p.N;
  if (idx >= MN) return;
  const int m = (int)(idx / p.N), n = (int)(idx % p.N);
  const int nb = n >> 4, n_local = n & 15;
  const bool paired = p.epi == EPI_SWIGLU || p.epi == EPI_QKV;
  // the partner of an unpaired output is itself (loaded, never used)
  const size_t pi = paired ? (size_t)m * p.N + (n ^ 8) : idx;
  float tot, partner;
  if constexpr (KS > 0) {
    float tv[KS], pv[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      tv[s] = part[s * MN + idx];
      pv[s] = part[s * MN + pi];
    }
    tot = tv[0];
    partner = pv[0];
#pragma unroll
    for (int s = 1; s < KS; ++s) {
      tot += tv[s];
      partner += pv[s];
    }
  } else {
    tot = part[idx];
    partner = part[pi];
    for (int s = 1; s < ks_count; ++s) {
      tot += part[s * MN + idx];
      partner += part[s * MN + pi];
    }
  }
  if (!paired) partner = 0.0f;
  store_output(p, p.epi, nb, n_local, m, tot, partner, epi_load(p, p.epi, nb, n_local, m));
}

// Split-K finish of the gate/up GEMM that also emits the down projection's
// digit planes: one thread per SwiGLU output (m, o), o < N / 2, whose gate
// and up rows are device rows 16 (o / 8) + o % 8 and that + 8 (the
// interleaved layout); every split sum in a fixed order, then the epilogue's
// silu(g) * u. A half-wave holds 32 consecutive outputs of one row, which
// is one quantisation group of the planes.
template <int KS, int D>
__global__ __launch_bounds__(256) void splitk_swiglu_emit_kernel(GemvArgs p, const float *part) {
  const int No = p.N >> 1;
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t MN = (size_t)p.M * p.N;
  if (idx >= (size_t)p.M * No) return;  // whole half-waves: No is a multiple of 32
  const int m = (int)(idx / No), o = (int)(idx % No);
  const size_t gi = (size_t)m * p.N + ((o >> 3) << 4) + (o & 7), ui = gi + 8;
  float gv[KS], uv[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    gv[s] = part[s * MN + gi];
    uv[s] = part[s * MN + ui];
  }
  float g = gv[0], u = uv[0];
#pragma unroll
  for (int s = 1; s < KS; ++s) {
    g += gv[s];
    u += uv[s];
  }
  const float v = silu_mul(g, u);
  if (p.y) p.y[(size_t)m * No + o] = v;
  quantize_group<D>(v, o & 31, o >> 5, m, p.M, p.out_q, p.out_meta);
}

// Split-K finish of a residual GEMM (O, down) that also produces the next
// projection's input: y = resid + (fixed-order sum of the splits) is
// written, then the row's RMSNorm with emit_norm_w (kernels.zig:141-220:
// y / sqrt(mean(y^2) + eps) * w) and the group quantiser give the digit
// planes prep_act_kernel would make from y. One workgroup per row; each
// thread owns 8 consecutive outputs (two 16-byte loads per split, all of a
// thread's loads issued before the first add), so 4 threads (one quad) hold
// a 32-wide group and reduce it with quad DPP exchanges.
constexpr int kEmitThreads = 512;  // rows of up to 4096
template <int KS, int D>
__global__ __launch_bounds__(kEmitThreads) void splitk_resid_emit_kernel(GemvArgs p,
                                                                         const float *part) {
  const int m = blockIdx.x, t = threadIdx.x, N = p.N;
  const size_t MN = (size_t)p.M * N, row = (size_t)m * N;
  const bool act = 8 * t < N;  // N is a multiple of 32: whole quads
  const int n0 = act ? 8 * t : 0;
  __shared__ float red[kEmitThreads / 64 + 1];
  float4 pv[KS][2], rv[2], wv[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    rv[h] = *(const float4 *)(p.resid + row + n0 + 4 * h);
    wv[h] = *(const float4 *)(p.emit_norm_w + n0 + 4 * h);
#pragma unroll
    for (int s = 0; s < KS; ++s) pv[s][h] = *(const float4 *)(part + s * MN + row + n0 + 4 * h);
  }
  float y[8], w8[8];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int h = i >> 2, e = i & 3;
    float tot = pv[0][h][e];
#pragma unroll
    for (int s = 1; s < KS; ++s) tot += pv[s][h][e];
    y[i] = rv[h][e] + tot;
    w8[i] = wv[h][e];
    ss = fmaf(y[i], y[i], ss);
  }
  if (act) {
    *(float4 *)(p.y + row + n0) = make_float4(y[0], y[1], y[2], y[3]);
    *(float4 *)(p.y + row + n0 + 4) = make_float4(y[4], y[5], y[6], y[7]);
  } else {
    ss = 0.0f;
  }
  ss = wave_sum(ss);
  if ((t & 63) == 0) red[t >> 6] = ss;
  __syncthreads();
  if (t == 0) {
    float sum = 0.0f;
#pragma unroll
    for (int w = 0; w < kEmitThreads / 64; ++w) sum += red[w];
    red[kEmitThreads / 64] = 1.0f / sqrtf(sum / (float)N + p.in_eps);
  }
  __syncthreads();
  const float inv = red[kEmitThreads / 64];
  // group quantiser (int4_matmul.zig:380-398), the same arithmetic as
  // quantize_group, over the quad's 32 values
  float v[8];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[i] = (y[i] * inv) * w8[i];
    amax = fmaxf(amax, fabsf(v[i]));
  }
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
    const float yq = v[i] * inv_s;
    float q0f = roundf(yq);
    q0f = fminf(fmaxf(q0f, -127.0f), 127.0f);
    int qd[3] = {(int)q0f, 0, 0};
    if (D == 3) {
      const float r1 = (yq - q0f) * 128.0f;
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
  if (act) {
    const int g = n0 >> 5, qp = (n0 >> 3) & 3;
#pragma unroll
    for (int d = 0; d < D; ++d)
      *(uint64_t *)(p.out_q + (((size_t)g * D + d) * p.M + m) * 32 + qp * 8) = packed[d];
    if (qp == 0) {
      ActMeta mm;
      mm.scale = D == 3 ? scale * (1.0f / 16384.0f) : scale;
      mm.corr = 7 * csum;
      p.out_meta[(size_t)g * p.M + m] = mm;
    }
  }
}

}  // namespace

GemmShape plan_gemm(int N, int M, int K, int D, size_t ws_floats) {
  GemmShape s;
  const int bm = M <= 16 ? 16 : M <= 32 ? 32 : 64;
  s.mt = bm / 16;
  s.m_tiles = (M + bm - 1) / bm;
  // Row blocks per wave and the workgroup target, from sweeps of the 7B
  // shapes: 16- and 32-row tiles (decode lanes; 16 rows up to 16, so small
  // batches do not pay for 32 rows of MFMA and scaling work) 1 row block per wave for one-digit
  // planes, 2 for three, toward about 1024 workgroups; 64-row tiles (prompt
  // chunks) 2 for one digit (4 workgroups per CU), 4 for three once that
  // still fills the GPU, toward about 512.
  const int NB = N / 16, KQ = K / 128;
  const long big = (long)s.m_tiles * ((NB + 15) / 16);
  int target;
  if (bm <= 32) {
    s.nt = D == 1 ? 4 : 8;
    target = 1024;
  } else {
    s.nt = D == 3 && big >= 384 ? 16 : 8;
    target = 512;
  }
  s.n_tiles = (NB + s.nt - 1) / s.nt;
  s.grid = s.m_tiles * s.n_tiles;
  // split K over workgroups (at least 2 quads each) toward the target, as far
  // as the partial sums fit the workspace
  s.ks = 1;
  while (s.grid * s.ks < target && 2 * s.ks <= KQ / 2 && s.ks < 16 &&
         (size_t)(2 * s.ks) * M * N <= ws_floats)
    s.ks *= 2;
  return s;
}

size_t gemm_splitk_floats(int N, int M, int K, int D) {
  const GemmShape s = plan_gemm(N, M, K, D, (size_t)-1);
  return s.ks > 1 ? (size_t)s.ks * M * N : 0;
}

// The launch shape of these arguments (plan_gemm plus the tuning
// overrides); false when they are invalid.
static bool gemm_plan(const GemvArgs &a, GemmShape &s) {
  if (a.N % 16 || a.K % 128 || a.M < 1 || !a.act_q || !a.act_meta || (a.D != 1 && a.D != 3))
    return false;
  if (a.ss_out || a.arg_parts || a.x_in) return false;  // GEMV-only
  s = plan_gemm(a.N, a.M, a.K, a.D, a.splitk_ws ? a.splitk_ws_floats : 0);
  if (a.rb_override == 1 || a.rb_override == 2 || a.rb_override == 4) {  // tuning
    s.nt = 4 * a.rb_override;
    s.n_tiles = (a.N / 16 + s.nt - 1) / s.nt;
    s.grid = s.m_tiles * s.n_tiles;
  }
  if (a.ksplit_override > 0) {  // tuning: K splits (needs the workspace)
    if ((size_t)a.ksplit_override * a.M * a.N > (a.splitk_ws ? a.splitk_ws_floats : 0) &&
        a.ksplit_override > 1)
      return false;
    s.ks = std::min(a.ksplit_override, a.K / 128);
  }
  return true;
}

// Whether a tile of this shape stages its SwiGLU outputs for the plane
// emission in the kernel's LDS (BM rows x 32 kRB outputs in the two
// activation buffers).
static bool swiglu_stage_fits(int D, const GemmShape &s) {
  const int bm = 16 * s.mt, rb = s.nt / 4;
  const int buf = 4 * D * bm * 32 + 4 * bm * 4;  // ActStage<D, BM>::kBufBytes
  return bm * 32 * rb * 4 <= 2 * buf;
}

// A SwiGLU GEMM without a K split emits down's planes from its own tiles
// (their sums are complete), with no partial sums, when the staging fits.
static bool gemm_direct_emit(const GemvArgs &a, const GemmShape &s) {
  return a.out_q && a.epi == EPI_SWIGLU && s.ks == 1 && swiglu_stage_fits(a.D, s);
}

// Whether the planes a launch emits overlap the planes it reads.
static bool emit_overlaps_input(const GemvArgs &a) {
  const size_t in_bytes = (size_t)(a.K / 32) * a.D * a.M * 32;
  const size_t out_bytes = a.out_q ? (size_t)(a.N / 64) * a.out_D * a.M * 32 : 0;
  return a.out_q && (const int8_t *)a.out_q < a.act_q + in_bytes &&
         a.act_q < (const int8_t *)a.out_q + out_bytes;
}

bool gemm_emit_ok(const GemvArgs &a) {
  GemmShape s;
  if (!a.out_q || !a.out_meta || (a.out_D != 1 && a.out_D != 3) || !gemm_plan(a, s)) return false;
  if (s.ks != 1 && s.ks != 2 && s.ks != 4 && s.ks != 8 && s.ks != 16) return false;
  if (a.epi == EPI_SWIGLU && gemm_direct_emit(a, s) && !emit_overlaps_input(a))
    return (a.N / 2) % 32 == 0;
  if (!a.splitk_ws || (size_t)s.ks * a.M * a.N > a.splitk_ws_floats) return false;
  if (a.epi == EPI_SWIGLU) return (a.N / 2) % 32 == 0;
  if (a.epi == EPI_RESID)
    return a.emit_norm_w && a.resid && a.y && a.N % 32 == 0 && a.N <= 8 * kEmitThreads;
  return false;
}

hipError_t launch_gemm(const GemvArgs &a, hipStream_t st) {
  GemmShape s;
  if (!gemm_plan(a, s)) return hipErrorInvalidValue;
  const bool emit = a.out_q != nullptr;
  if (emit && !gemm_emit_ok(a)) return hipErrorInvalidValue;
  const dim3 grid(s.grid, s.ks), block(256);
  // the last-arriving split finishes its tile (no finishing kernel) when the
  // counters cover the grid, the tile has at most 32 rows and kFoldSplits
  // splits (their partial sums are read at once), and the epilogue is the
  // tile's own: any but the residual plane emission (whole-row RMSNorm);
  // without a K split any tile emits SwiGLU's planes itself (never when the
  // emitted planes overlap the input planes: a finished tile would
  // overwrite what the others still read)
  const bool overlap = emit_overlaps_input(a);
  const bool fold = (a.splitk_counters && s.grid <= a.splitk_counter_count && s.mt <= 2 &&
                     (!emit || (a.epi == EPI_SWIGLU && !overlap)) && (s.ks > 1 || emit) &&
                     s.ks <= kFoldSplits) ||
                    (emit && !overlap && gemm_direct_emit(a, s));
  float *part = s.ks > 1 || (emit && !fold) ? a.splitk_ws : nullptr;
  // (an emission that cannot fold, e.g. into its own input planes, needs
  // the partial sums in the workspace)
  if ((s.ks > 1 || (emit && !fold)) &&
      (!a.splitk_ws || (size_t)s.ks * a.M * a.N > a.splitk_ws_floats))
    return hipErrorInvalidValue;
#define GK_GEMM(DD, RB, BM)                                                                      \
  hipLaunchKernelGGL((gemm_kernel<DD, RB, BM>), grid, block, 0, st, a, s.m_tiles, s.ks, part, \
                     fold ? 1 : 0)
#define GK_GEMM_BM(DD, RB) \
  do {                       \
    if (s.mt == 1) GK_GEMM(DD, RB, 16);                           \
    else if (s.mt == 2) GK_GEMM(DD, RB, 32);                      \
    else GK_GEMM(DD, RB, 64);                                     \
  } while (0)
  if (a.D == 1) {
    if (s.nt == 16) GK_GEMM_BM(1, 4); else if (s.nt == 8) GK_GEMM_BM(1, 2); else GK_GEMM_BM(1, 1);
  } else {
    if (s.nt == 16) GK_GEMM_BM(3, 4); else if (s.nt == 8) GK_GEMM_BM(3, 2); else GK_GEMM_BM(3, 1);
  }
#undef GK_GEMM_BM
#undef GK_GEMM
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || fold) return e;
  if (emit) {
    const float *pc = part;
    const unsigned sw_grid = (unsigned)(((size_t)a.M * (a.N / 2) + 255) / 256);
#define GK_EMIT(KS, DD)                                                                      \
  do {                                                                                      \
    if (a.epi == EPI_SWIGLU)                                                                \
      hipLaunchKernelGGL((splitk_swiglu_emit_kernel<KS, DD>), dim3(sw_grid), dim3(256), 0, \
                         st, a, pc);                                                        \
    else                                                                                    \
      hipLaunchKernelGGL((splitk_resid_emit_kernel<KS, DD>), dim3(a.M), dim3(kEmitThreads), \
                         0, st, a, pc);                                                     \
  } while (0)
#define GK_EMIT_D(KS)                                  \
  do {                                                \
    if (a.out_D == 1) GK_EMIT(KS, 1); else GK_EMIT(KS, 3); \
  } while (0)
    switch (s.ks) {
      case 1: GK_EMIT_D(1); break;
      case 2: GK_EMIT_D(2); break;
      case 4: GK_EMIT_D(4); break;
      case 8: GK_EMIT_D(8); break;
      default: GK_EMIT_D(16); break;
    }
#undef GK_EMIT_D
#undef GK_EMIT
    return hipGetLastError();
  }
  if (s.ks == 1) return e;
  const size_t MN = (size_t)a.M * a.N;
  const dim3 rg((unsigned)((MN + 255) / 256));
  const float *pc = part;
  switch (s.ks) {
    case 2: hipLaunchKernelGGL((splitk_reduce_kernel<2>), rg, dim3(256), 0, st, a, s.ks, pc); break;
    case 4: hipLaunchKernelGGL((splitk_reduce_kernel<4>), rg, dim3(256), 0, st, a, s.ks, pc); break;
    case 8: hipLaunchKernelGGL((splitk_reduce_kernel<8>), rg, dim3(256), 0, st, a, s.ks, pc); break;
    case 16: hipLaunchKernelGGL((splitk_reduce_kernel<16>), rg, dim3(256), 0, st, a, s.ks, pc); break;
    default: hipLaunchKernelGGL((splitk_reduce_kernel<0>), rg, dim3(256), 0, st, a, s.ks, pc); break;
  }
  return hipGetLastError();
}

}  // namespace gk
