// kernels.h — launch interface of the gfx950 kernels (host-callable C++).
//
// Device data layouts shared by the kernels and the host runtime:
//
// INT4 weight tiles (replaces the reference's row-major packed layout,
// int4_weights.zig:79-107; arithmetic unchanged):
//   codes  uint4   [NB = N/16][KQ = K/128][64 lanes]
//          lane l = 16*j + n -> output row 16*nb + n, group g = 4*kq + j;
//          u32 word w (0..3) covers columns k = 32*g + 8*w + b (low nibble of
//          byte b) and k + 4 (high nibble), b = 0..3.
//          Code u decodes to (u - 7) (int4_matmul.zig:22-25).
//   scales uint16  [NB][KQ][64 lanes] = fp16 w_scale[row][g], same lane order.
//
// Activation digit planes (A operand of v_mfma_i32_16x16x32_i8):
//   q      int8   [G][D][M][32]   (D = digit planes: 1 for Q8, 3 for F32)
//   meta   {f32 scale, i32 corr} [G][M]
//   The group dot is  (f32(T - corr) * w_scale) * scale  with
//   T = sum_d 128^(D-1-d) * sum_k u_k * q_d[k]   (u = stored code).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gk {

struct ActMeta {
  float scale;
  int32_t corr;
};

// Destination of emitted activation planes (see the layout above): a
// producer quantises its outputs straight into the next projection's input.
struct PlanesDst {
  int8_t *q;
  ActMeta *meta;
  int D;
};

// Greedy candidate of one span of logits (sampling.zig:55-105, 194-206):
// best (value, lowest index) among its eligible non-NaN entries (i = -1:
// none), whether an eligible entry was NaN, how many entries were eligible,
// whether mask bits beyond the vocabulary were set, and whether logit 0 is
// NaN (the unmasked scan starts from index 0 and never leaves a NaN there).
struct ArgPartial {
  float v;
  int nan_flag;
  long i;
  unsigned long long rows;
  int bad_mask;
  int nan0;
};

enum Epilogue : int {
  EPI_PLAIN = 0,   // y = sum (+ bias)
  EPI_RESID = 1,   // y = resid + sum
  EPI_SWIGLU = 2,  // rows paired gate/up in 8-row halves; y = silu(g) * u
  EPI_QKV = 3,     // q/k RoPE pairs + KV page write
};

// Arguments of the fused QKV epilogue.
struct QkvArgs {
  float *q_out;            // [M][Hq*hd]
  void *kv_pool;           // pages [page][L][2][16][kv_dim]
  int kv_f16;
  const int32_t *page_table;  // [lanes][max_pages]
  int max_pages;
  const int32_t *lane_of_row; // [M] lane id of activation row m
  const int32_t *pos_of_row;  // [M] position of activation row m
  const float *rope_cos, *rope_sin;  // [positions][hd/2]
  int layer, num_layers;
  int num_heads, num_kv_heads, head_dim;
};

struct GemvArgs {
  const uint4 *codes;
  const uint2 *scales;
  int N, K;                 // device rows / columns
  const int8_t *act_q;
  const ActMeta *act_meta;
  int M, D;
  const float *bias;        // [N] logical order (EPI_PLAIN/QKV), may be null
  float *y;                 // EPI_PLAIN/RESID: [M][N]; SWIGLU: [M][N/2]
  const float *resid;       // EPI_RESID
  int epi;
  int ksplit_override;      // force the K split (tuning); 0 = heuristic
  int rb_override;          // row blocks per workgroup with ksplit_override
                            // (GEMM: 2 or 4 forces the row blocks per wave)
  int ksplit;               // set by launch_gemv
  int ksplit_lds_off;       // set by launch_gemv: LDS offset of the SwiGLU plane buffer
  QkvArgs qkv;
  // EPI_SWIGLU only: also (or instead, with y == null) emit the SwiGLU output
  // as digit planes [G][out_D][M][32] + meta [G][M] of width N/2, ready as
  // the next projection's input.
  int8_t *out_q;
  ActMeta *out_meta;
  int out_D;
  // EPI_RESID: also write ss_out [M][grid], each workgroup's sum of y^2 per
  // row, from which the next projection finishes its RMSNorm (deferred).
  float *ss_out;
  // Input mode: with x_in set the kernel builds its planes in LDS from
  // x_in [M][K] (f32), times norm_w when set, instead of reading act_q /
  // act_meta (needs the planes to fit in LDS).
  const float *x_in;
  const float *norm_w;
  // Deferred RMSNorm of the input: the kernel sums in_ss [M][in_ss_count]
  // and scales every output of row m by 1 / sqrt(sum / K + in_eps) before
  // the epilogue (the planes were quantised without that per-row factor).
  const float *in_ss;
  int in_ss_count;
  float in_eps;
  // EPI_PLAIN only, fused greedy head (a reference LM head fused with its
  // argmax over row tiles): every workgroup also reduces its logits of each
  // activation row m to one candidate arg_parts[m * grid + workgroup],
  // honouring the eligibility bits arg_words [M][arg_word_count] when set.
  ArgPartial *arg_parts;
  const uint64_t *arg_words;
  long arg_word_count;
  // With arg_parts and arg_words: a row block none of whose 16 rows is
  // eligible for any activation row streams no weights (its logits are never
  // computed and never candidates) -- the prehead domain mode. y may be null
  // with arg_parts (no logits are stored).
  int prehead;
  // GEMM split-K workspace (floats); null: no K split
  float *splitk_ws;
  size_t splitk_ws_floats;
  // GEMM split-K counters [splitk_counter_count], zero between launches:
  // with them, a tile's K splits meet at a counter and the last to arrive
  // adds the partial sums and runs the tile's epilogue, so no finishing
  // kernel runs (for every epilogue but the residual plane emission, whose
  // RMSNorm needs whole rows)
  unsigned *splitk_counters;
  int splitk_counter_count;
  // GEMM with out_q set (launch_gemm, when gemm_emit_ok): the finishing
  // pass also writes the next projection's digit planes [G][out_D][M][32] +
  // meta. EPI_SWIGLU: the SwiGLU outputs (width N/2); EPI_RESID: y after
  // the RMSNorm with these weights and in_eps (y itself is written too).
  const float *emit_norm_w;
};

// Launch shape of one GEMV: RB row blocks per workgroup, KS waves per row
// block splitting K, U quads in flight per wave, activation planes in LDS
// when they fit.
struct GemvShape {
  int ksplit, rb, waves, grid, unroll;
  bool lds_a;
  size_t lds_bytes;
};
GemvShape plan_gemv(int N, int K, int M, int D);
// The shape launch_gemv uses for these arguments (plan_gemv adjusted for
// emitted planes / fused stages / overrides); grid = workgroup count, which
// is also the number of ss_out partials per row. Returns false if invalid.
bool gemv_launch_shape(const GemvArgs &a, GemvShape *out);

// Prepare activation planes from x [M][K] (f32 or bf16), optionally
// RMS-normalised with weight `norm_w` first (kernels.zig:141-220).
hipError_t launch_prep_act(const void *x, int x_bf16, const float *norm_w, float eps,
                           int M, int K, int D, int8_t *act_q, ActMeta *meta,
                           float *normed_out, hipStream_t st);

hipError_t launch_gemv(const GemvArgs &a, hipStream_t st);

// Row counts up to this run the decode GEMV (K1, with its fused chain
// stages); more rows run the MFMA GEMM (K2). From 3 rows on the GEMM
// chain measured faster for the whole 7B decode step (3, 4, 5 lanes: 2.22,
// 2.27, 2.28 ms per step against 2.82, 2.91, 2.90 with the GEMV's batched
// dot4 at up to 5 rows) and on the C2 shapes at 4 rows except the smallest
// (11008x4096: 12.5 us against 16.2, 18944x3584: 15.2 against 17.0;
// 4096x4096: 8.8 against 8.2).
constexpr int kGemvMaxRows = 2;

// MFMA GEMM (K2) for more than kGemvMaxRows activation rows: same arguments
// and epilogues as launch_gemv without the GEMV-only stages (partial sums of
// squares, fused argmax, input mode; planes only through the finishing pass,
// gemm_emit_ok). Block tile 16*mt activation rows x nt weight row blocks (16
// rows each), 4 waves; ks > 1 splits K over workgroups, which needs
// splitk_ws (ks * M * N floats) and a second, fixed-order reduction kernel.
// ksplit_override / rb_override force the splits / row blocks per wave
// (tuning).
struct GemmShape {
  int mt, nt, m_tiles, n_tiles, grid, ks;
};
GemmShape plan_gemm(int N, int M, int K, int D, size_t ws_floats);
// Workspace floats the GEMM would use for these sizes with no limit.
// True when launch_gemm can emit planes for these arguments (out_q set):
// SwiGLU outputs or residual rows of at most 4096 in whole 32-wide groups,
// a K split of 1, 2, 4, 8 or 16 and a workspace for its partial sums.
bool gemm_emit_ok(const GemvArgs &a);
size_t gemm_splitk_floats(int N, int M, int K, int D);
hipError_t launch_gemm(const GemvArgs &a, hipStream_t st);


hipError_t launch_rmsnorm(const float *x, const float *w, int rows, int dim, float eps,
                          float *out, hipStream_t st);

// Embedding rows out[m] = table[ids[m]]; with ss_out set also
// gather_ss_parts(dim) partial sums of squares per row (deferred RMSNorm).
int gather_ss_parts(int dim);
hipError_t launch_gather_rows(const float *table, const int32_t *ids, int M, int dim, float *out,
                              hipStream_t st, float *ss_out = nullptr);

// Paged GQA decode attention. Writes out [M][Hq*hd]. Scratch must hold
// attention_scratch_floats(...) floats for any M up to max_rows.
size_t attention_scratch_floats(int max_rows, int num_heads, int num_kv_heads, int head_dim,
                                int max_ctx);
hipError_t launch_attention(const float *q, const void *kv_pool, int kv_f16,
                            const int32_t *page_table, int max_pages, const int32_t *lane_of_row,
                            const int32_t *ctx_len, int M, int layer, int num_layers,
                            int num_heads, int num_kv_heads, int head_dim, int max_ctx,
                            float *scratch, float *out, hipStream_t st,
                            PlanesDst emit = PlanesDst{nullptr, nullptr, 1});

// fp16-KV attention with an explicit launch shape: wp positions per wave,
// nw waves per workgroup (tuning; launch_attention picks the shape).
hipError_t launch_attention_f16(const float *q, const void *kv_pool, const int32_t *page_table,
                                int max_pages, const int32_t *lane_of_row, const int32_t *ctx_len,
                                int M, int layer, int num_layers, int num_heads, int num_kv_heads,
                                int head_dim, int max_ctx, float *scratch, float *out,
                                hipStream_t st, int wp, int nw,
                                PlanesDst emit = PlanesDst{nullptr, nullptr, 1});

// Batch-1 decode with fp16 KV: attention fused with the O projection.
// Workgroup (row-block group bg, KV head h) computes the attention of the
// G = Hq / Hkv query heads of KV head h over row 0's whole context, quantises
// it (the O projection's Q8 planes of that K slice, in LDS) and writes
// parts[h][n] = W_o[n, slice h] . attn[slice h] for its NW row blocks of 16
// rows. With y set, the last of a group's Hkv workgroups to finish (a
// counter per group) also writes the projection with its residual,
// y[n] = resid[n] + ((parts[0][n] + parts[1][n]) + ...), and the group's
// sum of y^2 to ss_out[bg] (the next RMSNorm's partial sums), then resets
// its counter to 0.
struct AttnOArgs {
  const float *q;              // [Hq * head_dim] row 0's queries
  const void *kv_pool;         // pages [page][L][2][16][kv_dim], fp16 (f32 with kv_f32)
  const int32_t *page_table;   // [lanes][max_pages]
  int max_pages;
  const int32_t *lane_of_row;  // [1]
  const int32_t *ctx_len;      // [1]
  // optional: row 0 packed in one line, {lane, ctx_len, -, -, then the
  // first row0_pages entries of its page-table row}; read instead of
  // lane_of_row / ctx_len, and instead of the page table when the context
  // fits those pages
  const int32_t *row0;
  int row0_pages;
  int layer, num_layers, num_heads, num_kv_heads, head_dim, max_ctx;
  const uint4 *codes;          // O weights, device tile layout, N x K (K = Hq * head_dim)
  const uint2 *scales;
  int N, K;
  float *parts;                // [num_kv_heads][N]
  const float *resid;          // [N]  (with y)
  float *y;                    // [N]  null: parts only
  float *ss_out;               // [attn_o_groups(N)]
  unsigned *counters;          // [attn_o_groups(N)], 0 between launches
  int kv_f32;                  // 1: f32 KV pages (the reference's storage)
};
constexpr int kMaxAttnOHeads = 8;  // KV heads (partial vectors) at most
// Whether launch_attn_o supports these shapes (head_dim 64 or 128, a K
// slice per KV head of whole 32-column groups).
bool attn_o_ok(const AttnOArgs &a);
// Row-block groups of the fused launch (= ss_out partials, counters).
int attn_o_groups(int N);
hipError_t launch_attn_o(const AttnOArgs &a, hipStream_t st);

// Causal prefill attention (fp16 KV) for one lane's chunk of T consecutive
// positions pos0 .. pos0 + T - 1 whose K/V rows are already in the lane's
// pages; q / out [T][Hq*hd] as launch_attention.
hipError_t launch_attention_prefill(const float *q, const void *kv_pool, const int32_t *page_table,
                                    int max_pages, int lane, int pos0, int T, int layer,
                                    int num_layers, int num_heads, int num_kv_heads, int head_dim,
                                    float *out, hipStream_t st);

// Argmax over rows x n. Eligible variant when words != null. Results to
// `result` [rows] = {index (u64), eligible_rows (u64), status (i32), pad}.
struct ArgmaxResult {
  uint64_t index;
  uint64_t eligible_rows;
  int32_t status;
  int32_t pad;
};
size_t argmax_scratch_bytes(int rows, long n);
// Candidates one fused-head GEMV writes per activation row (its grid size).
int gemv_argmax_parts(int N, int K, int M, int D);
// Final reduction of the fused head's candidates: parts [rows][nparts]; the
// eligible variant (words != null) also counts the eligible rows and checks
// the bits beyond n, as launch_argmax does.
hipError_t launch_argmax_parts(const ArgPartial *parts, int nparts, long n, int rows,
                               const uint64_t *words, long word_count, ArgmaxResult *result,
                               hipStream_t st);
hipError_t launch_argmax(const float *logits, long n, int rows, const uint64_t *words,
                         long word_count, void *scratch, uint32_t *counters,
                         ArgmaxResult *result, hipStream_t st);

}  // namespace gk
