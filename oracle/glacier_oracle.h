/*
 * glacier_oracle.h — CPU restatement of Glacier Engine's text-token-loop
 * numerics (the reference CPU path), used ONLY as a test checker.
 *
 * TEST INFRASTRUCTURE. Nothing in the product library links, loads or calls
 * this code. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may use it, and there only as the checker / the timed CPU
 * baseline, never as a fallback for the GPU path.
 *
 * Every function cites the reference file:line whose algorithm it restates
 * (paths relative to the reference's src/ tree).
 *
 * Parity status per function (what pins it) is listed next to each
 * declaration; "parity unpinned" marks behaviour nothing but the restatement
 * itself fixes (libm last-ulp behaviour of exp/cos/sin/pow and the reduction
 * order of Zig's @reduce on float vectors).
 */
#ifndef GLACIER_ORACLE_H
#define GLACIER_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    GO_OK = 0,
    GO_SHAPE_MISMATCH = 1,     /* TensorError.ShapeMismatch */
    GO_BAD_GROUP_SIZE = 2,     /* quant.zig error.BadGroupSize */
    GO_TRUNCATED = 3,          /* quant.zig TruncatedScales/TruncatedPacked */
    GO_INVALID_MASK = 4,       /* sampling.EligibleArgmaxError.InvalidEligibleMask */
    GO_ELIGIBLE_NAN = 5,       /* sampling.EligibleArgmaxError.EligibleLogitNaN */
    GO_NO_MEMORY = 6,
};

/* Worker threads used by the row-split GEMVs (int4_matmul.zig:3046 row split
 * is bit-identical to serial, so this changes time, never bits). */
void go_set_threads(int n);
int go_get_threads(void);

/* ---- a1: INT4 code (quant.zig:36-191, int4_matmul.zig:22-25) ---------- */
/* pinned: KATs quant.zig:223-255, int4_weights.zig:449-461; round trip. */
int go_int4_quantize(const float *src, size_t n, uint32_t group_size,
                     uint8_t *packed_out, float *scales_out);
int go_int4_dequantize(const uint8_t *packed, size_t packed_len,
                       const float *scales, size_t scale_len,
                       uint32_t group_size, size_t n, float *out);
uint8_t go_read_nibble(const uint8_t *buf, size_t idx);
void go_write_nibble(uint8_t *buf, size_t idx, uint8_t val);
float go_f16_to_f32(uint16_t h);
uint16_t go_f32_to_f16(float f); /* round to nearest even */

/* ---- a2: linearInt4OnTheFly (int4_matmul.zig:215-311) ------------------- */
/* pinned: brute force vs dequantize + f64 dot (2e-6 abs, int4_matmul.zig:3254). */
int go_linear_int4_f32(const float *x, size_t batch,
                       const uint8_t *packed, const float *scales,
                       const float *bias, /* NULL or [out_f] */
                       float *out, size_t out_f, size_t in_f, size_t group_size);

/* ---- a3: Q8 activations (int4_matmul.zig:335-420, :534-560) ------------- */
/* pinned: closed form (exact integer dot per group), vs a2 closeness (:3375). */
int go_q8_quantize(const float *x, size_t in_f, size_t act_group,
                   int8_t *q_out, float *scales_out);
int go_linear_int4_q8(const float *x, size_t batch,
                      const uint8_t *packed, const float *scales,
                      const float *bias, float *out,
                      size_t out_f, size_t in_f, size_t group_size);
/* x86 dispatch of linearInt4WeightQ8 (int4_matmul.zig:422-531): out_f > 65536
 * takes the f32 path (:461-463); otherwise the portable Q8 path, which itself
 * falls back to f32 when in_f > 16384 or > 2048 activation groups (:372-374). */
int go_linear_int4_weight_q8(const float *x, size_t batch,
                             const uint8_t *packed, const float *scales,
                             const float *bias, float *out,
                             size_t out_f, size_t in_f, size_t group_size);

/* ---- a5: rmsNormF32 (kernels.zig:141-220) ------------------------------- */
/* pinned: textbook closed form on integer-valued inputs (exact). */
int go_rmsnorm(const float *x, size_t batch, size_t dim, const float *w,
               float eps, float *out);

/* ---- a8: siluMulF32 (kernels.zig:465-520) ------------------------------- */
void go_silu_mul(const float *gate, const float *up, float *out, size_t n);

/* ---- a6: RopeTable (generate.zig:784-832), direct form forward.zig:353-377 */
/* pinned: KATs forward.zig:1265-1287 (pos 0 identity, pos 1 angle 1 rad),
 * table == direct formula (generate.zig:5616). libm ulp: parity unpinned. */
void go_rope_table(size_t positions, size_t head_dim, float theta,
                   float *cos_out, float *sin_out);
void go_rope_apply(const float *cos_t, const float *sin_t, size_t half_dim,
                   float *row, size_t pos, size_t num_heads, size_t head_dim);
void go_rope_apply_direct(float *row, size_t pos, size_t num_heads,
                          size_t head_dim, float theta);

/* ---- a7: attentionHeadRange (forward.zig:478-533) ----------------------- */
/* Contiguous K/V [kv_seq, kv_dim]; q [q_seq, Hq*hd]. The 4096 context cap of
 * forward.zig:386 is lifted (same algorithm). */
int go_attention(const float *q, size_t q_seq, const float *k, const float *v,
                 size_t kv_seq, float *out, size_t num_heads,
                 size_t num_kv_heads, size_t head_dim);
/* Paged twin (paged_attention.zig:108-210). Page pool layout follows
 * paged_kv_cache.zig:1421-1444: page = [layer][K,V][16 rows][kv_dim].
 * page_table[p] = physical page of logical page p. kv_fp16 != 0 means the
 * pool holds fp16 (uint16) elements, else f32. */
int go_attention_paged(const float *q, size_t q_seq, const void *pool,
                       int kv_fp16, const int32_t *page_table, size_t kv_seq,
                       size_t layer, size_t num_layers, float *out,
                       size_t num_heads, size_t num_kv_heads, size_t head_dim);

/* ---- a12/a13: argmax (sampling.zig:194-206) / argmaxEligible (:55-105) -- */
/* pinned: KATs sampling.zig:223-286. */
size_t go_argmax(const float *v, size_t n);
int go_argmax_eligible(const float *logits, size_t n, const uint64_t *words,
                       size_t word_count, size_t *index_out,
                       size_t *eligible_rows_out);

/* ---- a9-a11: model token loop (generate.zig:1511-1967, 3653-3694,
 * 4665-5613) in the serial oracle mode of prepared_text_session.zig:81-105:
 * num_threads = 1 numerics, Q8 layer projections, f32 LM head, greedy. ---- */
typedef struct {
    const uint8_t *packed;   /* row-major [out_f * in_f / 2], low nibble = even */
    const float *scales;     /* [out_f * in_f / group] */
} go_int4_weight;

typedef struct {
    const float *input_norm;     /* [dim] */
    const float *post_attn_norm; /* [dim] */
    go_int4_weight wq, wk, wv, wo, w_gate, w_up, w_down;
    const float *bq, *bk, *bv;   /* NULL = no bias */
} go_layer;

typedef struct {
    uint32_t num_layers, dim, hidden_dim, num_heads, num_kv_heads, head_dim;
    uint32_t vocab_size, group_size;
    float rms_eps, rope_theta;
    const float *token_embedding; /* [vocab, dim] f32 */
    const float *final_norm;      /* [dim] */
    go_int4_weight lm_head;       /* [vocab, dim] */
    const go_layer *layers;       /* [num_layers] */
    uint32_t kv_fp16;             /* 0: f32 KV rows as the reference stores
                                   * them (paged_kv_cache.zig:1-8); 1: rows
                                   * rounded to fp16 on store (the fp16 page
                                   * pools of the GPU path) */
    uint32_t int4_activation_f32; /* 0: .q8 (generate.zig:925 default, with the
                                   * x86 f32 fallbacks); 1: .f32 for every
                                   * projection and the head */
} go_model;

/* Greedy generate. tokens_out gets max_new tokens. If logits_steps/logits_out
 * are given, the full logits of generated step s (0 = from the prompt) are
 * copied to logits_out[i * vocab] for each i with logits_steps[i] == s.
 * kv_sha256_out (optional) receives logicalKvPrefixSha256 of the final cache
 * (generate.zig:3150-3172); output_sha256_out the tokenSequenceSha256
 * (generate.zig:3193-3203). */
int go_generate(const go_model *m, const uint32_t *prompt, size_t prompt_len,
                size_t max_new, uint32_t *tokens_out,
                const int32_t *logits_steps, size_t n_logits_steps,
                float *logits_out, uint8_t *kv_sha256_out,
                uint8_t *output_sha256_out);
/* go_generate with the decode inputs given: step s >= 1 is fed forced[s - 1]
 * (max_new - 1 tokens) instead of the previous argmax; tokens_out still
 * receives every step's argmax. For comparing two runs at the same context. */
int go_generate_forced(const go_model *m, const uint32_t *prompt, size_t prompt_len,
                       size_t max_new, const uint32_t *forced, uint32_t *tokens_out,
                       const int32_t *logits_steps, size_t n_logits_steps, float *logits_out);

/* One decoder layer at position pos over a contiguous f32 KV cache
 * k_cache/v_cache [max_seq, kv_dim] that already holds pos rows. Writes the
 * new row at pos, and out_row = layer(x_row). (generate.zig:1511-1967) */
int go_forward_layer(const go_model *m, size_t layer, const float *x_row,
                     float *k_cache, float *v_cache, size_t pos,
                     const float *rope_cos, const float *rope_sin,
                     float *out_row);

/* ---- SHA-256 (FIPS 180-4) and the digests that use it ------------------- */
void go_sha256(const uint8_t *data, size_t len, uint8_t out[32]);
typedef struct { uint32_t h[8]; uint64_t len; uint8_t buf[64]; size_t fill; } go_sha256_ctx;
void go_sha256_init(go_sha256_ctx *c);
void go_sha256_update(go_sha256_ctx *c, const void *data, size_t len);
void go_sha256_final(go_sha256_ctx *c, uint8_t out[32]);

/* paged_kv_cache.zig:165-260 deriveCapacityLedger (all sizes in bytes). */
typedef struct {
    uint64_t page_count_capacity, page_elements, page_payload_bytes,
        tensor_capacity_bytes, page_map_bytes, allocation_capacity_bytes,
        contiguous_counterfactual_bytes, capacity_reclaimed_bytes,
        capacity_overhead_bytes, padded_positions;
} go_capacity_ledger;
int go_paged_capacity_ledger(uint64_t num_layers, uint64_t dim,
                             uint64_t max_seq, go_capacity_ledger *out);
/* paged_kv_cache.zig:323-353 */
void go_paged_empty_ownership_digest(uint64_t cache_instance,
                                     uint64_t num_layers, uint64_t dim,
                                     uint64_t max_seq, uint8_t out[32]);
void go_paged_append_ownership_digest(const uint8_t before[32],
                                      uint64_t cache_instance,
                                      uint64_t logical_page,
                                      uint64_t ownership_generation,
                                      uint8_t out[32]);
/* generate.zig:3193-3203 */
/* logicalKvPrefixSha256 (generate.zig:3150-3172); k, v are [L][max_seq][kv_dim]. */
void go_logical_kv_sha256(const float *k, const float *v, size_t L, size_t max_seq, size_t kv_dim,
                          size_t pos, uint8_t out[32]);
void go_token_sequence_sha256(const uint32_t *tokens, size_t n,
                              uint8_t out[32]);

/* Zig std.Random.DefaultPrng (Xoshiro256**) seeding through SplitMix64, as
 * used by generate.zig:5221. Greedy decoding never advances it. */
void go_xoshiro256_init(uint64_t seed, uint64_t s_out[4]);

#ifdef __cplusplus
}
#endif
#endif
