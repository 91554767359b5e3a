/*
 * glacier_hip.h — C ABI of the MI355X (gfx950) device backend for Glacier
 * Engine's text token loop.
 *
 * Conventions follow the reference's Metal extern set
 * (src/backends/metal/backend.zig:506-670): opaque context / weight handles,
 * `int` status returns with 0 = ok, caller-owned buffers with explicit
 * lengths, no ownership transfer of caller pointers, a destroy for every
 * create, and live-object counts for zero-orphan checks
 * (backend.zig:2182-2235). The header uses C types only so that a Zig host
 * can `@cImport` it; HIP streams are passed as `void *` (NULL = the
 * context's own stream).
 *
 * "dev" pointers are device (HBM) addresses; "host" pointers are host
 * memory. Every entry point validates shapes, alignment and handles on the
 * host before it launches anything and publishes nothing on error.
 */
#ifndef GLACIER_HIP_H
#define GLACIER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes -------------------------------------------------------- */
enum glacier_hip_status {
    GLACIER_HIP_OK = 0,
    GLACIER_HIP_SHAPE_MISMATCH = 1,      /* TensorError.ShapeMismatch */
    GLACIER_HIP_DTYPE_UNSUPPORTED = 2,   /* TensorError.DTypeUnsupported */
    GLACIER_HIP_INVALID_ARGUMENT = 3,
    GLACIER_HIP_OUT_OF_MEMORY = 4,
    GLACIER_HIP_DEVICE_ERROR = 5,        /* a HIP runtime call failed */
    GLACIER_HIP_INVALID_MASK = 6,        /* EligibleArgmaxError.InvalidEligibleMask */
    GLACIER_HIP_ELIGIBLE_NAN = 7,        /* EligibleArgmaxError.EligibleLogitNaN */
    GLACIER_HIP_CACHE_FULL = 8,          /* GenerateError.CacheFull / paged CacheFull */
    GLACIER_HIP_NO_DEVICE = 9,
    GLACIER_HIP_INVALID_HANDLE = 10,
    GLACIER_HIP_TRANSACTION_ACTIVE = 11, /* paged_kv_cache Error.TransactionActive */
    GLACIER_HIP_INVALID_TRANSACTION = 12,/* paged_kv_cache Error.InvalidTransaction */
    GLACIER_HIP_BUSY = 13,               /* concurrent submission rejected (int4_executor.zig:2267) */
    GLACIER_HIP_UNSUPPORTED = 14,
    GLACIER_HIP_STALE_HANDLE = 15,       /* LaneWeave Error.StaleHandle */
    GLACIER_HIP_NO_RUNNABLE = 16,        /* LaneWeave Error.NoRunnableRequest */
    GLACIER_HIP_INCOMPLETE_DRAIN = 17,   /* LaneWeave Error.IncompleteDrain */
    GLACIER_HIP_SCHEDULER_CLOSED = 18,   /* LaneWeave Error.SchedulerClosed */
    GLACIER_HIP_SCHEDULER_POISONED = 19, /* LaneWeave Error.InvariantViolation / BankDrift */
    GLACIER_HIP_BAD_IMAGE = 20,          /* a prepared runtime image failed validation
                                          * (the reason: glacier_hip_glrt_info_t.error) */
    GLACIER_HIP_NOT_FOUND = 21,          /* no record with that key */
    GLACIER_HIP_INVALID_CHECKPOINT = 22, /* a page image or checkpoint restore was rejected
                                          * (the reason: glacier_hip_page_image_v1_t.error) */
    GLACIER_HIP_SERVICE_IN_FLIGHT = 23,  /* LaneWeave Error.ServiceInFlight */
    GLACIER_HIP_STALE_SERVICE_PERMIT = 24, /* LaneWeave Error.StaleServicePermit */
    GLACIER_HIP_SINK_REJECTED = 25,      /* a publication sink refused a wave's stages */
};

/* ---- element types / activation modes ------------------------------------ */
enum glacier_hip_dtype {
    GLACIER_HIP_F32 = 0,
    GLACIER_HIP_F16 = 1,
    GLACIER_HIP_BF16 = 2,
};

/* How the INT4 GEMV treats activations.
 *  Q8   — the reference's blockwise Q8 path (int4_matmul.zig:335-420): per
 *         32-element group s = max|x|/127, q = clamp(round(x/s), +-127), exact
 *         integer dot per group, f32 across groups.
 *  F32  — the reference's f32-activation path (int4_matmul.zig:215-311),
 *         computed to ~2^-22 relative accuracy (three 7-bit digit planes).
 *  AUTO — the reference's x86 dispatch (int4_matmul.zig:372-374,461-463):
 *         F32 when out_f > 65536 or in_f > 16384, else Q8. */
enum glacier_hip_activation {
    GLACIER_HIP_ACT_Q8 = 0,
    GLACIER_HIP_ACT_F32 = 1,
    GLACIER_HIP_ACT_AUTO = 2,
};

/* ---- opaque handles ------------------------------------------------------ */
typedef struct glacier_hip_context glacier_hip_context;
typedef struct glacier_hip_int4_weight glacier_hip_int4_weight;
typedef struct glacier_hip_model glacier_hip_model;
typedef struct glacier_hip_session glacier_hip_session;

/* ---- context (backend.zig:506-531: init / deinit / device_info /
 *      allocation_limits) -------------------------------------------------- */
typedef struct {
    char name[64];
    char arch[32];             /* "gfx950" */
    uint32_t compute_units;
    uint32_t wavefront_size;
    uint64_t total_global_bytes;
    uint64_t max_single_allocation_bytes;
    uint32_t lds_bytes_per_block;
    uint32_t l2_bytes;
    uint32_t clock_khz;
    uint32_t memory_clock_khz;
    uint32_t memory_bus_width_bits;
    uint32_t device_ordinal;
} glacier_hip_device_info_t;

typedef struct {
    uint64_t max_single_allocation_bytes;
    uint64_t max_total_device_bytes;
    uint64_t allocation_granularity_bytes;
    uint64_t max_queue_slots;
} glacier_hip_allocation_limits_t;

glacier_hip_context *glacier_hip_init(int device_ordinal);
int glacier_hip_deinit(glacier_hip_context *ctx);
int glacier_hip_device_info(glacier_hip_context *ctx, glacier_hip_device_info_t *out);
int glacier_hip_allocation_limits(glacier_hip_context *ctx, glacier_hip_allocation_limits_t *out);
/* Last HIP error string recorded on this context ("" if none). */
const char *glacier_hip_last_error(glacier_hip_context *ctx);
/* Synchronize the context stream. */
int glacier_hip_synchronize(glacier_hip_context *ctx);

/* ---- device capability (device_capability_contract.zig:132-150,
 *      capabilityRootV1 :331-350) ------------------------------------------ */
typedef struct {
    uint64_t abi_version;            /* 0x4744434100000001 */
    uint64_t backend_kind;           /* 3 = portable_compute */
    uint64_t device_class;           /* 2 = accelerator */
    uint64_t operation_profile_bits; /* matvec_int4_f32_bounded (1<<2) */
    uint64_t operator_bits;
    uint64_t element_type_bits;
    uint64_t numerical_policy_bits;
    uint64_t feature_bits;
    uint64_t max_single_allocation_bytes;
    uint64_t max_total_device_bytes;
    uint64_t max_queue_slots;
    uint8_t backend_sha256[32];
    uint8_t device_sha256[32];
    uint8_t driver_sha256[32];
    uint8_t placement_sha256[32];
    uint8_t capability_sha256[32];   /* sealed root over every field above */
} glacier_hip_device_capability_v1_t;

int glacier_hip_device_capability_v1(glacier_hip_context *ctx,
                                     glacier_hip_device_capability_v1_t *out);

/* ---- buffers (backend.zig:532-550) and the allocation lease adapter
 *      (device_allocation_lease.zig:323-348: quote is side-effect free,
 *      a failed allocate creates nothing, a failed free leaves it live) ---- */
typedef struct {
    uint64_t id;                 /* 0 = none */
    uint64_t requested_bytes;
    uint64_t charged_bytes;      /* granularity-rounded */
} glacier_hip_buffer_token_t;

typedef struct {
    uint64_t id;
    uint64_t requested_bytes;
    uint64_t charged_bytes;
    uint64_t device_address;     /* HBM address, for kernels and tests */
} glacier_hip_buffer_info_t;

typedef struct {
    uint64_t requested_bytes;
    uint64_t charged_bytes;
    uint64_t context_epoch;      /* binds the quote to this context */
} glacier_hip_allocation_quote_t;

int glacier_hip_buffer_create(glacier_hip_context *ctx, uint64_t requested_length,
                              glacier_hip_buffer_token_t *out);
int glacier_hip_buffer_info(glacier_hip_context *ctx, const glacier_hip_buffer_token_t *token,
                            glacier_hip_buffer_info_t *out);
int glacier_hip_buffer_release(glacier_hip_context *ctx, const glacier_hip_buffer_token_t *token);
int glacier_hip_live_buffer_count(glacier_hip_context *ctx, uint64_t *out);
int glacier_hip_allocation_quote(glacier_hip_context *ctx, uint64_t requested_bytes,
                                 glacier_hip_allocation_quote_t *out);
int glacier_hip_allocation_allocate(glacier_hip_context *ctx,
                                    const glacier_hip_allocation_quote_t *quote,
                                    glacier_hip_buffer_token_t *out);
int glacier_hip_allocation_free(glacier_hip_context *ctx, const glacier_hip_buffer_token_t *token);
/* Device bytes the context holds for every object it created (buffers,
 * weights, models, sessions, scratch): requested and charged at the
 * allocation granularity. Models and sessions quote their exact charge
 * (glacier_hip_model_quote / glacier_hip_session_quote) without allocating,
 * so a host charges its ResourceBank before it creates them
 * (device_allocation_lease.zig:1-14). */
int glacier_hip_live_device_bytes(glacier_hip_context *ctx, uint64_t *requested_out,
                                  uint64_t *charged_out);

/* ---- persistent INT4 weights (backend.zig:570-598) -----------------------
 * `packed` is the reference's row-major layout [out_f * in_f / 2] bytes, low
 * nibble = even element, code u decodes to (u - 7) * scale (quant.zig:50-54,
 * int4_matmul.zig:22-25). Scales are row-major [out_f][in_f / group]. The
 * weight is re-laid out on the device into 16-row x 128-column MFMA tiles;
 * the arithmetic is unchanged. Requirements: group_size == 32,
 * out_f % 16 == 0, in_f % 128 == 0. */
glacier_hip_int4_weight *glacier_hip_int4_weight_create(
    glacier_hip_context *ctx, const uint8_t *packed, uint64_t packed_bytes,
    const float *scales, uint64_t scale_count, uint32_t group_size,
    uint32_t in_features, uint32_t out_features);
/* Same with IEEE fp16 scales (the reference's optional fp16 mirror,
 * int4_weights.zig:346-384). */
glacier_hip_int4_weight *glacier_hip_int4_weight_create_f16scales(
    glacier_hip_context *ctx, const uint8_t *packed, uint64_t packed_bytes,
    const uint16_t *scales_f16, uint64_t scale_count, uint32_t group_size,
    uint32_t in_features, uint32_t out_features);
void glacier_hip_int4_weight_destroy(glacier_hip_int4_weight *weight);
int glacier_hip_live_weight_count(glacier_hip_context *ctx, uint64_t *out);
/* Bytes the weight occupies in HBM (codes + fp16 scales). */
uint64_t glacier_hip_int4_weight_device_bytes(const glacier_hip_int4_weight *weight);

/* Synchronous host-buffer matvec (glacier_metal_int4_matvec_dispatch,
 * backend.zig:599-606): y[out_f] = W x, one row, F32 activation semantics. */
int glacier_hip_int4_matvec_dispatch(glacier_hip_context *ctx, glacier_hip_int4_weight *weight,
                                     const float *input, uint64_t input_count,
                                     float *output, uint64_t output_count);

/* ---- asynchronous registered-buffer dispatch (backend.zig:600-668;
 *      shim.m registered_buffers_submit_async .. int4_registered_output_read)
 * submit_async copies a reference-layout INT4 weight, its f32 scales and an
 * f32 input into four registered buffers (buffer_create tokens), queues the
 * f32-semantics matvec into the output buffer on the context stream and
 * returns a command token bound to the caller's 32-byte submission binding.
 * poll / wait report the command (pending, completed, error) with GPU start
 * and end times (seconds from the context's creation); output_read copies the
 * output after completion; finalize retires a completed command whose exact
 * completion record the caller presents. Until finalize the command keeps
 * its buffers alive (buffer_release returns BUSY). Status codes: OK,
 * INVALID_ARGUMENT (malformed call), INVALID_HANDLE (no such live command for
 * this token and binding), INVALID_TRANSACTION (not completed, or the
 * completion record differs), SHAPE_MISMATCH (buffer too small / not the
 * command's output). */
typedef struct {
    uint64_t context_nonce[4];
    uint64_t generation;             /* 0 = none */
} glacier_hip_command_token_t;          /* MetalCommandToken (backend.zig:101-112) */

enum glacier_hip_command_state {
    GLACIER_HIP_COMMAND_PENDING = 1, GLACIER_HIP_COMMAND_COMPLETED = 2,
    GLACIER_HIP_COMMAND_ERROR = 3, GLACIER_HIP_COMMAND_UNKNOWN = 4,
};

typedef struct {
    uint64_t abi_version;            /* 0x474d415300000001 */
    glacier_hip_command_token_t token;
    uint8_t submission_binding[32];
    uint32_t disposition;            /* 1 submitted, 2 submitted_or_ambiguous */
    uint32_t reserved;
} glacier_hip_async_submission_t;       /* MetalAsyncSubmission (:135-142) */

typedef struct {
    uint64_t abi_version;            /* 0x474d414300000001 */
    glacier_hip_command_token_t token;
    uint8_t submission_binding[32];
    uint64_t current_allocated_before, current_allocated_after;  /* live buffer bytes */
    double gpu_start_time, gpu_end_time;
    int64_t error_code;              /* hipError_t of a failed command */
    uint32_t state;                  /* glacier_hip_command_state */
    uint32_t command_status, error_domain_kind, error_present, callback_fault, reserved;
} glacier_hip_async_completion_t;       /* MetalAsyncCompletion (:144-159) */

int glacier_hip_int4_registered_buffers_submit_async(
    glacier_hip_context *ctx, const glacier_hip_buffer_token_t *packed_token,
    const glacier_hip_buffer_token_t *scales_token, const glacier_hip_buffer_token_t *input_token,
    const glacier_hip_buffer_token_t *output_token, const uint8_t *packed_weights,
    uint64_t packed_bytes, const float *scales, uint64_t scale_count, const float *input,
    uint64_t input_count, uint32_t group_size, uint32_t in_features, uint32_t out_features,
    const uint8_t submission_binding[32], glacier_hip_async_submission_t *submission);
int glacier_hip_registered_dispatch_poll(glacier_hip_context *ctx,
                                         const glacier_hip_command_token_t *token,
                                         const uint8_t submission_binding[32],
                                         glacier_hip_async_completion_t *completion);
int glacier_hip_registered_dispatch_wait(glacier_hip_context *ctx,
                                         const glacier_hip_command_token_t *token,
                                         const uint8_t submission_binding[32],
                                         glacier_hip_async_completion_t *completion);
int glacier_hip_registered_dispatch_finalize(glacier_hip_context *ctx,
                                             const glacier_hip_command_token_t *token,
                                             const uint8_t submission_binding[32],
                                             const glacier_hip_async_completion_t *expected);
int glacier_hip_int4_registered_output_read(glacier_hip_context *ctx,
                                            const glacier_hip_command_token_t *token,
                                            const uint8_t submission_binding[32],
                                            const glacier_hip_async_completion_t *expected,
                                            const glacier_hip_buffer_token_t *output_token,
                                            float *output, uint64_t output_count);
/* Submitted commands not yet finalized (backend.zig:664). */
int glacier_hip_live_command_count(glacier_hip_context *ctx, uint64_t *out);

/* Device-resident batched projection: y[m][out_f] = x[m][in_f] W^T
 * (+ bias[out_f]), m in 1..GLACIER_HIP_MAX_ROWS. x is f32 or bf16 (x_dtype),
 * y is f32. Replaces linearInt4WeightQ8 / linearInt4Weight
 * (int4_matmul.zig:422-531, 2957-2981) for one projection over m rows: up
 * to 2 rows run the decode GEMV; more rows (decode batches, prompt chunks,
 * the packed batch of
 * forwardLayerPackedBatch, generate.zig:2105) the MFMA GEMM; both compute
 * every row with the same per-group arithmetic. Asynchronous on `stream`;
 * each stream has its own activation planes and split-K workspace (grown on
 * the first call with larger sizes; later calls only launch kernels). */
#define GLACIER_HIP_MAX_ROWS 65536u
int glacier_hip_int4_gemv(glacier_hip_context *ctx, glacier_hip_int4_weight *weight,
                          const void *x_dev, int x_dtype, uint32_t m,
                          const float *bias_dev, float *y_dev, int activation,
                          void *stream);

/* glacier_hip_int4_gemv without any allocation. No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). Its
 * activation planes and GEMM split-K partial sums live in one fixed 16 MiB
 * array per GPU (4 MiB of planes, 12 MiB of partial sums), held from the
 * library's load until the process ends; m is at most 64 rows and the planes
 * of m x in_f at most 4 MiB (SHAPE_MISMATCH otherwise, nothing launched).
 * Same arithmetic as glacier_hip_int4_gemv (a smaller workspace may lower a
 * K split, which reorders only the f32 sum across splits). Every call on one
 * GPU shares that array: calls that overlap on a GPU (from several threads
 * or contexts, or on several streams) race; each call leaves its contents
 * behind and needs nothing cleared. Asynchronous on `stream`. */
int glacier_hip_int4_gemv_noalloc(glacier_hip_context *ctx, glacier_hip_int4_weight *weight,
                                  const void *x_dev, int x_dtype, uint32_t m,
                                  const float *bias_dev, float *y_dev, int activation,
                                  void *stream);

/* The same projection in two phases, as the reference splits it into
 * quantizeQ8Activation (int4_matmul.zig:537-560, glacier_q8_activation_quantize
 * int4_neon.c:453-486) and linearInt4WeightQ8Prepared (int4_matmul.zig:771):
 * the activation is converted once into device "digit planes" that several
 * projections with the same in_f can share. activation must be Q8 or F32
 * (F32 = three digit planes). act_dev must hold
 * glacier_hip_activation_bytes(m, in_f, activation) bytes. */
uint64_t glacier_hip_activation_bytes(uint32_t m, uint32_t in_f, int activation);
int glacier_hip_activation_prepare(glacier_hip_context *ctx, const void *x_dev, int x_dtype,
                                   uint32_t m, uint32_t in_f, int activation,
                                   void *act_dev, void *stream);
int glacier_hip_int4_gemv_prepared(glacier_hip_context *ctx, glacier_hip_int4_weight *weight,
                                   const void *act_dev, uint32_t m, int activation,
                                   const float *bias_dev, float *y_dev, void *stream);

/* ---- fused RMSNorm (kernels.zig:141-220) -------------------------------- */
int glacier_hip_rmsnorm(glacier_hip_context *ctx, const float *x_dev, const float *w_dev,
                        uint32_t rows, uint32_t dim, float eps, float *out_dev, void *stream);

/* ---- paged-KV GQA decode attention (forward.zig:478-533,
 *      paged_attention.zig:108-210) ----------------------------------------
 * One query row per lane. kv_pool_dev holds pages laid out as the reference's
 * page payload (paged_kv_cache.zig:1421-1444):
 *   page[layer][K=0,V=1][16 positions][num_kv_heads * head_dim]
 * in f32 or f16 (kv_dtype). page_table_dev is [lanes][max_pages_per_lane]
 * int32 physical page ids; ctx_lens_dev[lanes] int32 = attended positions
 * (the new row included). q_dev/out_dev are [lanes][num_heads * head_dim],
 * lanes <= 64. Asynchronous on `stream`; after a first call with the same or
 * larger sizes it only launches kernels (capturable in a HIP graph). */
int glacier_hip_paged_attention(glacier_hip_context *ctx, const float *q_dev,
                                const void *kv_pool_dev, int kv_dtype,
                                const int32_t *page_table_dev, uint32_t max_pages_per_lane,
                                const int32_t *ctx_lens_dev, uint32_t lanes,
                                uint32_t layer, uint32_t num_layers, uint32_t num_heads,
                                uint32_t num_kv_heads, uint32_t head_dim,
                                uint32_t max_ctx, float *out_dev, void *stream);

/* Causal attention for a chunk of T query rows of one lane at positions
 * pos0 .. pos0 + T - 1 (attentionMultiHead with q_seq = T and query_start =
 * pos0, forward.zig:478-533 / paged_attention.zig:108-210): row i attends to
 * positions 0 .. pos0 + i, whose K/V rows are already in the lane's pages.
 * fp16 pools only (the prompt-chunk kernel); page_table_dev is that lane's
 * int32[max_pages] physical page ids; q_dev / out_dev [T][num_heads * head_dim].
 * Asynchronous on `stream`; launches only (no scratch). */
int glacier_hip_paged_attention_prefill(glacier_hip_context *ctx, const float *q_dev,
                                        const void *kv_pool_dev, const int32_t *page_table_dev,
                                        uint32_t max_pages, uint32_t pos0, uint32_t T,
                                        uint32_t layer, uint32_t num_layers, uint32_t num_heads,
                                        uint32_t num_kv_heads, uint32_t head_dim, float *out_dev,
                                        void *stream);

/* Attention of one decode row fused with the O projection (the one-lane
 * decode step's launch; the reference runs attention then the O matvec,
 * forward.zig:478-533 and generate.zig:1561): for row 0 (page-table row 0,
 * ctx_len_dev[0] attended positions of fp16 pages at `layer`) every KV head
 * h computes the attention of its num_heads / num_kv_heads query heads,
 * quantises that slice of the attention output to Q8 groups of 32 (the O
 * projection's activation quantiser, int4_matmul.zig:380-398) and writes
 * parts_dev[h][n] = sum over the slice of W_o[n][k] * a[k] (Q8 group
 * arithmetic of glacier_hip_int4_gemv). The sum over h is the O projection
 * of the attention output. num_kv_heads <= 8, head_dim 64 or 128, a slice
 * of whole 32-column groups (with head_dim 64 a slice may share a 128-column
 * tile with its neighbour); o_weight is [out_f][num_heads * head_dim].
 * Asynchronous on `stream`; launches only. */
int glacier_hip_paged_attention_o(glacier_hip_context *ctx, const float *q_dev,
                                  const void *kv_pool_dev, const int32_t *page_table_dev,
                                  uint32_t max_pages, const int32_t *ctx_len_dev, uint32_t layer,
                                  uint32_t num_layers, uint32_t num_heads, uint32_t num_kv_heads,
                                  uint32_t head_dim, uint32_t max_ctx,
                                  const glacier_hip_int4_weight *o_weight, float *parts_dev,
                                  void *stream);

/* ---- greedy samplers (sampling.zig:194-206, :55-105) ---------------------
 * rows independent logit rows of length n. Results are written to host
 * memory after the call synchronizes the stream. */
typedef struct {
    uint64_t token_index;
    uint64_t eligible_rows;
    int32_t status;              /* GLACIER_HIP_OK / _INVALID_MASK / _ELIGIBLE_NAN */
    int32_t reserved;
} glacier_hip_argmax_result_t;

int glacier_hip_argmax(glacier_hip_context *ctx, const float *logits_dev, uint64_t n,
                       uint32_t rows, uint64_t *index_host, void *stream);
/* words_dev: [rows][word_count] u64 LSB-first eligibility bits;
 * word_count must equal ceil(n / 64) (checked on the host). */
int glacier_hip_eligible_argmax(glacier_hip_context *ctx, const float *logits_dev, uint64_t n,
                                const uint64_t *words_dev, uint64_t word_count, uint32_t rows,
                                glacier_hip_argmax_result_t *results_host, void *stream);

/* Prehead eligible greedy projection: Executor.runGreedyArgmaxEligible
 * (int4_executor.zig:1859-1967) with the EligibleGreedyContext tile walk
 * (:968-1150) and its result (EligibleGreedyResult, :786-801). The argmax of
 * x . W^T over the rows whose bit is set in words_host (LSB-first, exactly
 * ceil(out_f / 64) words, no bits past out_f, at least one set), lowest
 * index on ties. Row blocks of 16 with no eligible row stream no weights;
 * full-vocabulary logits never exist. x_dev: [in_f] f32 on the device,
 * every element finite; activation GLACIER_HIP_ACT_AUTO or _Q8 (the
 * reference executor's Q8 arithmetic) or _F32. As in the reference, every
 * failure -- a wrong word count, bits past out_f, an empty mask, a
 * non-finite input, an eligible NaN logit -- is GLACIER_HIP_SHAPE_MISMATCH,
 * and a rejected call writes nothing. The counts are the reference's:
 * producer_rows = 4 x (4-row groups holding an eligible row; a fully
 * eligible 64-row tile counts whole), producer_runs = maximal runs of such
 * groups per 64-row tile, skipped = out_f - producer_rows, overcomputed =
 * producer_rows - eligible_rows; device_rows is what this device streamed
 * (16-row blocks holding an eligible row). Synchronous. */
typedef struct {
    uint64_t token_index;
    uint64_t eligible_rows;
    uint64_t producer_rows;
    uint64_t skipped_rows;
    uint64_t overcomputed_rows;
    uint64_t producer_runs;
    uint64_t device_rows;
} glacier_hip_eligible_greedy_result_t;

int glacier_hip_int4_eligible_greedy(glacier_hip_context *ctx, glacier_hip_int4_weight *w,
                                     const float *x_dev, uint32_t in_f,
                                     const uint64_t *words_host, uint64_t word_count,
                                     int activation, glacier_hip_eligible_greedy_result_t *out,
                                     void *stream);

/* ---- model: Llama/Qwen pre-norm decoder with INT4 projections ------------
 * (forward.zig:36-81 LayerWeights/LayerConfig, loader.zig:31 ModelConfig) */
typedef struct {
    uint32_t num_layers, dim, hidden_dim, num_heads, num_kv_heads, head_dim;
    uint32_t vocab_size, group_size;
    float rms_eps, rope_theta;
} glacier_hip_model_config_t;

/* Host-side tensors of one layer in the reference's layouts. Biases may be
 * NULL. Scales are f32 (fp16 values are accepted exactly). */
typedef struct {
    const float *input_norm, *post_attn_norm;              /* [dim] */
    const uint8_t *wq, *wk, *wv, *wo, *w_gate, *w_up, *w_down;
    const float *sq, *sk, *sv, *so, *s_gate, *s_up, *s_down;
    const float *bq, *bk, *bv;
} glacier_hip_layer_host_t;

glacier_hip_model *glacier_hip_model_create(glacier_hip_context *ctx,
                                            const glacier_hip_model_config_t *cfg);
int glacier_hip_model_set_layer(glacier_hip_model *model, uint32_t layer,
                                const glacier_hip_layer_host_t *w);
int glacier_hip_model_set_globals(glacier_hip_model *model, const float *token_embedding,
                                  const float *final_norm, const uint8_t *lm_head_packed,
                                  const float *lm_head_scales);
/* Random-init every tensor from `seed` with the synthetic generator below
 * (host-generated, then uploaded). */
int glacier_hip_model_init_random(glacier_hip_model *model, uint64_t seed);
void glacier_hip_model_destroy(glacier_hip_model *model);
uint64_t glacier_hip_model_weight_bytes(const glacier_hip_model *model);
/* The device bytes a model of `cfg` takes once every layer and the globals
 * are set (side-effect free). */
int glacier_hip_model_quote(glacier_hip_context *ctx, const glacier_hip_model_config_t *cfg,
                            int with_qkv_bias, glacier_hip_allocation_quote_t *out);

/* ---- sessions: paged KV pool + lanes, the per-token step -----------------
 * A session owns a pool of KV pages (each holds 16 positions of every layer,
 * paged_kv_cache.zig:1-8) and up to max_lanes request-local page tables.
 * Each decode step runs one token for each listed lane: embedding gather ->
 * layers -> final norm -> LM head -> greedy argmax (optionally eligible).
 * The per-token publication is atomic (paged_token_txn.zig:346-600): the
 * kernels write K/V rows into a provisional row of the lane's current page;
 * only after the argmax result is read back does the host commit, per lane,
 * the KV length + page-map root, the sampling counter and the output token.
 * On any error nothing of that step is committed. */
typedef struct {
    uint32_t max_lanes;
    uint32_t max_positions;      /* per lane */
    uint32_t total_pages;        /* pool size; 0 = max_lanes * ceil(max_positions/16) */
    int32_t kv_dtype;            /* GLACIER_HIP_F32 or GLACIER_HIP_F16 */
    int32_t layer_activation;    /* GLACIER_HIP_ACT_*; AUTO = reference x86 dispatch */
    int32_t head_activation;     /* usually AUTO (=> F32 for V > 65536) */
    int32_t use_graph;           /* sealed step plans: 0 = plan and launch every step;
                                  * 1 = capture each step shape once and replay its
                                  * recorded kernel launches; 2 = replay the captured
                                  * hipGraph */
    int32_t prefill_chunk;       /* prompt rows per prefill launch sequence;
                                  * 0 = min(max_positions, 2048) */
    int32_t split_attention_o;   /* 0: a one-lane decode step at a context of up to
                                  * 256 positions (fp16 KV) runs attention and the O
                                  * projection as one launch; 1: always two */
} glacier_hip_session_options_t;

typedef struct {
    uint64_t abi_version;        /* 0x47504d5200000001 */
    uint64_t cache_instance;
    uint64_t generation;
    uint64_t committed_len;
    uint64_t committed_pages;
    uint8_t ownership_sha256[32];
} glacier_hip_page_map_root_t;     /* PageMapRootV1 (paged_kv_cache.zig:64-71) */

typedef struct {
    uint64_t abi_version;        /* 0x4750524600000001 */
    uint64_t cache_instance;
    uint64_t logical_page;
    uint64_t ownership_generation;
} glacier_hip_page_ref_t;          /* PageRefV1 (paged_kv_cache.zig:55-60) */

typedef struct {
    uint64_t abi_version;        /* 0x4750525400000001 */
    uint64_t cache_id;           /* identity of the page map that staged the row */
    uint64_t cache_instance;
    uint64_t generation;         /* row transaction generation */
    uint64_t base_len;
    uint64_t row_count;          /* 1 */
    uint64_t root_before_generation;
    uint64_t root_after_generation;
    glacier_hip_page_ref_t page_ref;
} glacier_hip_row_txn_mark_t;      /* RowTxnMark (paged_kv_cache.zig:255-265) */

typedef struct {
    uint64_t page_count_capacity, allocated_pages, committed_pages, provisional_pages;
    uint64_t reusable_pages, page_map_bytes, resident_tensor_payload_bytes;
    uint64_t resident_allocation_bytes, committed_tensor_payload_bytes;
} glacier_hip_kv_resident_ledger_t; /* ResidentLedger (paged_kv_cache.zig:92-102), f32 payloads */

/* ---- host page map of one paged KV cache (no device) ----------------------
 * The page-map half of the reference's PagedKVCache (paged_kv_cache.zig:
 * 511-1520) over a pool of `pool_pages` payload slots: beginRow (:1006-1072)
 * consumes the next page ownership generation (on a page's row 0) and the
 * next root generation whether or not the row commits; abortRow (:1146-1158)
 * only clears the page's ownership generation, so a retry reuses the payload
 * under a fresh generation; reset (:1162-1182) invalidates every root and
 * page ref and keeps the payloads. Sessions run the same transaction for
 * each lane over their device pool. One staged row at a time. */
typedef struct glacier_hip_kv_pages glacier_hip_kv_pages;
glacier_hip_kv_pages *glacier_hip_kv_pages_create(uint32_t num_layers, uint32_t kv_dim,
                                                  uint32_t max_seq, uint32_t pool_pages);
void glacier_hip_kv_pages_destroy(glacier_hip_kv_pages *p);
int glacier_hip_kv_pages_begin_row(glacier_hip_kv_pages *p, glacier_hip_row_txn_mark_t *mark_out);
int glacier_hip_kv_pages_commit_row(glacier_hip_kv_pages *p, const glacier_hip_row_txn_mark_t *mark);
int glacier_hip_kv_pages_abort_row(glacier_hip_kv_pages *p, const glacier_hip_row_txn_mark_t *mark);
/* prepareCommit (:1105-1118): the roots the staged row moves between. */
int glacier_hip_kv_pages_staged_root(glacier_hip_kv_pages *p, const glacier_hip_row_txn_mark_t *mark,
                                     glacier_hip_page_map_root_t *before,
                                     glacier_hip_page_map_root_t *after);
int glacier_hip_kv_pages_reset(glacier_hip_kv_pages *p);
int glacier_hip_kv_pages_root(glacier_hip_kv_pages *p, glacier_hip_page_map_root_t *out);
/* Payload slot (-1 = none) and ownership generation (0 = not owned) of a logical page. */
int glacier_hip_kv_pages_page(glacier_hip_kv_pages *p, uint32_t logical_page,
                              int32_t *physical_out, uint64_t *ownership_generation_out);
/* validateCommittedPageRef (:944-957): OK or INVALID_TRANSACTION. */
int glacier_hip_kv_pages_validate_page_ref(glacier_hip_kv_pages *p, const glacier_hip_page_ref_t *ref);
int glacier_hip_kv_pages_ledger(glacier_hip_kv_pages *p, glacier_hip_kv_resident_ledger_t *out);

typedef struct {
    uint64_t kv_positions;
    uint64_t published_tokens;
    uint64_t sampling_calls;
    uint64_t rng_state[4];       /* DefaultPrng state; greedy never advances it */
    uint8_t output_sha256[32];   /* tokenSequenceSha256 (generate.zig:3193) */
} glacier_hip_lane_state_t;

glacier_hip_session *glacier_hip_session_create(glacier_hip_model *model,
                                                const glacier_hip_session_options_t *opts);
void glacier_hip_session_destroy(glacier_hip_session *s);
/* The device bytes glacier_hip_session_create would allocate for these
 * options (side-effect free; computed from the same allocation list). */
int glacier_hip_session_quote(glacier_hip_model *model, const glacier_hip_session_options_t *opts,
                              glacier_hip_allocation_quote_t *out);
/* Start a request on `lane` (resets its cache and counters). */
int glacier_hip_session_lane_begin(glacier_hip_session *s, uint32_t lane, uint64_t seed);
/* Prefill: run `n` prompt tokens on `lane` and produce the first greedy
 * token (generate.zig:5080-5160). logits_host: optional [vocab]. The prompt
 * runs in chunks of up to prefill_chunk rows: every projection of a chunk is
 * one MFMA GEMM over its rows, attention is causal per row over the lane's
 * pages, and only the last prompt row goes through the LM head. Each row is
 * computed as the reference's token-at-a-time prefill computes it; a chunk's
 * KV rows commit together once the chunk has run, and rows of earlier chunks
 * stay committed if a later chunk fails (the reference commits per token). */
int glacier_hip_session_prefill(glacier_hip_session *s, uint32_t lane, const uint32_t *tokens,
                                uint32_t n, uint32_t *first_token, float *logits_host);
/* One decode step for `count` lanes: lanes[i] consumes tokens[i] at its next
 * position. next_tokens receives the greedy result per lane. logits_host:
 * optional [count][vocab]. eligible_words_host: optional
 * [count][ceil(vocab/64)] masks (sampling.zig:55-105 semantics). */
int glacier_hip_session_decode_step(glacier_hip_session *s, const uint32_t *lanes,
                                    const uint32_t *tokens, uint32_t count,
                                    const uint64_t *eligible_words_host,
                                    uint32_t *next_tokens, float *logits_host);
int glacier_hip_session_lane_root(glacier_hip_session *s, uint32_t lane,
                                  glacier_hip_page_map_root_t *out);
int glacier_hip_session_lane_state(glacier_hip_session *s, uint32_t lane,
                                   glacier_hip_lane_state_t *out);
/* Logical KV digest of a lane (logicalKvPrefixSha256, generate.zig:3150),
 * computed over K/V values widened to f32 bit patterns. */
int glacier_hip_session_lane_kv_sha256(glacier_hip_session *s, uint32_t lane, uint8_t out[32]);
/* Copy one K or V row (f32) of a lane out of the paged pool. */
int glacier_hip_session_read_kv_row(glacier_hip_session *s, uint32_t lane, uint32_t layer,
                                    int value, uint32_t position, float *out_host);
/* Physical page holding a lane's logical page (-1 if none; an aborted
 * install keeps its payload, with ownership generation 0). */
int glacier_hip_session_page_of(glacier_hip_session *s, uint32_t lane, uint32_t logical_page,
                                int32_t *physical_out);
int glacier_hip_session_page_generation(glacier_hip_session *s, uint32_t lane,
                                        uint32_t logical_page, uint64_t *ownership_generation_out);
/* Head domain of eligible steps (GreedyOutputMode, generate.zig:415-426):
 * POSTHEAD computes every logit, then applies the mask (domain_posthead);
 * PREHEAD applies it before the head's dot products: a 16-row block with no
 * eligible row for any lane of a fused-head step (up to 2 lanes) streams no
 * weights (domain_prehead). Tokens are identical; in PREHEAD an eligible step
 * cannot return logits (INVALID_ARGUMENT). Wider steps scan full logits. */
#define GLACIER_HIP_HEAD_DOMAIN_POSTHEAD 0
#define GLACIER_HIP_HEAD_DOMAIN_PREHEAD 1
int glacier_hip_session_set_head_domain(glacier_hip_session *s, int mode);
/* Test hook: make the next decode step fail after its kernels ran but before
 * commit (forces the abort path, as a failed sink/ack would). */
int glacier_hip_session_inject_failure(glacier_hip_session *s, int enable);
/* Test hook: with `enable`, every later decode step copies the residual
 * stream after each layer (the output of forwardLayerCached,
 * generate.zig:1511-1967) into a session buffer of num_layers x max_lanes x
 * dim floats (allocated here through the allocation lease, freed when
 * disabled or with the session); traced steps launch their kernels directly
 * instead of replaying a sealed plan. layer_trace copies the last traced
 * step's [num_layers][rows][dim] residuals to the host and its row count to
 * *rows_out (rows in the step's lane order). */
int glacier_hip_session_trace_layers(glacier_hip_session *s, int enable);
int glacier_hip_session_layer_trace(glacier_hip_session *s, float *out_host, uint32_t *rows_out);

/* ---- LaneWeave QoS v1 multi-request scheduler ----------------------------
 * The reference's deterministic interleaved weighted round-robin scheduler
 * (src/core/lane_weave_qos.zig:576-2830) over its own dedicated flat
 * ResourceBank (src/core/resource_bank.zig:867-3200): admission reserves and
 * commits the request's claim before any request state exists and rejects
 * (no_slot / duplicate_tenant / resource_limit / projection_limit /
 * deadline_infeasible) without touching the Bank; one service quantum is one
 * decode token of one lane; every committed decision is an Event-v1 record
 * chained by SHA-256 (eventSha256 :4004-4038, initialRoot :4040-4064) with
 * the reference's field order, domains and little-endian encoding.
 *
 * A decode wave batches the next quanta of distinct lanes:
 * glacier_hip_lane_weave_plan_wave simulates the IWRR selections that the
 * next serve_one calls will make (stopping before a lane would repeat), the
 * caller runs those lanes' tokens in one device step, then commits them with
 * serve_one in the same order; the committed event chain is the one a serial
 * caller would produce. Layouts below are the reference's fields in order;
 * events are values, not live handles. */
typedef struct {
    uint64_t capsule_bytes, kv_bytes, activation_bytes, partial_bytes, logits_bytes;
    uint64_t output_journal_bytes, staging_bytes, device_bytes, io_bytes, queue_slots;
} glacier_hip_claim_t;                 /* resource_bank.zig:61-72 */

typedef struct {
    uint64_t host_bytes, capsule_bytes, kv_bytes, activation_bytes, partial_bytes;
    uint64_t logits_bytes, output_journal_bytes, staging_bytes, device_bytes, io_bytes;
    uint64_t queue_slots;
} glacier_hip_limits_t;                /* resource_bank.zig:101-113 (UINT64_MAX = unlimited) */

typedef struct {
    uint64_t tenant_key, request_key, request_generation, resource_owner_key;
    uint64_t weight;                   /* u16 in the reference: 1..max_weight */
    uint64_t work_quanta;
    uint64_t deadline_tick;            /* absolute logical tick; 0 = none */
    glacier_hip_claim_t claim;
} glacier_hip_request_spec_t;          /* RequestSpec lane_weave_qos.zig:96-106 */

typedef struct {
    uint64_t scheduler_epoch;
    uint64_t slot_index;               /* u32 in the reference */
    uint64_t slot_generation, tenant_key, request_key, request_generation;
} glacier_hip_lane_handle_t;           /* Handle :109-116 */

typedef struct {
    uint64_t bank_epoch;
    uint64_t slot_index;               /* u32 in the reference */
    uint64_t generation, owner_key;
    glacier_hip_claim_t claim;
    uint64_t integrity;
} glacier_hip_bank_receipt_t;          /* Receipt resource_bank.zig:506-513 */

enum glacier_hip_lane_event_kind {
    GLACIER_HIP_EVENT_ADMISSION_ACCEPTED = 0, GLACIER_HIP_EVENT_ADMISSION_REJECTED = 1,
    GLACIER_HIP_EVENT_SERVICE = 2, GLACIER_HIP_EVENT_CANCEL = 3, GLACIER_HIP_EVENT_RETIRE = 4,
    GLACIER_HIP_EVENT_CLOSE = 5,
};
enum glacier_hip_lane_rejection {
    GLACIER_HIP_REJECT_NONE = 0, GLACIER_HIP_REJECT_NO_SLOT = 1,
    GLACIER_HIP_REJECT_DUPLICATE_TENANT = 2, GLACIER_HIP_REJECT_RESOURCE_LIMIT = 3,
    GLACIER_HIP_REJECT_PROJECTION_LIMIT = 4, GLACIER_HIP_REJECT_DEADLINE_INFEASIBLE = 5,
};

typedef struct {
    uint64_t abi_version, scheduler_epoch, event_sequence;
    uint32_t kind, rejection_reason;
    uint8_t previous_sha256[32], event_sha256[32];
    uint8_t state_before_sha256[32], state_after_sha256[32];
    uint64_t logical_tick_before, logical_tick_after;
    uint32_t cursor_before, cursor_after, level_before, level_after;
    glacier_hip_lane_handle_t handle;
    glacier_hip_request_spec_t spec;
    glacier_hip_bank_receipt_t resource_receipt;
    uint8_t resource_receipt_sha256[32];
    uint64_t remaining_before, remaining_after, wait_quanta, maximum_service_gap;
    uint32_t active_before, active_after, finished_before, finished_after;
    glacier_hip_claim_t bank_used_before, bank_used_after;
} glacier_hip_lane_event_t;            /* EventV1 :303-332 */

typedef struct glacier_hip_lane_weave glacier_hip_lane_weave;

/* Scheduler.init over a fresh dedicated Bank of `capacity` slots
 * (:634-735): NULL on an invalid configuration (zero capacity / epoch /
 * weight / budgets, all-zero challenge). */
glacier_hip_lane_weave *glacier_hip_lane_weave_create(
    uint32_t capacity, const glacier_hip_limits_t *bank_limits, uint64_t bank_epoch,
    uint64_t scheduler_epoch, const uint8_t challenge[32], uint32_t max_weight,
    uint64_t max_projection_quanta, uint64_t max_projection_operations);
void glacier_hip_lane_weave_destroy(glacier_hip_lane_weave *lw);
/* admit (:742-900). *admitted = 1 with handle_out set, or 0 (a rejection
 * event, Bank untouched). A malformed spec returns INVALID_ARGUMENT and emits
 * nothing. */
int glacier_hip_lane_weave_admit(glacier_hip_lane_weave *lw, const glacier_hip_request_spec_t *spec,
                                 int *admitted, glacier_hip_lane_handle_t *handle_out,
                                 glacier_hip_lane_event_t *event_out);
/* serveOne (:1196-1270): commit the next IWRR quantum. */
int glacier_hip_lane_weave_serve_one(glacier_hip_lane_weave *lw, glacier_hip_lane_event_t *event_out);
/* The slots the next serve_one calls select, in order, up to max_count and
 * stopping before a slot would repeat; nothing is mutated. */
int glacier_hip_lane_weave_plan_wave(glacier_hip_lane_weave *lw, uint32_t max_count,
                                     uint32_t *slots_out, uint32_t *count_out);
int glacier_hip_lane_weave_retire(glacier_hip_lane_weave *lw, const glacier_hip_lane_handle_t *h,
                                  glacier_hip_lane_event_t *event_out);
int glacier_hip_lane_weave_cancel(glacier_hip_lane_weave *lw, const glacier_hip_lane_handle_t *h,
                                  glacier_hip_lane_event_t *event_out);
int glacier_hip_lane_weave_close(glacier_hip_lane_weave *lw, glacier_hip_lane_event_t *event_out);
/* Handle of a slot (handleFor :2665) and whether it is free / active / finished (0/1/2). */
int glacier_hip_lane_weave_slot(glacier_hip_lane_weave *lw, uint32_t slot,
                                glacier_hip_lane_handle_t *handle_out, uint32_t *state_out,
                                uint64_t *remaining_out);
int glacier_hip_lane_weave_chain_head(glacier_hip_lane_weave *lw, uint8_t out[32]);
int glacier_hip_lane_weave_state_sha256(glacier_hip_lane_weave *lw, uint8_t out[32]);

/* ServicePermitV1 (lane_weave_qos.zig:122-142): the next IWRR selection
 * frozen by prepareService without advancing the tick, cursor, request work,
 * Bank charge or event chain; bound to this scheduler's lifetime (a
 * process-wide coordinator id) and address. permit_sha256 is
 * servicePermitSha256 (:3557-3581). */
typedef struct {
    uint64_t abi_version, scheduler_epoch, coordinator_id, coordinator_address;
    uint64_t permit_generation, event_sequence;
    glacier_hip_lane_handle_t handle;
    uint64_t logical_tick_before;
    uint32_t cursor_before, level_before;  /* level: u16 in the reference */
    uint32_t cursor_after, level_after;
    uint64_t remaining_before, wait_quanta, maximum_service_gap;
    uint8_t state_before_sha256[32], chain_head_before_sha256[32];
    glacier_hip_bank_receipt_t resource_receipt;
    uint8_t resource_receipt_sha256[32], permit_sha256[32];
} glacier_hip_service_permit_v1_t;
/* prepareService (:1127-1192): one permit may be pending; while it is,
 * prepare / serve_one / admit / cancel / retire / close / waves return
 * GLACIER_HIP_SERVICE_IN_FLIGHT and change nothing. commitService
 * (:1272-1286) consumes the pending permit and emits the service event
 * serve_one would have emitted (byte-identical); abortService (:1438-1452)
 * consumes it with no logical change. A permit that is not exactly the
 * pending one (mutated, consumed, foreign, from an earlier scheduler) is
 * GLACIER_HIP_STALE_SERVICE_PERMIT and consumes nothing. */
int glacier_hip_lane_weave_prepare_service(glacier_hip_lane_weave *lw,
                                           glacier_hip_service_permit_v1_t *permit_out);
int glacier_hip_lane_weave_commit_service(glacier_hip_lane_weave *lw,
                                          const glacier_hip_service_permit_v1_t *permit,
                                          glacier_hip_lane_event_t *event_out);
int glacier_hip_lane_weave_abort_service(glacier_hip_lane_weave *lw,
                                         const glacier_hip_service_permit_v1_t *permit);
int glacier_hip_service_permit_sha256(const glacier_hip_service_permit_v1_t *permit, uint8_t out[32]);

/* One LaneWeave decode wave (the multi-request service loop of
 * prepared_text_session.zig:1840-1885 with one token per service quantum):
 * plan the next quanta of distinct lanes (at most max_count), run those
 * lanes' tokens as ONE batched decode step on the device, then commit the
 * quanta with serve_one in plan order. lane_of_slot[slot] names the session
 * lane of each scheduler slot (slot_count entries). tokens_by_lane[lane] holds
 * each lane's last token and receives its next one. eligible_by_lane:
 * optional [session max_lanes][ceil(vocab/64)] masks (eligible argmax,
 * sampling.zig:55-105). slots_out / events_out (optional) receive the
 * committed slots and their Event-v1 records; count_out the number of quanta.
 * The scheduler stays locked from planning to commit, and the plan holds
 * only quanta whose serve_one commits (it stops before a deadline or service
 * gap the next quantum would break). The device step runs privately (KV rows
 * provisional); then each planned quantum publishes inside the reference's
 * service transaction, in plan order: prepareService (its permit must select
 * the planned slot), the lane's KV row, sampler counter and output word
 * published, commitService (the quantum's Event-v1). A failed device step
 * publishes nothing: no KV row, token, sampler counter or scheduler event; a
 * permit that selects another slot aborts it (abortService), publishes
 * nothing more and poisons the scheduler. NO_RUNNABLE when no lane is
 * runnable; SERVICE_IN_FLIGHT while a caller's permit is pending. */
int glacier_hip_session_lane_weave_wave(glacier_hip_session *s, glacier_hip_lane_weave *lw,
                                        const uint32_t *lane_of_slot, uint32_t slot_count,
                                        uint32_t *tokens_by_lane,
                                        const uint64_t *eligible_by_lane, uint32_t max_count,
                                        uint32_t *slots_out, glacier_hip_lane_event_t *events_out,
                                        uint32_t *count_out);

/* ---- staged per-token publication (paged_token_txn.zig:346-600) ----------
 * The reference publishes a decode wave in three phases: the engine stages
 * every lane's token transition as a proposal (KV row / page-map root
 * transition, RNG, sampler counter, output word, token, terminal flag) sealed
 * by proposalSha256; the host's sink reserves it (prepare -> ack); then the
 * engine commits, a step with no failure path, and hands the sink one receipt.
 * step_prepare runs the device step with the KV rows left provisional and
 * returns the proposal; step_commit checks the sink's ack and publishes;
 * step_abort (a rejected or abandoned proposal) publishes nothing: the rows
 * are aborted (their generations stay consumed) and the RNG, sampler counter
 * and outputs are unchanged. Records keep the reference's fields in order
 * (u8/bool fields widened to u32); proposalSha256 hashes them with the
 * reference's widths. A wave holds 1..GLACIER_HIP_PUBLICATION_WIDTH lanes
 * (the reference's fixed B4 width). The Bank receipt, fence permit and
 * sequence are the host's (its ResourceBank), passed in the binding. */
#define GLACIER_HIP_PUBLICATION_WIDTH 4

typedef struct {
    uint64_t abi_version;            /* 0x4750545200000001 */
    uint64_t kv_row_txn_abi, page_map_root_abi, page_ref_abi;
    uint64_t cache_instance, row_txn_generation;
    uint64_t root_before_generation, root_after_generation;
    uint64_t root_before_len, root_after_len, root_before_pages, root_after_pages;
    uint8_t root_before_ownership_sha256[32], root_after_ownership_sha256[32];
    uint64_t logical_page, page_ownership_generation;
    uint32_t installs_new_page, reserved;
    uint8_t initial_logical_kv_sha256[32];  /* first wave only */
    uint8_t row_payload_sha256[32];         /* logicalRowTxnSha256 of the staged row */
    uint8_t state_chain_before[32], state_chain_after[32];
} glacier_hip_root_transition_v1_t;     /* RootTransitionV1 (paged_token_txn.zig:61-89) */

typedef struct {
    uint32_t lane_index, has_kv_transition;
    uint64_t step_index, prompt_len, kv_before, kv_after, kv_capacity_bytes;
    glacier_hip_root_transition_v1_t kv_transition;
    uint64_t output_before, output_after;
    uint64_t rng_before[4], rng_after[4];
    uint64_t sampling_calls_before, sampling_calls_after;
    uint32_t token_id, terminal;
} glacier_hip_lane_proposal_v1_t;       /* LaneProposalV1 (:91-108) */

typedef struct {
    uint64_t abi_version;            /* 0x4750545800000001 */
    uint64_t resource_bank_abi, resource_publication_fence_abi, paged_kv_abi;
    uint64_t page_map_root_abi, page_ref_abi, page_transition_abi, kv_row_txn_abi;
    uint64_t execution_abi, request_epoch, transaction_sequence, resource_permit_generation;
    uint32_t live_mask, live_lane_count;
    uint64_t kv_capacity_bytes;
    glacier_hip_bank_receipt_t receipt;
    glacier_hip_lane_proposal_v1_t lanes[GLACIER_HIP_PUBLICATION_WIDTH];
} glacier_hip_token_proposal_v1_t;      /* ProposalV1 (:110-131) */

/* A LaneWeave wave published through a sink: one stage per planned quantum,
 * in plan order (the scheduler slot, the session lane, and the lane's token
 * transition as a LaneProposalV1: the staged KV row's page-map root
 * transition and row payload digest, output, RNG and sampler counters
 * before / after, token; the state-chain fields are the lane's when it
 * publishes staged waves, else zero). */
typedef struct {
    uint32_t slot, lane;
    glacier_hip_lane_proposal_v1_t stage;
} glacier_hip_wave_stage_v1_t;
/* The sink acknowledges (0) or rejects (nonzero) the whole wave before any
 * quantum publishes (the prepare -> ack of paged_token_txn.zig:503-515,
 * taken once per wave). */
typedef int (*glacier_hip_wave_sink_fn)(void *ctx, const glacier_hip_wave_stage_v1_t *stages,
                                        uint32_t count);
/* glacier_hip_session_lane_weave_wave with the wave's stages put to `sink`
 * after the private device step and before the first service permit: a
 * rejection aborts every staged row and returns GLACIER_HIP_SINK_REJECTED;
 * no lane publishes, the scheduler's state and event chain do not move and
 * the same quanta are planned again by the next wave. */
int glacier_hip_session_lane_weave_wave_staged(
    glacier_hip_session *s, glacier_hip_lane_weave *lw, const uint32_t *lane_of_slot,
    uint32_t slot_count, uint32_t *tokens_by_lane, const uint64_t *eligible_by_lane,
    uint32_t max_count, glacier_hip_wave_sink_fn sink, void *sink_ctx, uint32_t *slots_out,
    glacier_hip_lane_event_t *events_out, uint32_t *count_out);

typedef struct {
    uint64_t abi_version;            /* 0x4750544100000001 */
    uint8_t proposal_sha256[32];
    uint64_t sink_epoch;             /* nonzero */
    uint64_t reservation_id;         /* nonzero */
} glacier_hip_prepare_ack_v1_t;         /* PrepareAckV1 (:133-138) */

typedef struct {
    uint64_t abi_version;            /* 0x4750544300000001 */
    uint8_t proposal_sha256[32];
    glacier_hip_prepare_ack_v1_t prepare_ack;
    uint8_t commit_sha256[32];       /* commitSha256 (:1132-1148) */
} glacier_hip_commit_receipt_v1_t;      /* CommitReceiptV1 (:140-146); its proposal is prepare's */

/* The host publication session's side of a wave (Session.init / Batch.begin,
 * :262-471): its execution ABI, request epoch, sequence, the fence permit's
 * generation, the cohort's KV capacity and its Bank receipt, and for each
 * wave lane (in the order of the step's lanes) its publication slot and
 * whether this token ends its request. */
typedef struct {
    uint64_t execution_abi, request_epoch, transaction_sequence, resource_permit_generation;
    uint64_t kv_capacity_bytes;
    glacier_hip_bank_receipt_t receipt;
    uint32_t lane_index[GLACIER_HIP_PUBLICATION_WIDTH];
    uint32_t terminal[GLACIER_HIP_PUBLICATION_WIDTH];
} glacier_hip_publication_binding_t;

/* Prefill for staged publication: the prompt rows commit as in
 * glacier_hip_session_prefill, the first greedy token is computed and held
 * back for the first wave (published by step_prepare/step_commit). */
int glacier_hip_session_prefill_staged(glacier_hip_session *s, uint32_t lane,
                                       const uint32_t *tokens, uint32_t n,
                                       uint32_t *first_token, float *logits_host);
/* Stage one wave of `count` lanes (1..4). Either every lane holds a staged
 * first token (the first wave: no KV row, an initial transition over the
 * lane's logical KV digest; tokens[] unused) or every lane has published it
 * (a decode wave: lanes[i] consumes tokens[i], its row stays provisional).
 * next_tokens receives the proposed tokens; nothing is published. Until
 * commit or abort every other step on the session is TRANSACTION_ACTIVE. */
int glacier_hip_session_step_prepare(glacier_hip_session *s, const uint32_t *lanes,
                                     const uint32_t *tokens, uint32_t count,
                                     const uint64_t *eligible_words_host,
                                     const glacier_hip_publication_binding_t *binding,
                                     glacier_hip_token_proposal_v1_t *proposal_out,
                                     uint8_t proposal_sha256_out[32], uint32_t *next_tokens,
                                     float *logits_host);
/* Publish the prepared wave after the sink's ack (abi, nonzero epoch and
 * reservation, the proposal's digest). An invalid ack aborts the wave and
 * returns INVALID_TRANSACTION. */
int glacier_hip_session_step_commit(glacier_hip_session *s, const glacier_hip_prepare_ack_v1_t *ack,
                                    glacier_hip_commit_receipt_v1_t *receipt_out);
int glacier_hip_session_step_abort(glacier_hip_session *s);
/* proposalSha256 / commitSha256 of a record (pure host functions). */
int glacier_hip_token_proposal_sha256(const glacier_hip_token_proposal_v1_t *proposal,
                                      uint8_t out[32]);
int glacier_hip_token_commit_sha256(const uint8_t proposal_sha256[32],
                                    const glacier_hip_prepare_ack_v1_t *ack, uint8_t out[32]);
/* tokenSequenceSha256 (generate.zig:3193-3203): the output digest a lane's
 * state reports, for a host that verifies a receipt's token journal. */
int glacier_hip_token_sequence_sha256(const uint32_t *tokens, uint64_t count, uint8_t out[32]);

/* ---- paged-KV checkpoint page images ------------------------------------
 * src/continuation_paged_kv_restore.zig (PageImageV1, :18-360) and
 * PagedKVCache.restoreCheckpointV1 (paged_kv_cache.zig:570-762). A page
 * image is one committed page of a lane in the portable layout: a 208-byte
 * header (magic "GCKVPG01", ABI 0x4743_4b50_0000_0001, length, flags, the
 * source PageMapRootV1, num_layers, kv dim, max_seq, the page's PageRefV1,
 * committed rows, element count, challenge), the committed rows as
 * little-endian f32 in (layer, K/V, row, dim) order, and SHA-256 of
 * "glacier-continuation-paged-kv-page-image-v1\0" ++ everything before it.
 * The device pages are read back (fp16 pages widen to f32 exactly) or
 * written (restore) by these entry points; the host keeps the bytes. */
enum glacier_hip_page_image_error {
    GLACIER_HIP_PAGE_IMAGE_OK = 0,
    GLACIER_HIP_PAGE_IMAGE_INVALID_LENGTH = 1,
    GLACIER_HIP_PAGE_IMAGE_INVALID_MAGIC = 2,
    GLACIER_HIP_PAGE_IMAGE_INVALID_ABI = 3,
    GLACIER_HIP_PAGE_IMAGE_INVALID_FLAGS = 4,
    GLACIER_HIP_PAGE_IMAGE_INVALID_PAGE_IMAGE = 5,
    GLACIER_HIP_PAGE_IMAGE_CAPACITY_EXCEEDED = 6,
    GLACIER_HIP_PAGE_IMAGE_UNSAFE_DESTINATION = 7,
    GLACIER_HIP_PAGE_IMAGE_FOREIGN_CHECKPOINT = 8,
    GLACIER_HIP_PAGE_IMAGE_INVALID_CHECKPOINT = 9,
    GLACIER_HIP_PAGE_IMAGE_INVALID_RESTORE_PLAN = 10,
    GLACIER_HIP_PAGE_IMAGE_ARITHMETIC_OVERFLOW = 11,
};

typedef struct {
    uint32_t error;                  /* glacier_hip_page_image_error of a failed call */
    uint32_t reserved;
    glacier_hip_page_map_root_t source_root;
    uint64_t num_layers, dim, max_seq;
    glacier_hip_page_ref_t source_ref;
    uint64_t committed_rows, payload_element_count;
    uint64_t payload_offset;         /* byte offset of the canonical f32 rows (208) */
    uint8_t challenge_sha256[32];
    uint8_t image_sha256[32];
} glacier_hip_page_image_v1_t;

typedef struct {
    uint64_t abi_version;            /* 0x4750435200000001 (checkpoint_restore_abi) */
    glacier_hip_page_map_root_t source_root;
    glacier_hip_page_map_root_t target_root;
    uint64_t restored_pages;
    uint64_t restored_payload_bytes; /* f32 page payloads, as the reference counts them */
    uint32_t error;                  /* glacier_hip_page_image_error of a failed restore */
    uint32_t reserved;
} glacier_hip_checkpoint_restore_v1_t;

/* encodedPageImageBytesV1 (:68-97); 0 for an invalid geometry. */
uint64_t glacier_hip_page_image_bytes(uint64_t num_layers, uint64_t dim, uint64_t committed_rows);
/* encodeCanonicalPageImageV1 (:101-170) from caller-owned canonical bytes.
 * info (may be NULL) receives the failure reason. Host only. */
int glacier_hip_page_image_encode_canonical(const glacier_hip_page_map_root_t *source_root,
                                            uint64_t num_layers, uint64_t dim, uint64_t max_seq,
                                            const glacier_hip_page_ref_t *source_ref,
                                            uint64_t committed_rows,
                                            const uint8_t *canonical_f32_le, uint64_t canonical_len,
                                            const uint8_t challenge_sha256[32], uint8_t *out,
                                            uint64_t out_capacity, uint64_t *out_len,
                                            glacier_hip_page_image_v1_t *info);
/* decodePageImageV1 (:263-360). Host only. */
int glacier_hip_page_image_decode(const uint8_t *image, uint64_t len,
                                  const uint8_t expected_challenge_sha256[32],
                                  glacier_hip_page_image_v1_t *out);
/* encodePageImageV1 (:174-261) for one committed page of a session lane:
 * the page is read back from HBM. info (may be NULL) receives the header. */
int glacier_hip_session_encode_page_image(glacier_hip_session *session, uint32_t lane,
                                          uint32_t logical_page,
                                          const uint8_t challenge_sha256[32], uint8_t *out,
                                          uint64_t out_capacity, uint64_t *out_len,
                                          glacier_hip_page_image_v1_t *info);
/* Restore a checkpoint into `lane`, which is begun afresh (lane_begin with
 * `seed`; a cache instance different from the source's): every image is
 * decoded against the challenge, must carry logical page = its index, the
 * same source root and geometry (ForeignCheckpoint otherwise), the session's
 * layer count, kv dim and max_positions (InvalidCheckpoint otherwise); the
 * source ownership chain is verified; only then are pool pages taken and the
 * rows written to HBM (zeros past the committed rows; an fp16 pool accepts
 * only values fp16 holds exactly). The lane's page map then has target refs
 * (this instance, page i, generation i + 1), root generation 2 and the next
 * root generation 3 (restoreCheckpointV1). target_refs may be NULL. On
 * failure the lane is left begun and empty. */
int glacier_hip_session_restore_checkpoint(glacier_hip_session *session, uint32_t lane,
                                           const uint8_t *const *images,
                                           const uint64_t *image_lens, uint32_t count,
                                           const uint8_t challenge_sha256[32], uint64_t seed,
                                           glacier_hip_checkpoint_restore_v1_t *out,
                                           glacier_hip_page_ref_t *target_refs);

/* ---- prepared runtime images (.glrt) -------------------------------------
 * src/model/runtime_image.zig (MappedImage, :770-1049) and the prepared-model
 * loader src/loader.zig:193-390 (loadPreparedWithOptions). An image is read
 * through a read-only file mapping and validated fail-closed before anything
 * is uploaded: header (magic, version, sizes, reserved bytes, CRC32), ABI
 * fingerprint (this backend runs the portable row-major INT4 + f32-scale
 * execution layout: GLRT v2 "row-major-f32-v2", v1 "row-major-f32-v1"),
 * index CRC32, every record descriptor (encoding / layout / shape / stream
 * bounds, 64-byte alignment, no overlap, no duplicates) and, by default,
 * each record's payload CRC32 and (v2) descriptor+payload SHA-256. */
typedef struct glacier_hip_glrt_image glacier_hip_glrt_image;

/* Failure reasons, named after the reference's errors. */
enum glacier_hip_glrt_error {
    GLACIER_HIP_GLRT_OK = 0,
    GLACIER_HIP_GLRT_TRUNCATED_HEADER = 1,
    GLACIER_HIP_GLRT_BAD_MAGIC = 2,
    GLACIER_HIP_GLRT_BAD_VERSION = 3,
    GLACIER_HIP_GLRT_BAD_HEADER_SIZE = 4,
    GLACIER_HIP_GLRT_BAD_RECORD_SIZE = 5,
    GLACIER_HIP_GLRT_BAD_ALIGNMENT = 6,
    GLACIER_HIP_GLRT_BAD_CONFIG = 7,
    GLACIER_HIP_GLRT_BAD_RESERVED_FIELD = 8,
    GLACIER_HIP_GLRT_HEADER_CRC_MISMATCH = 9,
    GLACIER_HIP_GLRT_LEGACY_VERSION_DISABLED = 10,
    GLACIER_HIP_GLRT_BAD_HEADER = 11,
    GLACIER_HIP_GLRT_BAD_BOUNDS = 12,
    GLACIER_HIP_GLRT_SOURCE_FINGERPRINT_MISMATCH = 13,
    GLACIER_HIP_GLRT_ABI_FINGERPRINT_MISMATCH = 14,
    GLACIER_HIP_GLRT_INDEX_CRC_MISMATCH = 15,
    GLACIER_HIP_GLRT_TRUNCATED_INDEX = 16,
    GLACIER_HIP_GLRT_BAD_TENSOR_KIND = 17,
    GLACIER_HIP_GLRT_BAD_ENCODING = 18,
    GLACIER_HIP_GLRT_BAD_PACKED_LAYOUT = 19,
    GLACIER_HIP_GLRT_BAD_ROLE = 20,
    GLACIER_HIP_GLRT_BAD_PAIR_NIBBLE_LAYOUT = 21,
    GLACIER_HIP_GLRT_BAD_FLAGS = 22,
    GLACIER_HIP_GLRT_BAD_VERSIONED_RECORD = 23,
    GLACIER_HIP_GLRT_MISSING_DIGEST = 24,
    GLACIER_HIP_GLRT_BAD_TENSOR_SHAPE = 25,
    GLACIER_HIP_GLRT_MISSING_SCALES = 26,
    GLACIER_HIP_GLRT_OVERLAPPING_PAYLOAD = 27,
    GLACIER_HIP_GLRT_DUPLICATE_RECORD = 28,
    GLACIER_HIP_GLRT_CRC_MISMATCH = 29,
    GLACIER_HIP_GLRT_DIGEST_MISMATCH = 30,
    GLACIER_HIP_GLRT_FILE_ERROR = 31,        /* open / stat / mmap failed */
    /* loader (loader.zig LoaderError) */
    GLACIER_HIP_GLRT_MISSING_TENSOR = 32,
    GLACIER_HIP_GLRT_BAD_PAYLOAD = 33,
    GLACIER_HIP_GLRT_NO_LAYERS = 34,
    GLACIER_HIP_GLRT_UNSUPPORTED = 35,       /* valid, but not a shape this device runs */
};

typedef struct {
    int32_t verify_payload_crc;      /* OpenOptions defaults: 1 */
    int32_t verify_payload_digest;   /* 1 */
    int32_t allow_v1;                /* 1 */
    int32_t check_source_fingerprint;/* 0: any source */
    uint8_t expected_source_fingerprint[32];
} glacier_hip_glrt_open_options_t;

typedef struct {
    uint32_t error;                  /* glacier_hip_glrt_error of a failed open/load */
    uint32_t version;                /* 1 or 2 */
    uint64_t record_count, data_offset, file_size;
    uint8_t source_fingerprint[32], abi_fingerprint[32];
    uint32_t dim, hidden_dim, layers, vocab, heads, head_dim, kv_heads;
    uint32_t tie_embeddings;
    float rms_eps, rope_theta;
} glacier_hip_glrt_info_t;

/* One decoded record (Record, runtime_image.zig:300-323). Streams: 0 packed
 * weights, 1 f32 scales, 2 f16 scales, 3 f16 rows4 scales, 4 raw f32. */
typedef struct {
    uint32_t layer_idx, kind;        /* kind: format.zig TensorKind */
    uint16_t role, encoding, packed_layout, pair_nibble_layout;
    uint32_t group_size, out_f, in_f, flags, payload_crc32, reserved;
    uint64_t num_elements;
    uint64_t offset[5], length[5];
    uint8_t payload_digest[32];
} glacier_hip_glrt_record_t;

/* Opens and validates `path` (opts NULL = the defaults). On failure returns
 * GLACIER_HIP_BAD_IMAGE with info->error set and *out NULL. Host only. */
int glacier_hip_glrt_open(const char *path, const glacier_hip_glrt_open_options_t *opts,
                          glacier_hip_glrt_image **out, glacier_hip_glrt_info_t *info);
void glacier_hip_glrt_close(glacier_hip_glrt_image *image);
int glacier_hip_glrt_record_at(const glacier_hip_glrt_image *image, uint64_t index,
                               glacier_hip_glrt_record_t *out);
/* findWithRole (:898-911): GLACIER_HIP_NOT_FOUND when absent. */
int glacier_hip_glrt_find(const glacier_hip_glrt_image *image, uint32_t layer_idx, uint32_t kind,
                          uint32_t role, glacier_hip_glrt_record_t *out);
/* A view into the mapping (valid until close); empty streams give len 0. */
int glacier_hip_glrt_stream(const glacier_hip_glrt_image *image,
                            const glacier_hip_glrt_record_t *record, uint32_t stream,
                            const void **data, uint64_t *len);
/* identityV1 (:860-870): SHA-256 over every byte of the container. */
int glacier_hip_glrt_identity(const glacier_hip_glrt_image *image, uint8_t container_sha256[32],
                              uint64_t *container_bytes);

/* Loader report: the loader-level failure reason (info.error codes), and
 * how many INT4 scales were taken from f32 values that fp16 does not hold
 * exactly (the device stores fp16 scales; an image with an f16 scale
 * mirror is uploaded from the mirror). */
typedef struct {
    uint32_t error;
    uint32_t separate_mlp;           /* 1: separate gate/up records (the only layout loaded) */
    uint64_t int4_records, raw_records;
    uint64_t inexact_scales;
    uint64_t uploaded_bytes;         /* device bytes of the model */
} glacier_hip_glrt_load_report_t;

/* loadPreparedWithOptions (loader.zig:202-306) onto the device: validates
 * the prepared record set (config, expected records only, required norms,
 * separate gate/up per layer, optional q/k/v biases), dequantizes the INT4
 * token embedding to f32 rows (dequantizeRow, int4_matmul.zig:3164-3194),
 * uploads every projection into the device tile layout and the LM head (or
 * the tied embedding matrix). Returns NULL on failure with report->error
 * set (and the context's last_error). */
glacier_hip_model *glacier_hip_model_load_glrt(glacier_hip_context *ctx,
                                               const glacier_hip_glrt_image *image,
                                               glacier_hip_glrt_load_report_t *report);

/* ---- portable .glacier source containers (src/model/format.zig) ----------
 * Header (256 bytes) | JSON metadata | page index (64-byte PageEntry each) |
 * page payloads; a quantized page's payload is the qio sub-header "QOIT"
 * (u32 magic, u32 num_elements, u32 group_size, u8 precision 0 int8 /
 * 1 int4, 3 zero bytes), f32 scales, then the packed codes (qio.zig:1-21).
 * Admission, CRCs and identities follow FileReader (format.zig:379-662) and
 * report the reference's error names (glacier_hip_glacier_error_name). */
typedef struct glacier_hip_glacier glacier_hip_glacier;

typedef struct {
    uint32_t version, header_size;
    uint64_t meta_offset, meta_len, num_pages, page_index_offset, page_data_offset;
    uint32_t page_size_log2, reserved;
    uint64_t container_bytes;
} glacier_hip_glacier_header_t;    /* Header (format.zig:67-137) + the file size */

typedef struct {
    uint64_t page_id;
    uint32_t layer_idx, tensor_kind;     /* TensorKind (format.zig:46-64) */
    uint64_t row_start, row_end;         /* element range of the page's tensor */
    uint32_t precision, quant_group;     /* core.Precision: fp16 0, bf16 1, int8 2, int4 3, int2 4, tri1p58 5, fp32 6 */
    uint64_t data_offset, data_len;
    uint32_t crc32, reserved;
} glacier_hip_glacier_page_t;      /* PageEntry (format.zig:141-199) */

enum {
    GLACIER_HIP_GLAC_OK = 0,
    GLACIER_HIP_GLAC_TRUNCATED_HEADER = 1, GLACIER_HIP_GLAC_BAD_MAGIC = 2,
    GLACIER_HIP_GLAC_BAD_VERSION = 3, GLACIER_HIP_GLAC_BAD_HEADER_SIZE = 4,
    GLACIER_HIP_GLAC_BAD_PAGE_SIZE = 5, GLACIER_HIP_GLAC_BAD_RESERVED_FIELD = 6,
    GLACIER_HIP_GLAC_BAD_LAYOUT = 7, GLACIER_HIP_GLAC_METADATA_TOO_LARGE = 8,
    GLACIER_HIP_GLAC_INDEX_TOO_LARGE = 9, GLACIER_HIP_GLAC_LAYOUT_OVERFLOW = 10,
    GLACIER_HIP_GLAC_TRUNCATED_META = 11, GLACIER_HIP_GLAC_TRUNCATED_INDEX = 12,
    GLACIER_HIP_GLAC_BAD_METADATA = 13, GLACIER_HIP_GLAC_BAD_TENSOR_KIND = 14,
    GLACIER_HIP_GLAC_BAD_PRECISION = 15, GLACIER_HIP_GLAC_BAD_PAGE_ID = 16,
    GLACIER_HIP_GLAC_BAD_ROW_RANGE = 17, GLACIER_HIP_GLAC_EMPTY_PAGE = 18,
    GLACIER_HIP_GLAC_BAD_QUANT_GROUP = 19, GLACIER_HIP_GLAC_PAGE_GEOMETRY_TOO_LARGE = 20,
    GLACIER_HIP_GLAC_BAD_PAGE_GEOMETRY = 21, GLACIER_HIP_GLAC_UNSUPPORTED_PRECISION = 22,
    GLACIER_HIP_GLAC_NON_CONTIGUOUS_PAYLOAD = 23, GLACIER_HIP_GLAC_TRUNCATED_PAGE = 24,
    GLACIER_HIP_GLAC_TRAILING_BYTES = 25, GLACIER_HIP_GLAC_CRC_MISMATCH = 26,
    GLACIER_HIP_GLAC_BAD_QUANT_PAYLOAD = 27, GLACIER_HIP_GLAC_BUFFER_TOO_SMALL = 28,
    GLACIER_HIP_GLAC_EMPTY_STREAM_BUFFER = 29, GLACIER_HIP_GLAC_FILE_ERROR = 30,
    GLACIER_HIP_GLAC_SIZE_MISMATCH = 31,
    /* qio / quant */
    GLACIER_HIP_GLAC_BAD_GROUP_SIZE = 32, GLACIER_HIP_GLAC_TRUNCATED_SCALES = 33,
    GLACIER_HIP_GLAC_TRUNCATED_PACKED = 34, GLACIER_HIP_GLAC_INVALID_PAYLOAD_SIZE = 35,
    GLACIER_HIP_GLAC_INVALID_VALUE = 36,       /* encode: a non-finite source value */
    /* loader (loader.zig:20-28) and this device's limits */
    GLACIER_HIP_GLAC_NO_LAYERS = 37, GLACIER_HIP_GLAC_MISSING_TENSOR = 38,
    GLACIER_HIP_GLAC_BAD_PAYLOAD = 39, GLACIER_HIP_GLAC_UNSUPPORTED = 40,
    GLACIER_HIP_GLAC_INVALID_ARGUMENT = 41,
};
const char *glacier_hip_glacier_error_name(uint32_t code);

/* FileReader.open (:383-478): strict admission of `path`; returns a
 * GLACIER_HIP_GLAC_* code, *out set only on success. */
int glacier_hip_glacier_open(const char *path, glacier_hip_glacier **out);
void glacier_hip_glacier_close(glacier_hip_glacier *c);
int glacier_hip_glacier_header(const glacier_hip_glacier *c, glacier_hip_glacier_header_t *out);
int glacier_hip_glacier_page(const glacier_hip_glacier *c, uint64_t index,
                             glacier_hip_glacier_page_t *out);
/* The metadata blob (a view into the mapping, valid until close). */
int glacier_hip_glacier_metadata(const glacier_hip_glacier *c, const void **data, uint64_t *len);
/* readPage (:488-494): copies the page's payload after its CRC check. */
int glacier_hip_glacier_read_page(const glacier_hip_glacier *c, uint64_t index, void *dst,
                                  uint64_t dst_len);
/* readPageDequant (:638-662) to f32: raw pages decoded, quantized pages
 * schema-checked and dequantized; *count = the page's element count. */
int glacier_hip_glacier_read_page_f32(const glacier_hip_glacier *c, uint64_t index, float *dst,
                                      uint64_t capacity, uint64_t *count);
/* validateAllPageCrcsWithBufferV1 (:503-531): every page's payload schema
 * and CRC, read in chunks of buffer_bytes (0: EmptyStreamBuffer). */
int glacier_hip_glacier_validate_crcs(const glacier_hip_glacier *c, uint64_t buffer_bytes);
/* containerIdentityV1 (:536-575): SHA-256 of every byte of the file. */
int glacier_hip_glacier_identity(const glacier_hip_glacier *c, uint8_t container_sha256[32],
                                 uint64_t *container_bytes);
/* sourceFingerprint (loader.zig:167-189): metadata and typed page entries,
 * physical offsets omitted. */
int glacier_hip_glacier_source_fingerprint(const glacier_hip_glacier *c, uint8_t out[32]);
/* qio.encodePage over f32 source (qio.zig:72-112, quant.quantize
 * quant.zig:36-112): precision 0 int8 / 1 int4; *len = payload bytes (with
 * capacity too small nothing is written and BUFFER_TOO_SMALL returned). */
int glacier_hip_qio_encode_f32(const float *src, uint64_t count, uint32_t precision,
                               uint32_t group_size, uint8_t *out, uint64_t capacity,
                               uint64_t *len);
/* qio.decodePage to f32 (qio.zig:115-162, quant.dequantize :114-163). */
int glacier_hip_qio_decode_f32(const uint8_t *payload, uint64_t len, float *out,
                               uint64_t capacity, uint64_t *count);

/* The loader's host-side assembly alone (no device): the geometry pass
 * (loader.zig:1226-1268) and every (layer, kind) group materialised as the
 * device loader takes them, summarised by a digest over the groups in
 * (layer, kind) order: SHA-256 of "glacier-hip-assembly-v1\0", u64 group
 * count, then per group u32 layer, u32 kind, u32 int4, u32 group size,
 * u64 elements, then the packed nibbles and f32 scales (INT4 groups) or the
 * f32 values (all LE). A test-facing summary of this library. */
typedef struct {
    uint32_t error;                  /* GLACIER_HIP_GLAC_* */
    uint32_t num_layers;
    uint64_t dim, hidden_dim, vocab_size;
    uint64_t groups, int4_groups;
    uint8_t sha256[32];
} glacier_hip_glacier_assembly_t;
int glacier_hip_glacier_assemble(const glacier_hip_glacier *c, glacier_hip_glacier_assembly_t *out);

typedef struct {
    uint32_t error;                  /* GLACIER_HIP_GLAC_* */
    uint32_t int4_tensors, raw_tensors, reserved;
    uint64_t inexact_scales;         /* f32 scales fp16 does not hold exactly */
    uint64_t uploaded_bytes;
    glacier_hip_model_config_t config;  /* the configuration loaded */
} glacier_hip_glacier_load_report_t;

/* loadWithOptions (loader.zig:1214-1592) with compact INT4 onto the device:
 * model geometry from the page metadata (norm lengths, element counts),
 * `override` fields that are non-zero replacing it as the reference's JSON
 * sidecar does (heads default dim / 64 with head_dim 64, kv heads = heads,
 * rms_eps 1e-6, rope_theta 10000), groups materialised in (layer, kind)
 * order (INT4 pages of the projections, embedding and head merged by
 * concatInt4Pages :1636-1720, the rest decoded to f32), then every layer
 * uploaded into the device tile layout (f32 scales rounded to fp16) and the
 * INT4 embedding dequantized for the gather. The device runs INT4 group-32
 * projections and LM head: other encodings load as UNSUPPORTED. NULL on
 * failure with report->error set. */
glacier_hip_model *glacier_hip_model_load_glacier(glacier_hip_context *ctx,
                                                  const glacier_hip_glacier *c,
                                                  const glacier_hip_model_config_t *override,
                                                  int tie_word_embeddings,
                                                  glacier_hip_glacier_load_report_t *report);

/* ---- synthetic random-init generator (host, deterministic) ---------------
 * Counter-based SplitMix64 streams keyed by (seed, tensor id):
 *  - INT4 codes: uniform nibbles u in 0..15 (decode u - 7 in [-7, 8]);
 *  - scales: fp16(|N(0, sigma)|) via Box-Muller in double;
 *  - f32 tensors: N(0, sigma);
 *  - token ids: uniform in [0, vocab). */
void glacier_hip_synth_int4(uint64_t seed, uint64_t tensor_id, uint8_t *packed, uint64_t bytes);
void glacier_hip_synth_scales_f16(uint64_t seed, uint64_t tensor_id, float sigma,
                                  uint16_t *out, uint64_t count);
void glacier_hip_synth_normal_f32(uint64_t seed, uint64_t tensor_id, float sigma,
                                  float *out, uint64_t count);
void glacier_hip_synth_tokens(uint64_t seed, uint64_t tensor_id, uint32_t vocab,
                              uint32_t *out, uint64_t count);
/* Tensor ids used by glacier_hip_model_init_random. */
uint64_t glacier_hip_synth_tensor_id(uint32_t layer, uint32_t which);
float glacier_hip_f16_to_f32(uint16_t h);

/* ---- leased paged KV: page payloads charged through a LeaseTree ----------
 * The reference's LeaseTree-backed page ownership (leased_paged_kv_cache.zig)
 * over its ResourceBank (core/resource_bank.zig). A lease bank holds
 * receipt slots (reserve :976-1044, commit :1046-1076, release :3166-3184)
 * and a LeaseTree per committed receipt: a tree (openLeaseTree :1368-1446)
 * carries zero-charge scopes, one per lane (openLeaseScope :1448-1514), and
 * one allocation leaf per live page payload. A leaf is reserved and charged
 * before the page map takes the payload (reserveAllocationsForSession
 * :1534-1783), settled once it has (commitAllocationsAfterAllocate
 * :1785-1823) or uncharged if it could not (abortAllocationsAfterFree
 * :1909-1956). Terminal reclaim retires a whole scope (beginRetireSubtree
 * :2227-2343, authorizeFree :2383-2452), frees the payloads, then uncharges
 * (commitFreeAfterAllocatorFree :2454-2502). Publication sessions bind a
 * request epoch and session id to a receipt and hand out one permit per
 * sequence number (bindPublicationSessionWithLeaseTree :2731-2750,
 * beginPublicationWithLeaseTree :2938-2960, commitPublicationAssumeValid
 * :3076-3089, closePublicationSession :3104-3124).
 *
 * Tokens (tree, node, receipt) are values the caller passes back; every
 * field must equal the bank's current state (a stale copy is rejected with
 * GLACIER_HIP_LEASE_STALE_RESERVATION). Integrity words are this library's
 * own keyed mixes of the token fields; they are not part of the reference's
 * published formats. Every lease verb returns a glacier_hip_lease_status. */
enum glacier_hip_lease_status {
    GLACIER_HIP_LEASE_OK = 0,
    GLACIER_HIP_LEASE_INVALID_ARGUMENT = 1,       /* NULL pointer / zero count */
    /* resource_bank.zig:43-53 */
    GLACIER_HIP_LEASE_INVALID_CONFIGURATION = 2,
    GLACIER_HIP_LEASE_INVALID_CLAIM = 3,
    GLACIER_HIP_LEASE_CLAIM_OVERFLOW = 4,
    GLACIER_HIP_LEASE_CAPACITY_EXCEEDED = 5,
    GLACIER_HIP_LEASE_SLOTS_EXHAUSTED = 6,        /* ReservationSlotsExhausted */
    GLACIER_HIP_LEASE_NODES_EXHAUSTED = 7,        /* LeaseNodesExhausted */
    GLACIER_HIP_LEASE_STALE_RESERVATION = 8,
    GLACIER_HIP_LEASE_INVALID_TRANSITION = 9,
    /* leased_paged_kv_cache.zig:37-51 */
    GLACIER_HIP_LEASE_INVALID_COORDINATOR = 10,
    GLACIER_HIP_LEASE_INVALID_BINDING_STORAGE = 11,
    GLACIER_HIP_LEASE_INVALID_BINDING = 12,
    GLACIER_HIP_LEASE_INVALID_LEASED_PLAN = 13,
    GLACIER_HIP_LEASE_INVALID_LEASED_TRANSACTION = 14,
    GLACIER_HIP_LEASE_ALREADY_TERMINAL = 15,
    GLACIER_HIP_LEASE_TERMINAL_REQUIRED = 16,
    GLACIER_HIP_LEASE_INVALID_TERMINAL_SEAL = 17,
    GLACIER_HIP_LEASE_RECLAIM_PENDING = 18,
    GLACIER_HIP_LEASE_RECLAIM_COMPLETE = 19,
    GLACIER_HIP_LEASE_INVALID_FREED_PAYLOAD = 20,
    /* the page map's errors (paged_kv_cache.zig) */
    GLACIER_HIP_LEASE_INVALID_ROOT = 21,
    GLACIER_HIP_LEASE_CACHE_RETIRED = 22,
    GLACIER_HIP_LEASE_OUT_OF_MEMORY = 23,         /* no free payload in the pool */
    GLACIER_HIP_LEASE_CACHE_FULL = 24,
    GLACIER_HIP_LEASE_TRANSACTION_ACTIVE = 25,
    GLACIER_HIP_LEASE_INVALID_TRANSACTION = 26,
    GLACIER_HIP_LEASE_DEVICE_ERROR = 27,          /* a session lane's KV read failed */
};

typedef struct {
    uint64_t abi_version;        /* 0x474c545200000001 */
    glacier_hip_bank_receipt_t parent;
    uint64_t tree_key, authority_key, identity_generation, generation, structural_revision;
    glacier_hip_claim_t ceiling, current;
    uint32_t active_nodes, reserved0;
    uint64_t state_digest, integrity;
} glacier_hip_lease_tree_t;        /* LeaseTreeV1 (resource_bank.zig:296-312) */

enum { GLACIER_HIP_LEASE_NODE_SCOPE = 0, GLACIER_HIP_LEASE_NODE_ALLOCATION = 1 };
typedef struct {
    uint64_t abi_version;        /* 0x474c4e4400000001 */
    glacier_hip_bank_receipt_t parent;
    uint64_t tree_key, tree_identity_generation;
    uint32_t node_index, reserved0;
    uint64_t generation;
    uint32_t parent_index, reserved1;   /* 0xffffffff for a scope */
    uint64_t parent_generation, node_key, tenant_key, binding_key;
    uint32_t kind, reserved2;
    glacier_hip_claim_t ceiling, claim;
    uint64_t integrity;
} glacier_hip_lease_node_t;        /* LeaseNodeV1 (resource_bank.zig:314-330) */

typedef struct {
    glacier_hip_claim_t used, peak;
    uint64_t peak_host_bytes, active_reservations, committed_receipts;
    uint64_t active_lease_trees, active_lease_scopes, active_lease_nodes;
    uint64_t reserved_unmaterialized_allocations, live_allocations;
    uint64_t quiescing_allocations, free_authorized_allocations;
    uint64_t successful_reservations, successful_commits, cancellations, releases;
    uint64_t rejected_capacity, rejected_slots;
    uint64_t lease_tree_opens, lease_scope_opens, lease_allocation_reserves;
    uint64_t lease_allocation_materializations, lease_allocation_aborts;
    uint64_t lease_reclaim_prepares, lease_reclaim_authorizations, lease_reclaim_cancels;
    uint64_t lease_reclaim_commits, lease_tree_closes;
    uint64_t rejected_lease_capacity, rejected_lease_nodes;
} glacier_hip_lease_bank_snapshot_t;  /* SnapshotV3's accounting fields (resource_bank.zig:703-754) */

typedef struct glacier_hip_lease_bank glacier_hip_lease_bank;
/* Bank.initWithLeaseTree (:929-974): `slot_count` receipt slots, one tree
 * root per slot, `node_count` lease nodes shared by every tree. */
glacier_hip_lease_bank *glacier_hip_lease_bank_create(uint32_t slot_count, uint32_t node_count,
                                                      const glacier_hip_limits_t *limits,
                                                      uint64_t epoch);
void glacier_hip_lease_bank_destroy(glacier_hip_lease_bank *b);
/* reserve (:976-1044) then commit (:1046-1076); cancel (:1078-1095) a reservation. */
int glacier_hip_lease_bank_reserve(glacier_hip_lease_bank *b, uint64_t owner_key,
                                   const glacier_hip_claim_t *claim,
                                   glacier_hip_bank_receipt_t *reservation_out);
int glacier_hip_lease_bank_commit(glacier_hip_lease_bank *b,
                                  const glacier_hip_bank_receipt_t *reservation,
                                  glacier_hip_bank_receipt_t *receipt_out);
int glacier_hip_lease_bank_cancel(glacier_hip_lease_bank *b,
                                  const glacier_hip_bank_receipt_t *reservation);
/* release (:3166-3184): no publication session, no live tree. */
int glacier_hip_lease_bank_release(glacier_hip_lease_bank *b, const glacier_hip_bank_receipt_t *receipt);
int glacier_hip_lease_tree_open(glacier_hip_lease_bank *b, const glacier_hip_bank_receipt_t *receipt,
                                uint64_t tree_key, uint64_t authority_key,
                                const glacier_hip_claim_t *ceiling, glacier_hip_lease_tree_t *tree_out);
/* Adds a scope; *tree is replaced by the tree after the change. */
int glacier_hip_lease_scope_open(glacier_hip_lease_bank *b, glacier_hip_lease_tree_t *tree,
                                 uint64_t scope_key, uint64_t tenant_key,
                                 const glacier_hip_claim_t *ceiling, glacier_hip_lease_node_t *scope_out);
/* closeLeaseTree (:2582-2622): only empty scopes left, session unbound. */
int glacier_hip_lease_tree_close(glacier_hip_lease_bank *b, const glacier_hip_lease_tree_t *tree);
int glacier_hip_lease_tree_validate(glacier_hip_lease_bank *b, const glacier_hip_lease_tree_t *tree);
int glacier_hip_lease_node_validate(glacier_hip_lease_bank *b, const glacier_hip_lease_tree_t *tree,
                                    const glacier_hip_lease_node_t *node);
int glacier_hip_lease_session_bind(glacier_hip_lease_bank *b, const glacier_hip_lease_tree_t *tree,
                                   uint64_t request_epoch, uint64_t session_id);
int glacier_hip_lease_session_close(glacier_hip_lease_bank *b, const glacier_hip_bank_receipt_t *receipt,
                                    uint64_t request_epoch, uint64_t session_id,
                                    uint64_t expected_next_sequence);
int glacier_hip_lease_bank_snapshot(glacier_hip_lease_bank *b, glacier_hip_lease_bank_snapshot_t *out);
/* A publication fence permit (PublicationPermit, resource_bank.zig:2938-3102):
 * one live permit per receipt slot; commit advances the slot's sequence,
 * abort returns the permit and keeps the sequence. */
typedef struct {
    glacier_hip_bank_receipt_t receipt;
    uint64_t request_epoch, session_id, sequence, generation, integrity;
} glacier_hip_publication_permit_t;
/* beginPublicationWithLeaseTree (:2938-2960): the tree has no pending batch,
 * the session is bound at `expected_sequence` and no permit is live. */
int glacier_hip_lease_publication_begin(glacier_hip_lease_bank *b, const glacier_hip_lease_tree_t *tree,
                                        uint64_t request_epoch, uint64_t session_id,
                                        uint64_t expected_sequence,
                                        glacier_hip_publication_permit_t *permit_out);
/* commitPublicationAssumeValid (:3076-3089) and abortPublication (:3091-3102),
 * both behind validatePublicationPermit (:4133-4155): a stale, copied or
 * forged permit is GLACIER_HIP_LEASE_INVALID_TRANSITION and changes nothing. */
int glacier_hip_lease_publication_commit(glacier_hip_lease_bank *b,
                                         const glacier_hip_publication_permit_t *permit);
int glacier_hip_lease_publication_abort(glacier_hip_lease_bank *b,
                                        const glacier_hip_publication_permit_t *permit);

/* The page-lease coordinator of one lane (LeasedPagedKVCache :292-1466).
 * `bindings` is caller-owned storage, one entry per logical page of the
 * lane's page map (bindingStorageBytes :94-101); `tree` and `sequence` are
 * caller-owned cells shared by every lane of one cohort (the coordinators
 * read and replace them). */
enum { GLACIER_HIP_BINDING_FREE = 0, GLACIER_HIP_BINDING_LIVE = 1,
       GLACIER_HIP_BINDING_FREED_PENDING_UNCHARGE = 2 };
typedef struct {
    uint64_t abi_version;        /* 0x4750_4c42_0000_0001 */
    uint32_t state, has_leaf;
    uint64_t cache_instance, logical_page, payload_bytes;
    uint32_t scope_index, reserved0;
    uint64_t scope_generation;
    glacier_hip_lease_node_t leaf;
    uint64_t integrity;
} glacier_hip_page_lease_binding_t;  /* PageLeaseBindingV1 (:62-72) */

typedef struct {
    uint32_t count, reserved0;
    uint64_t payload_bytes;
    uint8_t digest[32];
} glacier_hip_binding_summary_t;     /* BindingSummaryV1 (:74-78) */

/* ---- leased publication waves: ProposalV3 (paged_lease_token_txn.zig) ----
 * A staged wave over leased lanes hashes the v3 proposal: the v1 head minus
 * the capacity word plus the LeaseTree and leased-KV ABIs, the cohort's
 * parent receipt, a redacted commitment to the cohort's tree, one resource
 * commitment per lane slot (lifecycle, coordinator and cache instances,
 * scope, page-map root after the wave, KV state chain after, the canonical
 * logical-KV digest after a first or terminal row, the terminal seal's
 * generation, the lane's binding summary and allocation-set commitment) and
 * LaneProposalV3 lanes (with the output digest after the token and the
 * terminal reason). Leased lanes publishing v3 waves chain their KV state
 * under the v3 domains. Layouts: the reference's fields in order, u8/bool
 * widened to u32, the reference's widths hashed. */
typedef struct {
    uint64_t abi_version;            /* 0x47504c4100000002 */
    uint32_t count, reserved;
    uint64_t payload_bytes;
    uint8_t sha256[32];
} glacier_hip_allocation_set_v2_t;      /* AllocationSetCommitmentV2 (leased_paged_kv_cache.zig:85-90) */

typedef struct {
    uint64_t abi_version;            /* 0x47504c5400000003 */
    uint64_t tree_key, identity_generation, generation, structural_revision;
    glacier_hip_claim_t ceiling, current;
    uint32_t active_nodes, reserved;
    uint64_t state_digest, token_integrity;
} glacier_hip_lease_tree_commitment_v3_t;  /* LeaseTreeCommitmentV3 (paged_lease_token_txn.zig:127-139) */

enum { GLACIER_HIP_LIFECYCLE_LIVE = 0, GLACIER_HIP_LIFECYCLE_TERMINAL_RETAINED = 1,
       GLACIER_HIP_LIFECYCLE_FREED_PENDING_UNCHARGE = 2, GLACIER_HIP_LIFECYCLE_RECLAIMED = 3 };

typedef struct {
    uint64_t abi_version;            /* 0x47504c4300000005 */
    uint32_t lane_index, lifecycle;
    uint64_t coordinator_instance, cache_instance;
    uint32_t scope_index, reserved0;
    uint64_t scope_generation;
    glacier_hip_page_map_root_t root;
    uint8_t kv_state_chain_after[32];
    uint32_t has_canonical_after, reserved1;
    uint8_t canonical_after_sha256[32];
    uint32_t has_terminal_generation, reserved2;
    uint64_t terminal_generation;
    uint32_t has_binding_summary, reserved3;
    glacier_hip_binding_summary_t binding_summary;
    glacier_hip_allocation_set_v2_t allocation_set;
} glacier_hip_resource_commitment_v3_t;  /* ResourceCommitmentV3 (:141-160) */

typedef struct {
    uint32_t lane_index, has_kv_transition;
    uint64_t step_index, prompt_len, kv_before, kv_after;
    glacier_hip_root_transition_v1_t kv_transition;  /* RootTransitionV3: the same fields */
    uint64_t output_before, output_after;
    uint8_t output_sha256[32];
    uint64_t rng_before[4], rng_after[4];
    uint64_t sampling_calls_before, sampling_calls_after;
    uint32_t token_id;
    uint32_t terminal_reason;        /* 0 none, 1 + TerminalReason */
} glacier_hip_lane_proposal_v3_t;       /* LaneProposalV3 (:107-124) */

typedef struct {
    uint64_t abi_version;            /* 0x47504c5800000004 */
    uint64_t resource_bank_abi, resource_lease_tree_abi, resource_publication_fence_abi;
    uint64_t leased_paged_kv_abi, paged_kv_abi, page_transition_abi;
    uint64_t execution_abi, request_epoch, transaction_sequence, resource_permit_generation;
    uint32_t live_mask, live_lane_count;
    glacier_hip_bank_receipt_t parent_receipt;
    glacier_hip_lease_tree_commitment_v3_t tree;
    glacier_hip_resource_commitment_v3_t resources[GLACIER_HIP_PUBLICATION_WIDTH];
    glacier_hip_lane_proposal_v3_t lanes[GLACIER_HIP_PUBLICATION_WIDTH];
} glacier_hip_token_proposal_v3_t;      /* ProposalV3 (:162-180) */

/* proposalSha256 (:1013-1084) and commitSha256 (:1086-1098) of the v3 wave. */
int glacier_hip_token_proposal_v3_sha256(const glacier_hip_token_proposal_v3_t *proposal,
                                         uint8_t out[32]);
int glacier_hip_token_commit_v3_sha256(const uint8_t proposal_sha256[32],
                                       const glacier_hip_prepare_ack_v1_t *ack, uint8_t out[32]);
/* Kernel probe (a measurement hook of this library, no reference
 * counterpart): with kind >= 0 every later decode step launches directly
 * and records HIP events on its stream around that launch of every layer,
 * adding the elapsed times; -1 turns it off. Each call resets the totals. */
enum { GLACIER_HIP_PROBE_QKV = 0, GLACIER_HIP_PROBE_ATTENTION = 1, GLACIER_HIP_PROBE_O = 2,
       GLACIER_HIP_PROBE_GATE_UP = 3, GLACIER_HIP_PROBE_DOWN = 4 };
int glacier_hip_session_probe_kernel(glacier_hip_session *s, int kind);
int glacier_hip_session_probe_read(glacier_hip_session *s, double *total_us, uint64_t *launches);
/* Replays the last decode step's gate/up or down launches of all layers
 * (kind GLACIER_HIP_PROBE_GATE_UP / _DOWN: launches that write only step
 * scratch) `reps` times back to back on the step stream, with the step's
 * own inputs and each layer's weights, HIP events around the whole run;
 * *avg_us = elapsed / (reps x layers). Lane state is not touched. */
int glacier_hip_session_probe_replay(glacier_hip_session *s, int kind, uint32_t reps, double *avg_us);

/* step_prepare for a wave whose lanes are all leased lanes of one cohort,
 * sealed as ProposalV3 (Batch.begin :1117-1250). terminal_reason[i]: 0, or
 * 1 + the TerminalReason of lane i's token (eos / max_tokens / cancelled).
 * The ack names the v3 digest; step_commit / step_abort finish the wave (the
 * commit digest is commitSha256 v3, terminal seals bind both v3 digests). */
int glacier_hip_session_step_prepare_v3(glacier_hip_session *s, const uint32_t *lanes,
                                        const uint32_t *tokens, uint32_t count,
                                        const uint64_t *eligible_words_host,
                                        const glacier_hip_publication_binding_t *binding,
                                        const uint32_t *terminal_reason,
                                        glacier_hip_token_proposal_v3_t *proposal_out,
                                        uint8_t proposal_sha256_out[32], uint32_t *next_tokens);

typedef struct {
    uint64_t abi_version;        /* RowAllocationPlanV1 (paged_kv_cache.zig:113-128) */
    uint64_t cache_id, cache_instance, base_len, logical_page, row_in_page;
    uint64_t root_generation, row_txn_generation, root_after_generation;
    uint64_t page_ownership_generation, next_page_ownership_generation, allocated_pages;
    uint32_t page_payload_present, reserved0;
    uint64_t allocation_bytes;
} glacier_hip_row_allocation_plan_t;

typedef struct {
    uint64_t abi_version;        /* 0x4750_4c50_0000_0001 */
    uint64_t coordinator_instance;
    glacier_hip_lease_tree_t tree;
    uint64_t publication_sequence;
    glacier_hip_row_allocation_plan_t cache_plan;
    glacier_hip_binding_summary_t bindings;
    uint64_t integrity;
} glacier_hip_leased_row_plan_t;     /* LeasedRowPlanV1 (:103-111) */

typedef struct {
    uint64_t abi_version;        /* 0x4750_4c52_0000_0001 */
    uint64_t coordinator_instance, generation;
    glacier_hip_row_txn_mark_t mark;
    uint32_t installed_new_binding, reserved0;
    uint8_t bindings_digest[32];
    uint64_t integrity;
} glacier_hip_leased_row_txn_t;      /* LeasedRowTxnV1 (:113-121) */

enum { GLACIER_HIP_TERMINAL_EOS = 0, GLACIER_HIP_TERMINAL_MAX_TOKENS = 1,
       GLACIER_HIP_TERMINAL_CANCELLED = 2 };
typedef struct {
    uint64_t abi_version;        /* 0x4750_4c53_0000_0001 */
    uint64_t coordinator_instance, cache_id, cache_instance;
    uint32_t scope_index, reserved0;
    uint64_t scope_generation, tree_identity_generation, tree_generation;
    uint64_t tree_structural_revision, tree_state_digest;
    glacier_hip_page_map_root_t root;
    uint8_t logical_kv_sha256[32];
    glacier_hip_binding_summary_t bindings;
    uint64_t transaction_sequence;
    uint32_t terminal_reason, terminal_token;
    uint64_t generation;
    uint8_t digest[32];
} glacier_hip_terminal_seal_t;       /* TerminalSealV1 (:150-171) */

typedef struct {
    uint64_t abi_version;        /* 0x4750_4c46_0000_0001 */
    uint64_t coordinator_instance, generation;
    uint8_t terminal_seal_digest[32];
    uint64_t permit_generation;
    glacier_hip_page_map_root_t root_before, root_after;
    uint32_t binding_count, reserved0;
    uint64_t payload_bytes;
    uint8_t bindings_digest[32];
    uint64_t integrity;
} glacier_hip_freed_payload_t;       /* FreedPayloadV1 (:241-253) */

typedef struct {
    uint64_t abi_version;        /* 0x4750_4c43_0000_0002 */
    uint64_t coordinator_instance, generation;
    glacier_hip_freed_payload_t freed;
    glacier_hip_lease_tree_t tree_after;
    uint64_t integrity;
} glacier_hip_reclaim_receipt_t;     /* ReclaimReceiptV1 (:255-262) */

enum { GLACIER_HIP_LEASE_LIVE = 0, GLACIER_HIP_LEASE_TERMINAL_RETAINED = 1,
       GLACIER_HIP_LEASE_FREED_PENDING_UNCHARGE = 2, GLACIER_HIP_LEASE_RECLAIMED = 3 };

typedef struct glacier_hip_leased_kv glacier_hip_leased_kv;
/* LeasedPagedKVCache.init (:311-357) over a host page map (which must be
 * empty and not yet leased) or over one lane of a device session (begun and
 * empty; its decode steps and prefills then charge each new page payload
 * through the lease before the step takes it, and a failed step uncharges
 * it). A page payload is page_payload_bytes of the map: f32 for host maps,
 * the session's KV dtype for lanes. */
int glacier_hip_leased_kv_create(glacier_hip_lease_bank *b, glacier_hip_lease_tree_t *tree,
                                 const glacier_hip_lease_node_t *scope, glacier_hip_kv_pages *pages,
                                 glacier_hip_page_lease_binding_t *bindings, uint32_t binding_count,
                                 uint64_t request_epoch, uint64_t session_id, uint64_t *sequence,
                                 glacier_hip_leased_kv **out);
int glacier_hip_leased_kv_create_for_lane(glacier_hip_lease_bank *b, glacier_hip_lease_tree_t *tree,
                                          const glacier_hip_lease_node_t *scope,
                                          glacier_hip_session *s, uint32_t lane,
                                          glacier_hip_page_lease_binding_t *bindings,
                                          uint32_t binding_count, uint64_t request_epoch,
                                          uint64_t session_id, uint64_t *sequence,
                                          glacier_hip_leased_kv **out);
/* Ends the coordinator object; a session lane is unleased (its pages stay). */
void glacier_hip_leased_kv_destroy(glacier_hip_leased_kv *c);
/* planNextRow (:453-480) / beginRowPlanned (:482-565) / commitRowTxn
 * (:666-676) / abortRowTxn (:678-689), for host page maps. */
int glacier_hip_leased_kv_plan_next_row(glacier_hip_leased_kv *c, glacier_hip_leased_row_plan_t *out);
int glacier_hip_leased_kv_begin_row(glacier_hip_leased_kv *c, const glacier_hip_leased_row_plan_t *plan,
                                    glacier_hip_leased_row_txn_t *txn_out);
int glacier_hip_leased_kv_commit_row(glacier_hip_leased_kv *c, const glacier_hip_leased_row_txn_t *txn,
                                     glacier_hip_page_map_root_t *root_out);
int glacier_hip_leased_kv_abort_row(glacier_hip_leased_kv *c, const glacier_hip_leased_row_txn_t *txn);
int glacier_hip_leased_kv_binding_summary(glacier_hip_leased_kv *c, glacier_hip_binding_summary_t *out);
int glacier_hip_leased_kv_lifecycle(glacier_hip_leased_kv *c, uint32_t *out);
/* allocationSetCommitment (:364-369, allocationSetCommitmentForState
 * :1253-1291): the exact live allocation set, each non-free binding with its
 * LeaseNode leaf, as AllocationSetCommitmentV2. */
int glacier_hip_leased_kv_allocation_set(glacier_hip_leased_kv *c,
                                         glacier_hip_allocation_set_v2_t *out);
int glacier_hip_leased_kv_root(glacier_hip_leased_kv *c, glacier_hip_page_map_root_t *out);
int glacier_hip_leased_kv_kv_sha256(glacier_hip_leased_kv *c, uint8_t out[32]);
/* sealTerminalForPublication (:691-757): binds the committed root and
 * logical KV digest, then takes and commits the cohort's publication permit
 * for `transaction_sequence` (the shared sequence cell advances). */
int glacier_hip_leased_kv_seal_terminal(glacier_hip_leased_kv *c, const glacier_hip_page_map_root_t *root,
                                        const uint8_t logical_kv_sha256[32],
                                        uint64_t transaction_sequence, uint32_t reason,
                                        uint32_t terminal_token, glacier_hip_terminal_seal_t *seal_out);
/* beginTerminalReclaim (:852-867, beginReclaimExact :918-1036): retire the
 * lane's scope, free every payload back to the pool (the map is retired),
 * charges stay until commit_reclaim (commitReclaimAfterFree :1040-1080). */
int glacier_hip_leased_kv_begin_reclaim(glacier_hip_leased_kv *c, const glacier_hip_terminal_seal_t *seal,
                                        uint64_t expected_sequence, glacier_hip_freed_payload_t *out);
int glacier_hip_leased_kv_commit_reclaim(glacier_hip_leased_kv *c, const glacier_hip_freed_payload_t *freed,
                                         glacier_hip_reclaim_receipt_t *out);
/* The lane's terminal seal: the one seal_terminal made, or the one a staged
 * publication wave made when it published the lane's terminal token (then
 * its digest also binds that wave's proposal and commit digests, returned
 * here; zeros for a seal_terminal seal). TERMINAL_REQUIRED before either. */
int glacier_hip_leased_kv_terminal_seal(glacier_hip_leased_kv *c, glacier_hip_terminal_seal_t *out,
                                        uint8_t proposal_sha256[32], uint8_t commit_sha256[32]);
/* reclaimForTeardown (:894-916): abort a staged row, retire and uncharge. */
int glacier_hip_leased_kv_reclaim_for_teardown(glacier_hip_leased_kv *c, uint64_t expected_sequence);

/* Host rows of a host page map: the K and V rows of a staged row at one
 * layer (appendRowTxn, paged_kv_cache.zig:1074-1103) and the logical KV
 * digest of the committed rows (logicalKvSha256, the session lanes' digest
 * over f32 rows). */
int glacier_hip_kv_pages_append_row(glacier_hip_kv_pages *p, const glacier_hip_row_txn_mark_t *mark,
                                    uint32_t layer, const float *k, const float *v);
int glacier_hip_kv_pages_kv_sha256(glacier_hip_kv_pages *p, uint8_t out[32]);
/* A retired map (after a leased reclaim) rejects every row. */
int glacier_hip_kv_pages_is_retired(glacier_hip_kv_pages *p, int32_t *out);
/* The payload pool as an allocator with a limit: at most `pages` payloads
 * held by the map and free together (not below what the map holds). */
int glacier_hip_kv_pages_set_pool_capacity(glacier_hip_kv_pages *p, uint32_t pages);

/* Version of this ABI. */
uint64_t glacier_hip_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif
