// session.hip — model + session: the per-token decode step over paged KV.
//
// Host-side semantics restated from the reference:
//  * layer composition  generate.zig:1511-1967 (forwardLayerCached)
//  * token loop         generate.zig:4665-5613 (prefill one token at a time,
//                       then greedy decode; first token from the prompt logits)
//  * paged KV pages     paged_kv_cache.zig:1006-1160 (beginRow installs a page
//                       at row 0 with ownership_generation = next++, the root
//                       digest chain appendOwnershipDigest :341-353, commit /
//                       abort of the row transaction)
//  * digests            generate.zig:3150-3203
//  * RNG                std.Random.DefaultPrng.init(seed) (generate.zig:5221)
#include <math.h>
#include <string.h>

#include <algorithm>
#include <array>

#include "host_util.h"
#include "lane_weave.h"
#include "leased_kv.h"
#include "paged_kv.h"
#include "publication.h"
#include "runtime.h"
#include "page_image.h"

#include <map>
#include "runtime_image.h"
#include "glacier_container.h"

using gh::hip_fail;

namespace {

struct LayerDev {
  float *in_norm = nullptr, *post_norm = nullptr, *qkv_bias = nullptr;
  glacier_hip_int4_weight *qkv = nullptr, *o = nullptr, *gu = nullptr, *down = nullptr;
};

}  // namespace

struct glacier_hip_model {
  glacier_hip_context *ctx = nullptr;
  glacier_hip_model_config_t cfg{};
  std::vector<LayerDev> layers;
  std::vector<bool> layer_set;
  bool globals_set = false;
  float *embed = nullptr, *final_norm = nullptr;
  glacier_hip_int4_weight *head = nullptr;
  uint64_t bytes = 0;
};

struct Lane {
  gpk::Cache kv;                  // page map, generations, committed root
  uint64_t sampling_calls = 0;
  uint64_t rng[4] = {0, 0, 0, 0};
  std::vector<uint32_t> output;
  // staged publication (paged_token_txn.zig): the prompt length, a first
  // token held back for the first wave, the lane's KV state chain
  uint64_t prompt_len = 0;
  bool first_pending = false;
  uint32_t first_token = 0;
  bool chain_init = false;
  uint8_t chain[32] = {};
  bool retired = false;           // a terminal token was published
  glacier_hip_leased_kv *lease = nullptr;  // page payloads charged through a LeaseTree
  // leased v3 waves (paged_lease_token_txn.zig): the lane's chain runs under
  // the v3 domains and its publication slot is fixed by its first v3 wave
  bool chain_v3 = false;
  int v3_slot = -1;
};

// A staged publication wave between step_prepare and commit / abort.
struct PreparedWave {
  bool active = false, first = false, elig = false;
  std::vector<gpk::RowTxn> txns;
  std::vector<uint32_t> lanes, slots, tokens;
  glacier_hip_token_proposal_v1_t proposal{};
  uint8_t sha[32] = {};
  // leased lanes: the cohort's publication permit fences the whole wave
  // (paged_lease_token_txn.zig: one Bank permit per B4 wave)
  glacier_hip_leased_kv *cohort = nullptr;
  glb::PubPermit permit{};
  // a v3 wave (every lane a leased lane of the cohort): the proposal hashed,
  // and each lane's terminal reason (0 none, 1 + TerminalReason)
  bool v3 = false;
  glacier_hip_token_proposal_v3_t proposal_v3{};
  std::vector<uint32_t> reasons;
};

constexpr int kRow0Pages = 28;  // page ids of row 0 carried in the step inputs
struct StepInputs {  // uploaded once per decode step, in one copy
  // row 0 in one 128-byte line: lane, context length, position, 0, then its
  // first kRow0Pages page ids, so the one-lane attention reads everything
  // its page walk needs in one memory round trip
  alignas(128) int32_t row0[4 + kRow0Pages];
  int32_t tokens[64];
  int32_t lane_of_row[64];
  int32_t pos_of_row[64];
  int32_t ctx_len[64];
};

// Device arrays describing the activation rows of one launch sequence.
struct RowPtrs {
  const int32_t *tokens, *lane_of_row, *pos_of_row, *ctx_len;
  const int32_t *row0 = nullptr;  // StepInputs::row0, or null
  // a prefill chunk: every row is lane chunk_lane, rows at consecutive
  // positions from chunk_pos0 (-1: rows of arbitrary lanes / positions)
  int chunk_lane = -1, chunk_pos0 = 0;
};

struct glacier_hip_session {
  glacier_hip_model *model = nullptr;
  glacier_hip_session_options_t opt{};
  uint32_t max_pages = 0;  // per lane
  uint32_t total_pages = 0;
  uint32_t rows_cap = 0;   // max(max_lanes, prefill_chunk): rows of the scratch buffers
  uint32_t prefill_chunk = 0;
  // eligible-step head domain: GLACIER_HIP_HEAD_DOMAIN_POSTHEAD (every
  // logit, then the masked argmax) or _PREHEAD (row blocks with no eligible
  // token stream no weights)
  int head_domain = GLACIER_HIP_HEAD_DOMAIN_POSTHEAD;
  gpk::PagePool pool;
  std::vector<Lane> lanes;
  // device
  void *kv_pool = nullptr;
  int32_t *page_table = nullptr;
  float *rope_cos = nullptr, *rope_sin = nullptr;
  float *x_res = nullptr, *h = nullptr, *q = nullptr, *attn = nullptr, *act = nullptr,
        *logits = nullptr;
  int8_t *act_q = nullptr;
  gk::ActMeta *act_meta = nullptr;
  int8_t *act_q2 = nullptr;         // planes emitted by the gate/up epilogue for down
  gk::ActMeta *act_meta2 = nullptr;
  uint32_t planes2_rows = 0;        // rows act_q2 / act_meta2 hold
  float *splitk_ws = nullptr;       // GEMM split-K partial sums
  size_t splitk_floats = 0;
  unsigned *splitk_counters = nullptr;  // GEMM split-K arrivals per tile (0 at rest)
  float *ss_parts = nullptr;        // deferred RMSNorm partial sums [32][1024]
  float *o_parts = nullptr;         // fused attention + O: [num_kv_heads][dim]
  unsigned *o_counters = nullptr;   // fused attention + O: arrivals per row group (0 at rest)
  int attn_o = -1;                  // fused attention + O usable: -1 not yet known, 0, 1
  float *att_scratch = nullptr;
  void *arg_scratch = nullptr;
  uint32_t *arg_counters = nullptr;
  gk::ArgmaxResult *arg_result = nullptr;
  uint64_t *elig_words = nullptr;
  StepInputs *step_dev = nullptr;
  int32_t *pf_dev = nullptr;     // prefill rows: tokens, lane, pos, ctx [4][prefill_chunk]
  // host pinned
  StepInputs *step_host = nullptr;
  int32_t *pf_host = nullptr;
  int32_t *pt_host = nullptr;    // mirror of page_table [max_lanes][max_pages]
  gk::ArgmaxResult *res_host = nullptr;
  bool inject_failure = false;
  // test tap: with a buffer, each decode step copies the residual after
  // every layer into tap_x [num_layers][rows][dim] (direct launches only)
  float *tap_x = nullptr;
  uint32_t tap_rows = 0;
  bool tap_now = false;
  // kernel probe: with a kind (GLACIER_HIP_PROBE_*), each decode step
  // records HIP events on the step stream around that launch in every layer
  // (direct launches, as the traced step) and adds their elapsed times
  int probe_kind = -1;
  bool probe_now = false;
  std::vector<hipEvent_t> probe_ev;
  uint32_t probe_used = 0;
  double probe_ms = 0.0;
  uint64_t probe_count = 0;
  // probe replay: enqueue_layers launches only this kind (-1: every launch);
  // the last decode step's shape, which a replay repeats
  int probe_only = -1;
  uint32_t last_rows = 0;
  bool last_fused = false;
  PreparedWave prep;
  // sealed step plans: key = (rows, with_head, eligible, prehead, fused
  // attention + O). The step's launches are captured once (every host-side
  // check and launch-shape choice made then); use_graph 1 replays the
  // recorded kernel launches, 2 the instantiated graph.
  struct GraphEntry {
    uint32_t rows;
    bool head, elig, pre, fused;
    hipGraph_t graph;                            // kept: `launches` point into it
    hipGraphExec_t exec;                         // use_graph 2
    std::vector<hipKernelNodeParams> launches;   // use_graph 1, in dependency order
  };
  std::vector<GraphEntry> graphs;
};

// ---------------------------------------------------------------------------
// model
// ---------------------------------------------------------------------------
static int upload_f32(glacier_hip_context *ctx, float **dst, const float *src, size_t n) {
  if (!*dst) GH_CHECK(ctx, gh::dev_malloc(ctx, (void **)dst, n * 4));
  if (src) GH_CHECK(ctx, hipMemcpy(*dst, src, n * 4, hipMemcpyHostToDevice));
  else GH_CHECK(ctx, hipMemset(*dst, 0, n * 4));
  return GLACIER_HIP_OK;
}

extern "C" {

glacier_hip_model *glacier_hip_model_create(glacier_hip_context *ctx,
                                            const glacier_hip_model_config_t *cfg) {
  if (!ctx || !cfg) return nullptr;
  const auto &c = *cfg;
  if (c.num_layers == 0 || c.dim == 0 || c.hidden_dim == 0 || c.num_heads == 0 ||
      c.num_kv_heads == 0 || c.num_heads % c.num_kv_heads != 0 ||
      c.num_heads / c.num_kv_heads > 8 || (c.head_dim != 64 && c.head_dim != 128) ||
      c.dim % 128 != 0 || c.hidden_dim % 128 != 0 || c.vocab_size % 16 != 0 ||
      c.group_size != 32 || c.num_heads * c.head_dim != c.dim) {
    ctx->last_error = "model config unsupported";
    return nullptr;
  }
  auto *m = new glacier_hip_model();
  m->ctx = ctx;
  m->cfg = c;
  m->layers.resize(c.num_layers);
  m->layer_set.assign(c.num_layers, false);
  return m;
}

static int set_layer_impl(glacier_hip_model *m, uint32_t li, const glacier_hip_layer_host_t &w,
                          const uint16_t *s16[7]) {
  glacier_hip_context *ctx = m->ctx;
  const auto &c = m->cfg;
  const uint32_t D = c.dim, F = c.hidden_dim, hd = c.head_dim;
  const uint32_t kvd = c.num_kv_heads * hd;
  LayerDev &L = m->layers[li];
  int rc;
  if ((rc = upload_f32(ctx, &L.in_norm, w.input_norm, D))) return rc;
  if ((rc = upload_f32(ctx, &L.post_norm, w.post_attn_norm, D))) return rc;
  auto src = [&](const uint8_t *p, const float *s32, int idx, uint64_t row) {
    return gh::RowSrc{p, s32, s16 ? s16[idx] : nullptr, row};
  };
  // fused QKV: q and k rows grouped as RoPE pairs (p, p + hd/2), 8 pairs per block
  std::vector<gh::RowSrc> rows;
  rows.reserve(D + 2 * kvd);
  auto add_rope_rows = [&](const uint8_t *p, const float *s32, int idx, uint32_t heads) {
    for (uint32_t h = 0; h < heads; ++h)
      for (uint32_t b = 0; b < hd / 16; ++b) {
        for (uint32_t i = 0; i < 8; ++i) rows.push_back(src(p, s32, idx, h * hd + 8 * b + i));
        for (uint32_t i = 0; i < 8; ++i)
          rows.push_back(src(p, s32, idx, h * hd + 8 * b + i + hd / 2));
      }
  };
  add_rope_rows(w.wq, w.sq, 0, c.num_heads);
  add_rope_rows(w.wk, w.sk, 1, c.num_kv_heads);
  for (uint32_t r = 0; r < kvd; ++r) rows.push_back(src(w.wv, w.sv, 2, r));
  std::vector<uint32_t> codes;
  std::vector<uint16_t> scales;
  auto build = [&](glacier_hip_int4_weight **dst, uint32_t K) -> int {
    gh::repack_tiles(rows, K, codes, scales);
    if (*dst) glacier_hip_int4_weight_destroy(*dst);
    *dst = gh::upload_weight(ctx, (uint32_t)rows.size(), K, codes, scales);
    return *dst ? GLACIER_HIP_OK : GLACIER_HIP_OUT_OF_MEMORY;
  };
  if ((rc = build(&L.qkv, D))) return rc;
  if (w.bq || w.bk || w.bv) {
    std::vector<float> b(D + 2 * kvd, 0.0f);
    if (w.bq) memcpy(b.data(), w.bq, D * 4);
    if (w.bk) memcpy(b.data() + D, w.bk, kvd * 4);
    if (w.bv) memcpy(b.data() + D + kvd, w.bv, kvd * 4);
    if ((rc = upload_f32(ctx, &L.qkv_bias, b.data(), b.size()))) return rc;
  }
  rows.clear();
  for (uint32_t r = 0; r < D; ++r) rows.push_back(src(w.wo, w.so, 3, r));
  if ((rc = build(&L.o, D))) return rc;
  // fused gate/up: rows 0..7 gate 8b..8b+7, rows 8..15 up 8b..8b+7
  rows.clear();
  for (uint32_t b = 0; b < F / 8; ++b) {
    for (uint32_t i = 0; i < 8; ++i) rows.push_back(src(w.w_gate, w.s_gate, 4, 8 * b + i));
    for (uint32_t i = 0; i < 8; ++i) rows.push_back(src(w.w_up, w.s_up, 5, 8 * b + i));
  }
  if ((rc = build(&L.gu, D))) return rc;
  rows.clear();
  for (uint32_t r = 0; r < D; ++r) rows.push_back(src(w.w_down, w.s_down, 6, r));
  if ((rc = build(&L.down, F))) return rc;
  m->layer_set[li] = true;
  return GLACIER_HIP_OK;
}

int glacier_hip_model_set_layer(glacier_hip_model *m, uint32_t layer,
                                const glacier_hip_layer_host_t *w) {
  if (!m || !w) return GLACIER_HIP_INVALID_ARGUMENT;
  if (layer >= m->cfg.num_layers) return GLACIER_HIP_SHAPE_MISMATCH;
  if (!w->wq || !w->wk || !w->wv || !w->wo || !w->w_gate || !w->w_up || !w->w_down || !w->sq ||
      !w->sk || !w->sv || !w->so || !w->s_gate || !w->s_up || !w->s_down || !w->input_norm ||
      !w->post_attn_norm)
    return GLACIER_HIP_INVALID_ARGUMENT;
  return set_layer_impl(m, layer, *w, nullptr);
}

int glacier_hip_model_set_globals(glacier_hip_model *m, const float *token_embedding,
                                  const float *final_norm, const uint8_t *lm_head_packed,
                                  const float *lm_head_scales) {
  if (!m || !token_embedding || !final_norm || !lm_head_packed || !lm_head_scales)
    return GLACIER_HIP_INVALID_ARGUMENT;
  const auto &c = m->cfg;
  int rc;
  if ((rc = upload_f32(m->ctx, &m->embed, token_embedding, (size_t)c.vocab_size * c.dim))) return rc;
  if ((rc = upload_f32(m->ctx, &m->final_norm, final_norm, c.dim))) return rc;
  if (m->head) glacier_hip_int4_weight_destroy(m->head);
  m->head = glacier_hip_int4_weight_create(m->ctx, lm_head_packed, (uint64_t)c.vocab_size * c.dim / 2,
                                           lm_head_scales, (uint64_t)c.vocab_size * c.dim / 32, 32,
                                           c.dim, c.vocab_size);
  if (!m->head) return GLACIER_HIP_OUT_OF_MEMORY;
  m->globals_set = true;
  return GLACIER_HIP_OK;
}

int glacier_hip_model_init_random(glacier_hip_model *m, uint64_t seed) {
  if (!m) return GLACIER_HIP_INVALID_ARGUMENT;
  const auto &c = m->cfg;
  const uint32_t D = c.dim, F = c.hidden_dim, kvd = c.num_kv_heads * c.head_dim, V = c.vocab_size;
  const float sigma = 0.02f;
  std::vector<float> n1(D), n2(D);
  std::vector<uint8_t> wq((size_t)D * D / 2), wk((size_t)kvd * D / 2), wv((size_t)kvd * D / 2),
      wo((size_t)D * D / 2), wg((size_t)F * D / 2), wu((size_t)F * D / 2), wd((size_t)D * F / 2);
  std::vector<uint16_t> sq((size_t)D * D / 32), sk((size_t)kvd * D / 32), sv((size_t)kvd * D / 32),
      so((size_t)D * D / 32), sg((size_t)F * D / 32), su((size_t)F * D / 32), sd((size_t)D * F / 32);
  for (uint32_t l = 0; l < c.num_layers; ++l) {
    auto id = [&](uint32_t which) { return glacier_hip_synth_tensor_id(l, which); };
    glacier_hip_synth_normal_f32(seed, id(0), sigma, n1.data(), D);
    glacier_hip_synth_normal_f32(seed, id(1), sigma, n2.data(), D);
    uint8_t *ws[7] = {wq.data(), wk.data(), wv.data(), wo.data(), wg.data(), wu.data(), wd.data()};
    size_t wb[7] = {wq.size(), wk.size(), wv.size(), wo.size(), wg.size(), wu.size(), wd.size()};
    uint16_t *ss[7] = {sq.data(), sk.data(), sv.data(), so.data(), sg.data(), su.data(), sd.data()};
    size_t sn[7] = {sq.size(), sk.size(), sv.size(), so.size(), sg.size(), su.size(), sd.size()};
    for (int i = 0; i < 7; ++i) {
      glacier_hip_synth_int4(seed, id(2 + 2 * i), ws[i], wb[i]);
      glacier_hip_synth_scales_f16(seed, id(3 + 2 * i), sigma, ss[i], sn[i]);
    }
    glacier_hip_layer_host_t w{};
    w.input_norm = n1.data();
    w.post_attn_norm = n2.data();
    w.wq = wq.data(); w.wk = wk.data(); w.wv = wv.data(); w.wo = wo.data();
    w.w_gate = wg.data(); w.w_up = wu.data(); w.w_down = wd.data();
    const uint16_t *s16[7] = {sq.data(), sk.data(), sv.data(), so.data(), sg.data(), su.data(), sd.data()};
    int rc = set_layer_impl(m, l, w, s16);
    if (rc) return rc;
  }
  const uint32_t G = 0xFFFFFF;
  std::vector<float> emb((size_t)V * D), fn(D);
  glacier_hip_synth_normal_f32(seed, glacier_hip_synth_tensor_id(G, 20), sigma, emb.data(), emb.size());
  glacier_hip_synth_normal_f32(seed, glacier_hip_synth_tensor_id(G, 21), sigma, fn.data(), D);
  std::vector<uint8_t> hp((size_t)V * D / 2);
  std::vector<uint16_t> hs((size_t)V * D / 32);
  glacier_hip_synth_int4(seed, glacier_hip_synth_tensor_id(G, 22), hp.data(), hp.size());
  glacier_hip_synth_scales_f16(seed, glacier_hip_synth_tensor_id(G, 23), sigma, hs.data(), hs.size());
  int rc;
  if ((rc = upload_f32(m->ctx, &m->embed, emb.data(), emb.size()))) return rc;
  if ((rc = upload_f32(m->ctx, &m->final_norm, fn.data(), D))) return rc;
  if (m->head) glacier_hip_int4_weight_destroy(m->head);
  m->head = glacier_hip_int4_weight_create_f16scales(m->ctx, hp.data(), hp.size(), hs.data(),
                                                     hs.size(), 32, D, V);
  if (!m->head) return GLACIER_HIP_OUT_OF_MEMORY;
  m->globals_set = true;
  return GLACIER_HIP_OK;
}

void glacier_hip_model_destroy(glacier_hip_model *m) {
  if (!m) return;
  for (auto &L : m->layers) {
    gh::dev_free(m->ctx, L.in_norm);
    gh::dev_free(m->ctx, L.post_norm);
    gh::dev_free(m->ctx, L.qkv_bias);
    glacier_hip_int4_weight_destroy(L.qkv);
    glacier_hip_int4_weight_destroy(L.o);
    glacier_hip_int4_weight_destroy(L.gu);
    glacier_hip_int4_weight_destroy(L.down);
  }
  gh::dev_free(m->ctx, m->embed);
  gh::dev_free(m->ctx, m->final_norm);
  glacier_hip_int4_weight_destroy(m->head);
  delete m;
}

int glacier_hip_model_quote(glacier_hip_context *ctx, const glacier_hip_model_config_t *cfg,
                            int with_qkv_bias, glacier_hip_allocation_quote_t *out) {
  // the allocations set_layer (x num_layers) and set_globals make
  if (!ctx || !cfg || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  const auto &c = *cfg;
  if (c.num_layers == 0 || c.dim == 0 || c.hidden_dim == 0 || c.vocab_size == 0)
    return GLACIER_HIP_SHAPE_MISMATCH;
  const uint64_t D = c.dim, F = c.hidden_dim, V = c.vocab_size;
  const uint64_t kvd = (uint64_t)c.num_kv_heads * c.head_dim;
  uint64_t req = 0, chg = 0;
  auto add = [&](uint64_t b) {
    req += b;
    chg += gh::charged_bytes(b);
  };
  auto weight = [&](uint64_t N, uint64_t K) {  // tile codes + fp16 scales
    add(N * K / 2);
    add(N * K / 16);
  };
  for (uint32_t l = 0; l < c.num_layers; ++l) {
    add(D * 4);
    add(D * 4);
    weight(D + 2 * kvd, D);
    if (with_qkv_bias) add((D + 2 * kvd) * 4);
    weight(D, D);
    weight(2 * F, D);
    weight(D, F);
  }
  add(V * D * 4);
  add(D * 4);
  weight(V, D);
  out->requested_bytes = req;
  out->charged_bytes = chg;
  out->context_epoch = ctx->epoch;
  return GLACIER_HIP_OK;
}

uint64_t glacier_hip_model_weight_bytes(const glacier_hip_model *m) {
  if (!m) return 0;
  uint64_t b = 0;
  for (const auto &L : m->layers)
    b += glacier_hip_int4_weight_device_bytes(L.qkv) + glacier_hip_int4_weight_device_bytes(L.o) +
         glacier_hip_int4_weight_device_bytes(L.gu) + glacier_hip_int4_weight_device_bytes(L.down);
  return b + glacier_hip_int4_weight_device_bytes(m->head);
}

}  // extern "C"


// ---------------------------------------------------------------------------
// prepared runtime image -> device model (loader.zig:193-390)
// ---------------------------------------------------------------------------
namespace gri {
const Image *image_of(const glacier_hip_glrt_image *h);
}

namespace {

struct Int4View {
  const uint8_t *packed = nullptr;
  const float *s32 = nullptr;     // f32 scales (may be null)
  const uint16_t *s16 = nullptr;  // f16 scale mirror (may be null)
  uint64_t scales = 0;
};

// preparedRaw (loader.zig:785-809)
uint32_t prepared_raw(const gri::Image &img, uint32_t layer, uint32_t kind, uint64_t n,
                      bool required, const float **out) {
  *out = nullptr;
  const glacier_hip_glrt_record_t *r = gri::find(img, layer, kind, gri::kTensor);
  if (!r) return required ? GLACIER_HIP_GLRT_MISSING_TENSOR : GLACIER_HIP_GLRT_OK;
  if (r->encoding != gri::kRawF32 || r->packed_layout != gri::kLayoutNone || r->group_size != 0 ||
      r->out_f != 1 || r->in_f != n || r->num_elements != n)
    return GLACIER_HIP_GLRT_BAD_PAYLOAD;
  uint64_t len = 0;
  *out = (const float *)gri::stream(img, *r, gri::kRaw, &len);
  return len == n * 4 ? GLACIER_HIP_GLRT_OK : GLACIER_HIP_GLRT_BAD_PAYLOAD;
}

// preparedInt4 (loader.zig:811-868), then what this device runs: row-major
// nibbles, group 32, and f32 or f16 (non-rows4) scales
uint32_t prepared_int4(const gri::Image &img, uint32_t layer, uint32_t kind, uint64_t out_f,
                       uint64_t in_f, bool require_f32, Int4View *v) {
  const glacier_hip_glrt_record_t *r = gri::find(img, layer, kind, gri::kTensor);
  if (!r) return GLACIER_HIP_GLRT_MISSING_TENSOR;
  const uint64_t n = out_f * in_f;
  if (r->encoding != gri::kInt4 || r->group_size == 0 || r->out_f != out_f || r->in_f != in_f ||
      r->num_elements != n)
    return GLACIER_HIP_GLRT_BAD_PAYLOAD;
  uint64_t lp, l32, l16, l16r;
  v->packed = gri::stream(img, *r, gri::kPacked, &lp);
  v->s32 = (const float *)gri::stream(img, *r, gri::kScalesF32, &l32);
  v->s16 = (const uint16_t *)gri::stream(img, *r, gri::kScalesF16, &l16);
  gri::stream(img, *r, gri::kScalesF16Rows4, &l16r);
  const uint64_t sc = (n + r->group_size - 1) / r->group_size;
  if (lp != (n + 1) / 2 || (l32 && l32 != sc * 4) || (l16 && l16 != sc * 2) ||
      (l16r && l16r != sc * 2) || (!l32 && !l16 && !l16r) || (require_f32 && l32 != sc * 4))
    return GLACIER_HIP_GLRT_BAD_PAYLOAD;
  if (r->packed_layout == gri::kRows4K16 && (out_f % 4 || in_f % 16 || l16r != sc * 2))
    return GLACIER_HIP_GLRT_BAD_PAYLOAD;
  if (r->packed_layout == gri::kLayoutNone) return GLACIER_HIP_GLRT_BAD_PAYLOAD;
  // the device's tile layout is built from row-major nibbles and group-32
  // scales (f32 or the plain f16 mirror)
  if (r->packed_layout != gri::kRowMajor || r->group_size != 32 || (!l32 && !l16))
    return GLACIER_HIP_GLRT_UNSUPPORTED;
  v->scales = sc;
  return GLACIER_HIP_GLRT_OK;
}

// isExpectedPreparedRecord (loader.zig:731-768)
bool expected_record(const glacier_hip_glrt_info_t &c, const glacier_hip_glrt_record_t &r) {
  if (r.role == gri::kMlpGateUpPair) return r.layer_idx != gri::kGlobalLayer && r.layer_idx < c.layers;
  if (r.role != gri::kTensor) return false;
  if (r.layer_idx == gri::kGlobalLayer)
    return r.kind == gri::kFinalNorm || r.kind == gri::kEmbedding ||
           (r.kind == gri::kLmHead && !c.tie_embeddings);
  if (r.layer_idx >= c.layers) return false;
  switch (r.kind) {
    case gri::kInputNorm: case gri::kAttnQ: case gri::kAttnK: case gri::kAttnV: case gri::kAttnO:
    case gri::kAttnQBias: case gri::kAttnKBias: case gri::kAttnVBias: case gri::kAttnOBias:
    case gri::kPostAttnNorm: case gri::kMlpGate: case gri::kMlpUp: case gri::kMlpDown:
      return true;
    default:
      return false;
  }
}

// f16 scales for the tile layout: the mirror when present, else f32 -> f16
// (round to nearest even), counting the values fp16 does not hold exactly
const uint16_t *scales_f16(const Int4View &v, std::vector<uint16_t> &buf, uint64_t *inexact) {
  if (v.s16) return v.s16;
  buf.resize(v.scales);
  for (uint64_t i = 0; i < v.scales; ++i) {
    buf[i] = gh::f32_to_f16(v.s32[i]);
    if (gh::f16_to_f32(buf[i]) != v.s32[i]) ++*inexact;
  }
  return buf.data();
}

}  // namespace

extern "C" glacier_hip_model *glacier_hip_model_load_glrt(glacier_hip_context *ctx,
                                                          const glacier_hip_glrt_image *handle,
                                                          glacier_hip_glrt_load_report_t *report) {
  glacier_hip_glrt_load_report_t rep{};
  glacier_hip_model *m = nullptr;
  auto fail = [&](uint32_t e, const char *what) -> glacier_hip_model * {
    rep.error = e;
    if (report) *report = rep;
    if (ctx) ctx->last_error = std::string("glrt load: ") + gri::error_name(e) + " (" + what + ")";
    glacier_hip_model_destroy(m);
    return nullptr;
  };
  const gri::Image *img = gri::image_of(handle);
  if (!ctx || !img) return fail(GLACIER_HIP_GLRT_BAD_PAYLOAD, "null context or image");
  const glacier_hip_glrt_info_t &c = img->info;
  // validatePreparedConfig (loader.zig:618-654)
  if ((uint64_t)c.heads * c.head_dim != c.dim || c.kv_heads > c.heads || c.heads % c.kv_heads)
    return fail(GLACIER_HIP_GLRT_BAD_PAYLOAD, "config");
  // validatePreparedRecordSet (loader.zig:656-716): expected records only,
  // and one homogeneous MLP layout (separate gate/up is what this device runs)
  for (const auto &r : img->records)
    if (!expected_record(c, r)) return fail(GLACIER_HIP_GLRT_BAD_PAYLOAD, "unexpected record");
  for (uint32_t l = 0; l < c.layers; ++l) {
    const bool gate = gri::find(*img, l, gri::kMlpGate, gri::kTensor) != nullptr;
    const bool up = gri::find(*img, l, gri::kMlpUp, gri::kTensor) != nullptr;
    const bool pair = gri::find(*img, l, 0, gri::kMlpGateUpPair) != nullptr;
    if (pair) {
      if (gate || up) return fail(GLACIER_HIP_GLRT_BAD_PAYLOAD, "gate/up pair beside gate or up");
      return fail(GLACIER_HIP_GLRT_UNSUPPORTED, "PairNibble gate/up");
    }
    if (!gate || !up) return fail(GLACIER_HIP_GLRT_MISSING_TENSOR, "gate/up");
  }
  rep.separate_mlp = 1;
  const uint64_t D = c.dim, F = c.hidden_dim, V = c.vocab, kvd = (uint64_t)c.kv_heads * c.head_dim;
  glacier_hip_model_config_t mc{};
  mc.num_layers = c.layers;
  mc.dim = c.dim;
  mc.hidden_dim = c.hidden_dim;
  mc.num_heads = c.heads;
  mc.num_kv_heads = c.kv_heads;
  mc.head_dim = c.head_dim;
  mc.vocab_size = c.vocab;
  mc.group_size = 32;
  mc.rms_eps = c.rms_eps;
  mc.rope_theta = c.rope_theta;
  m = glacier_hip_model_create(ctx, &mc);
  if (!m) return fail(GLACIER_HIP_GLRT_UNSUPPORTED, "model shape");
  std::vector<uint16_t> sbuf[7];
  uint32_t e;
  for (uint32_t l = 0; l < c.layers; ++l) {
    glacier_hip_layer_host_t w{};
    const float *bo = nullptr;
    if ((e = prepared_raw(*img, l, gri::kInputNorm, D, true, &w.input_norm)) ||
        (e = prepared_raw(*img, l, gri::kPostAttnNorm, D, true, &w.post_attn_norm)) ||
        (e = prepared_raw(*img, l, gri::kAttnQBias, D, false, &w.bq)) ||
        (e = prepared_raw(*img, l, gri::kAttnKBias, kvd, false, &w.bk)) ||
        (e = prepared_raw(*img, l, gri::kAttnVBias, kvd, false, &w.bv)) ||
        (e = prepared_raw(*img, l, gri::kAttnOBias, D, false, &bo)))
      return fail(e, "layer norms / biases");
    if (bo) return fail(GLACIER_HIP_GLRT_UNSUPPORTED, "attn_o bias");
    const uint32_t kinds[7] = {gri::kAttnQ, gri::kAttnK, gri::kAttnV, gri::kAttnO,
                               gri::kMlpGate, gri::kMlpUp, gri::kMlpDown};
    const uint64_t outs[7] = {D, kvd, kvd, D, F, F, D}, ins[7] = {D, D, D, D, D, D, F};
    Int4View v[7];
    const uint16_t *s16[7];
    for (int i = 0; i < 7; ++i) {
      if ((e = prepared_int4(*img, l, kinds[i], outs[i], ins[i], false, &v[i])))
        return fail(e, "layer projection");
      s16[i] = scales_f16(v[i], sbuf[i], &rep.inexact_scales);
      rep.int4_records++;
    }
    w.wq = v[0].packed; w.wk = v[1].packed; w.wv = v[2].packed; w.wo = v[3].packed;
    w.w_gate = v[4].packed; w.w_up = v[5].packed; w.w_down = v[6].packed;
    int rc = set_layer_impl(m, l, w, s16);
    if (rc) return fail(GLACIER_HIP_GLRT_BAD_PAYLOAD, "device upload");
    rep.raw_records += 2 + (w.bq != nullptr) + (w.bk != nullptr) + (w.bv != nullptr);
  }
  const float *final_norm = nullptr;
  if ((e = prepared_raw(*img, gri::kGlobalLayer, gri::kFinalNorm, D, true, &final_norm)))
    return fail(e, "final_norm");
  // the token embedding is INT4 with f32 scales; dequantizeRow
  // (int4_matmul.zig:3164-3194) per element: NIBBLE_TO_OFFSET[u] * scale
  Int4View emb, head;
  if ((e = prepared_int4(*img, gri::kGlobalLayer, gri::kEmbedding, V, D, true, &emb)))
    return fail(e, "embedding");
  if (c.tie_embeddings) {
    head = emb;
  } else if ((e = prepared_int4(*img, gri::kGlobalLayer, gri::kLmHead, V, D, false, &head))) {
    return fail(e, "lm_head");
  }
  std::vector<float> table(V * D);
  gh::parallel_for(V, [&](size_t r0, size_t r1) {
    for (size_t r = r0; r < r1; ++r)
      for (size_t k = 0; k < D; ++k) {
        const size_t idx = r * D + k;
        const uint8_t b = emb.packed[idx / 2];
        const int u = (idx & 1) ? b >> 4 : b & 0xF;
        table[idx] = (float)(u - 7) * emb.s32[idx / 32];
      }
  }, 256);
  std::vector<float> head_s(head.scales);
  std::vector<uint16_t> hbuf;
  const uint16_t *h16 = scales_f16(head, hbuf, &rep.inexact_scales);
  for (uint64_t i = 0; i < head.scales; ++i) head_s[i] = gh::f16_to_f32(h16[i]);
  rep.int4_records += c.tie_embeddings ? 1 : 2;
  rep.raw_records += 1;
  int rc = glacier_hip_model_set_globals(m, table.data(), final_norm, head.packed, head_s.data());
  if (rc) return fail(GLACIER_HIP_GLRT_BAD_PAYLOAD, "device upload");
  rep.uploaded_bytes = m->bytes ? m->bytes : glacier_hip_model_weight_bytes(m);
  if (report) *report = rep;
  return m;
}

// ---------------------------------------------------------------------------
// portable .glacier container -> device model (loader.zig:1214-1592)
// ---------------------------------------------------------------------------
namespace gct {
const Container *container_of(const glacier_hip_glacier *h);
}

extern "C" glacier_hip_model *glacier_hip_model_load_glacier(glacier_hip_context *ctx,
                                                            const glacier_hip_glacier *handle,
                                                            const glacier_hip_model_config_t *override,
                                                            int tie_word_embeddings,
                                                            glacier_hip_glacier_load_report_t *report) {
  glacier_hip_glacier_load_report_t rep{};
  glacier_hip_model *m = nullptr;
  auto fail = [&](uint32_t e, const char *what) -> glacier_hip_model * {
    rep.error = e;
    if (report) *report = rep;
    if (ctx) ctx->last_error = std::string("glacier load: ") + gct::error_name(e) + " (" + what + ")";
    glacier_hip_model_destroy(m);
    return nullptr;
  };
  const gct::Container *c = gct::container_of(handle);
  if (!ctx || !c) return fail(GLACIER_HIP_GLAC_INVALID_ARGUMENT, "null context or container");
  gct::Geometry geo;
  if (uint32_t e = gct::derive_geometry(*c, &geo)) return fail(e, "geometry");
  std::map<gct::GroupKey, gct::Group> groups;
  if (uint32_t e = gct::materialize(*c, groups)) return fail(e, "tensor pages");
  // the JSON sidecar's overrides on top of the page geometry (:1540-1556)
  const glacier_hip_model_config_t o = override ? *override : glacier_hip_model_config_t{};
  glacier_hip_model_config_t mc{};
  mc.dim = o.dim ? o.dim : (uint32_t)geo.dim;
  mc.hidden_dim = o.hidden_dim ? o.hidden_dim : (uint32_t)geo.hidden_dim;
  mc.num_layers = o.num_layers ? o.num_layers : geo.num_layers;
  mc.vocab_size = o.vocab_size ? o.vocab_size : (uint32_t)geo.vocab_size;
  mc.rms_eps = o.rms_eps != 0.0f ? o.rms_eps : 1e-6f;
  mc.rope_theta = o.rope_theta != 0.0f ? o.rope_theta : 10000.0f;
  mc.num_heads = o.num_heads ? o.num_heads : (mc.dim >= 64 && mc.dim % 64 == 0 ? mc.dim / 64 : 1);
  mc.head_dim = o.head_dim ? o.head_dim : (mc.dim >= 64 && mc.dim % 64 == 0 ? 64 : mc.dim);
  mc.num_kv_heads = o.num_kv_heads ? o.num_kv_heads : mc.num_heads;
  mc.group_size = 32;
  rep.config = mc;
  m = glacier_hip_model_create(ctx, &mc);
  if (!m) return fail(GLACIER_HIP_GLAC_UNSUPPORTED, "model shape");
  const uint64_t D = mc.dim, F = mc.hidden_dim, V = mc.vocab_size;
  const uint64_t kvd = (uint64_t)mc.num_kv_heads * mc.head_dim;
  auto find = [&](uint32_t layer, uint32_t kind) -> const gct::Group * {
    auto it = groups.find({layer, kind});
    return it == groups.end() ? nullptr : &it->second;
  };
  // a decoded (f32) tensor of n values; required ones are MissingTensor when absent
  auto raw = [&](uint32_t layer, uint32_t kind, uint64_t n, bool required, const float **out) -> uint32_t {
    *out = nullptr;
    const gct::Group *g = find(layer, kind);
    if (!g) return required ? GLACIER_HIP_GLAC_MISSING_TENSOR : GLACIER_HIP_GLAC_OK;
    if (g->int4) return GLACIER_HIP_GLAC_UNSUPPORTED;  // a norm or bias must decode to values
    if (g->values.size() != n) return GLACIER_HIP_GLAC_BAD_PAYLOAD;
    *out = g->values.data();
    return GLACIER_HIP_GLAC_OK;
  };
  // a merged INT4 tensor of out_f x in_f, group 32 (what this device runs)
  auto int4 = [&](uint32_t layer, uint32_t kind, uint64_t out_f, uint64_t in_f,
                  const gct::Group **out) -> uint32_t {
    const gct::Group *g = find(layer, kind);
    *out = g;
    if (!g) return GLACIER_HIP_GLAC_MISSING_TENSOR;
    if (!g->int4 || g->group_size != 32) return GLACIER_HIP_GLAC_UNSUPPORTED;
    if (g->elements != out_f * in_f) return GLACIER_HIP_GLAC_BAD_PAYLOAD;
    return GLACIER_HIP_GLAC_OK;
  };
  auto f16_scales = [&](const gct::Group &g, std::vector<uint16_t> &buf) {
    buf.resize(g.scales.size());
    for (size_t i = 0; i < g.scales.size(); ++i) {
      buf[i] = gh::f32_to_f16(g.scales[i]);
      if (gh::f16_to_f32(buf[i]) != g.scales[i]) ++rep.inexact_scales;
    }
    return buf.data();
  };
  std::vector<uint16_t> sbuf[7];
  uint32_t e;
  for (uint32_t l = 0; l < mc.num_layers; ++l) {
    glacier_hip_layer_host_t w{};
    const float *bo = nullptr;
    const uint32_t kinds[7] = {gri::kAttnQ, gri::kAttnK, gri::kAttnV, gri::kAttnO,
                               gri::kMlpGate, gri::kMlpUp, gri::kMlpDown};
    const uint64_t outs[7] = {D, kvd, kvd, D, F, F, D}, ins[7] = {D, D, D, D, D, D, F};
    const gct::Group *g[7];
    const uint16_t *s16[7];
    for (int i = 0; i < 7; ++i) {
      if ((e = int4(l, kinds[i], outs[i], ins[i], &g[i]))) return fail(e, "layer projection");
      s16[i] = f16_scales(*g[i], sbuf[i]);
      rep.int4_tensors++;
    }
    if ((e = raw(l, gri::kInputNorm, D, true, &w.input_norm)) ||
        (e = raw(l, gri::kPostAttnNorm, D, true, &w.post_attn_norm)) ||
        (e = raw(l, gri::kAttnQBias, D, false, &w.bq)) ||
        (e = raw(l, gri::kAttnKBias, kvd, false, &w.bk)) ||
        (e = raw(l, gri::kAttnVBias, kvd, false, &w.bv)) ||
        (e = raw(l, gri::kAttnOBias, D, false, &bo)))
      return fail(e, "layer norms / biases");
    if (bo) return fail(GLACIER_HIP_GLAC_UNSUPPORTED, "attn_o bias");
    w.wq = g[0]->packed.data(); w.wk = g[1]->packed.data(); w.wv = g[2]->packed.data();
    w.wo = g[3]->packed.data(); w.w_gate = g[4]->packed.data(); w.w_up = g[5]->packed.data();
    w.w_down = g[6]->packed.data();
    if (set_layer_impl(m, l, w, s16)) return fail(GLACIER_HIP_GLAC_BAD_PAYLOAD, "device upload");
    rep.raw_tensors += 2 + (w.bq != nullptr) + (w.bk != nullptr) + (w.bv != nullptr);
  }
  // globals live at layer 0 (:1513-1530)
  const float *final_norm = nullptr;
  if ((e = raw(0, gri::kFinalNorm, D, true, &final_norm))) return fail(e, "final_norm");
  const gct::Group *emb = find(0, gri::kEmbedding);
  if (!emb) return fail(GLACIER_HIP_GLAC_MISSING_TENSOR, "embedding");
  std::vector<float> table;
  const float *table_p = nullptr;
  if (emb->int4) {
    if (emb->elements != V * D) return fail(GLACIER_HIP_GLAC_BAD_PAYLOAD, "embedding");
    // the gather table: each element's code offset times its group's f32 scale
    table.resize(V * D);
    const uint32_t gs = emb->group_size;
    gh::parallel_for(V, [&](size_t r0, size_t r1) {
      for (size_t r = r0; r < r1; ++r)
        for (size_t k = 0; k < D; ++k) {
          const size_t idx = r * D + k;
          const uint8_t b = emb->packed[idx / 2];
          const int u = (idx & 1) ? b >> 4 : b & 0xF;
          table[idx] = (float)(u - 7) * emb->scales[idx / gs];
        }
    }, 256);
    table_p = table.data();
  } else {
    if (emb->values.size() != V * D) return fail(GLACIER_HIP_GLAC_BAD_PAYLOAD, "embedding");
    table_p = emb->values.data();
  }
  const gct::Group *head = nullptr;
  if ((e = int4(0, tie_word_embeddings ? gri::kEmbedding : gri::kLmHead, V, D, &head)))
    return fail(e, tie_word_embeddings ? "tied head (INT4 embedding)" : "lm_head");
  std::vector<uint16_t> hbuf;
  const uint16_t *h16 = f16_scales(*head, hbuf);
  std::vector<float> head_s(head->scales.size());
  for (size_t i = 0; i < head_s.size(); ++i) head_s[i] = gh::f16_to_f32(h16[i]);
  rep.int4_tensors += tie_word_embeddings ? 1 : (emb->int4 ? 2 : 1);
  rep.raw_tensors += 1 + (emb->int4 ? 0 : 1);
  if (glacier_hip_model_set_globals(m, table_p, final_norm, head->packed.data(), head_s.data()))
    return fail(GLACIER_HIP_GLAC_BAD_PAYLOAD, "device upload");
  rep.uploaded_bytes = glacier_hip_model_weight_bytes(m);
  if (report) *report = rep;
  return m;
}

// ---------------------------------------------------------------------------
// session
// ---------------------------------------------------------------------------
namespace {

struct GemvPlan {
  int S;
};

int layer_D(const glacier_hip_session *s, uint32_t out_f, uint32_t in_f) {
  return gh::resolve_activation(s->opt.layer_activation, out_f, in_f) == GLACIER_HIP_ACT_Q8 ? 1 : 3;
}

int head_D(const glacier_hip_session *s) {
  const auto &c = s->model->cfg;
  return gh::resolve_activation(s->opt.head_activation, c.vocab_size, c.dim) == GLACIER_HIP_ACT_Q8 ? 1 : 3;
}

// One projection over `rows` activation rows with the given epilogue. The
// input is an f32 matrix x (optionally RMS-normalised with norm_w) or int8
// digit planes a producer already emitted. An f32 input is converted into
// planes (Q8, or the 3-digit f32 representation) either by a separate
// kernel or, for decode-sized row sets whose planes fit in LDS, by the GEMV
// itself while its weights stream in; in that input mode the RMSNorm is
// deferred: the planes are quantised from x * w and the per-row 1/rms factor
// (which cancels in the group quantiser, q = round(v * 127 / max|v|)) is
// applied to the outputs from the producer's partial sums of squares.
struct ProjIn {
  const float *x = nullptr;
  const float *norm_w = nullptr;
  const float *ss = nullptr;  // producer's partial sums of x^2 [rows][ss_count]
  int ss_count = 0;
  const int8_t *planes_q = nullptr;
  const gk::ActMeta *planes_m = nullptr;
};
struct ProjOut {
  float *y = nullptr;
  const float *resid = nullptr;
  const float *bias = nullptr;
  const gk::QkvArgs *qkv = nullptr;
  gk::PlanesDst emit{nullptr, nullptr, 1};  // next projection's planes (SwiGLU; GEMM: residual)
  const float *emit_norm_w = nullptr;       // GEMM residual emission: the next RMSNorm
  float *ss_out = nullptr;                  // EPI_RESID: partial sums of y^2
  gk::ArgPartial *arg_parts = nullptr;      // EPI_PLAIN: fused greedy head
  const uint64_t *arg_words = nullptr;
  long arg_word_count = 0;
  bool prehead = false;                     // skip row blocks with no eligible row
};

// GEMM tiles whose K splits can meet at a counter (the largest decode-lane
// grids are about 1200 tiles)
constexpr int kSplitkCounters = 4096;

gk::GemvArgs proj_args(glacier_hip_session *s, glacier_hip_int4_weight *w, int D, int rows,
                       int epi, const ProjIn &in, const ProjOut &out) {
  gk::GemvArgs a{};
  a.codes = w->codes;
  a.scales = w->scales;
  a.N = (int)w->out_f;
  a.K = (int)w->in_f;
  a.M = rows;
  a.D = D;
  a.epi = epi;
  a.bias = out.bias;
  a.y = out.y;
  a.resid = out.resid;
  if (out.qkv) a.qkv = *out.qkv;
  a.act_q = in.planes_q;
  a.act_meta = in.planes_m;
  a.out_q = out.emit.q;
  a.out_meta = out.emit.meta;
  a.out_D = out.emit.D;
  a.emit_norm_w = out.emit_norm_w;
  a.ss_out = out.ss_out;
  a.arg_parts = out.arg_parts;
  a.arg_words = out.arg_words;
  a.arg_word_count = out.arg_word_count;
  a.prehead = out.prehead ? 1 : 0;
  a.in_eps = s->model->cfg.rms_eps;
  a.splitk_ws = s->splitk_ws;
  a.splitk_ws_floats = s->splitk_floats;
  a.splitk_counters = s->splitk_counters;
  a.splitk_counter_count = s->splitk_counters ? kSplitkCounters : 0;
  return a;
}

// GEMV arguments in input mode (planes built in LDS, deferred RMSNorm), or
// false when this projection cannot run that way. Every workgroup quantises
// the whole input, so the mode only pays for a few rows: from 8 rows on the
// separate conversion kernel plus the plain GEMV measured faster (7B QKV and
// gate/up), about even at 4-5.
constexpr int kInputModeRows = 4;
// A prompt chunk of more rows than this (one lane, consecutive positions)
// runs the prefill attention kernel; shorter chunks the decode kernel.
constexpr int kPrefillAttnRows = 16;

bool input_mode_args(glacier_hip_session *s, glacier_hip_int4_weight *w, int D, int rows, int epi,
                     const ProjIn &in, const ProjOut &out, gk::GemvArgs *a) {
  if (!in.x || rows > kInputModeRows || (in.norm_w && !in.ss)) return false;
  *a = proj_args(s, w, D, rows, epi, in, out);
  a->x_in = in.x;
  a->norm_w = in.norm_w;
  a->in_ss = in.ss;
  a->in_ss_count = in.ss_count;
  gk::GemvShape p;
  return gk::gemv_launch_shape(*a, &p);
}

// Workgroups (= ss_out partials per row) of a decode projection.
int proj_grid(glacier_hip_session *s, glacier_hip_int4_weight *w, int D, int rows, int epi,
              const ProjIn &in, const ProjOut &out) {
  gk::GemvArgs a;
  if (!input_mode_args(s, w, D, rows, epi, in, out, &a)) {
    a = proj_args(s, w, D, rows, epi, in, out);
    if (in.x) {  // the separate conversion kernel fills these
      a.act_q = s->act_q;
      a.act_meta = s->act_meta;
    }
  }
  gk::GemvShape p;
  return gk::gemv_launch_shape(a, &p) ? p.grid : -1;
}

hipError_t run_proj(glacier_hip_session *s, glacier_hip_int4_weight *w, int D, int rows, int epi,
                    const ProjIn &in, const ProjOut &out, hipStream_t st) {
  const bool decode = rows <= gk::kGemvMaxRows;
  // partial sums and the fused head are GEMV-only (the GEMM emits planes
  // when gemm_emit_ok says so)
  if (!decode && (out.ss_out || out.arg_parts)) return hipErrorInvalidValue;
  gk::GemvArgs a;
  if (input_mode_args(s, w, D, rows, epi, in, out, &a)) return gk::launch_gemv(a, st);
  a = proj_args(s, w, D, rows, epi, in, out);
  if (in.x) {
    hipError_t e = gk::launch_prep_act(in.x, 0, in.norm_w, s->model->cfg.rms_eps, rows,
                                       (int)w->in_f, D, s->act_q, s->act_meta, nullptr, st);
    if (e != hipSuccess) return e;
    a.act_q = s->act_q;
    a.act_meta = s->act_meta;
  }
  return decode ? gk::launch_gemv(a, st) : gk::launch_gemm(a, st);
}

// Whether a GEMM-sized projection can finish by emitting the next
// projection's planes (its inputs come from planes or the conversion kernel,
// both into act_q, so that is what the check assumes).
bool gemm_emit_ok(glacier_hip_session *s, glacier_hip_int4_weight *w, int D, int rows, int epi,
                  const ProjIn &in, const ProjOut &out) {
  if (rows <= gk::kGemvMaxRows) return false;
  ProjIn pin;  // the planes the launch reads: in's, or the conversion kernel's
  pin.planes_q = in.x ? s->act_q : in.planes_q;
  pin.planes_m = in.x ? s->act_meta : in.planes_m;
  const gk::GemvArgs a = proj_args(s, w, D, rows, epi, pin, out);
  return gk::gemm_emit_ok(a);
}

// Embedding gather and every decoder layer for `rows` activation rows
// (generate.zig:1511-1967 per row; K/V rows land in the rows' pages).
//
// Decode-sized row sets (rows <= kGemvMaxRows) run a chain with no
// conversion kernels:
// the gather and each residual projection (O, down) also write per-workgroup
// sums of squares of their output, from which the next RMSNorm'd projection
// (QKV, gate/up) finishes its deferred norm while it quantises its input in
// LDS (up to kInputModeRows rows; more rows convert with the separate
// kernel); attention writes the O projection's planes and gate/up the down
// projection's. Longer row sets run the GEMM; where its split-K partial
// sums fit the workspace the finishing pass of O and down also writes the
// next RMSNorm'd projection's planes and that of gate/up the down
// projection's, otherwise each input is converted by a separate kernel.
// Arguments of the fused attention + O projection launch for row 0 of rp at
// layer l: the O projection plus the residual x_res into h, with its
// partial sums of squares (one per row group) into ss.
gk::AttnOArgs attn_o_args(glacier_hip_session *s, const RowPtrs &rp, uint32_t l, float *ss) {
  const auto &c = s->model->cfg;
  const glacier_hip_int4_weight *o = s->model->layers[l].o;
  gk::AttnOArgs a{};
  a.q = s->q;
  a.kv_pool = s->kv_pool;
  a.page_table = s->page_table;
  a.max_pages = (int)s->max_pages;
  a.lane_of_row = rp.lane_of_row;
  a.ctx_len = rp.ctx_len;
  a.row0 = rp.row0;
  a.row0_pages = rp.row0 ? (int)std::min<uint32_t>(kRow0Pages, s->max_pages) : 0;
  a.layer = (int)l;
  a.num_layers = (int)c.num_layers;
  a.num_heads = (int)c.num_heads;
  a.num_kv_heads = (int)c.num_kv_heads;
  a.head_dim = (int)c.head_dim;
  a.max_ctx = (int)s->opt.max_positions;
  a.codes = o->codes;
  a.scales = o->scales;
  a.N = (int)o->out_f;
  a.K = (int)o->in_f;
  a.parts = s->o_parts;
  a.resid = s->x_res;
  a.y = s->h;
  a.ss_out = ss;
  a.counters = s->o_counters;
  a.kv_f32 = s->opt.kv_dtype == GLACIER_HIP_F32 ? 1 : 0;
  return a;
}

// Largest context (positions) a fused one-lane step is used for: one work
// item of the fused kernel (longer contexts run correctly but serially
// inside each workgroup, slower than the two launches).
constexpr uint32_t kFusedMaxCtx = 256;

// Whether one-lane decode steps can run attention and the O projection as
// one launch: fp16 or f32 KV, Q8 inputs for O, shapes the fused kernel
// takes, and its row groups within the partial sums gate/up reads; not when
// the session options ask for two launches.
bool attn_o_usable(glacier_hip_session *s) {
  if (s->attn_o >= 0) return s->attn_o == 1;
  const auto &c = s->model->cfg;
  bool ok = !s->opt.split_attention_o &&
            (s->opt.kv_dtype == GLACIER_HIP_F16 || s->opt.kv_dtype == GLACIER_HIP_F32) &&
            s->planes2_rows >= 1 && s->o_parts && s->o_counters && s->ss_parts;
  const RowPtrs rp{s->step_dev->tokens, s->step_dev->lane_of_row, s->step_dev->pos_of_row,
                   s->step_dev->ctx_len};
  for (uint32_t l = 0; ok && l < c.num_layers; ++l) {
    const LayerDev &L = s->model->layers[l];
    ok = layer_D(s, L.o->out_f, L.o->in_f) == 1 && L.o->out_f == c.dim &&
         gk::attn_o_ok(attn_o_args(s, rp, l, s->ss_parts)) &&
         gk::attn_o_groups((int)c.dim) <= 1024;
  }
  s->attn_o = ok ? 1 : 0;
  return ok;
}

hipError_t enqueue_layers(glacier_hip_session *s, int rows, const RowPtrs &rp, hipStream_t st,
                          bool fused = false) {
  glacier_hip_model *m = s->model;
  const auto &c = m->cfg;
  const int D = (int)c.dim;
  const bool chain = rows <= gk::kGemvMaxRows && (uint32_t)rows <= s->planes2_rows;
  gk::QkvArgs q{};
  q.q_out = s->q;
  q.kv_pool = s->kv_pool;
  q.kv_f16 = s->opt.kv_dtype == GLACIER_HIP_F16;
  q.page_table = s->page_table;
  q.max_pages = (int)s->max_pages;
  q.lane_of_row = rp.lane_of_row;
  q.pos_of_row = rp.pos_of_row;
  q.rope_cos = s->rope_cos;
  q.rope_sin = s->rope_sin;
  q.num_layers = (int)c.num_layers;
  q.num_heads = (int)c.num_heads;
  q.num_kv_heads = (int)c.num_kv_heads;
  q.head_dim = (int)c.head_dim;
  // deferred RMSNorm partial sums, for consumers that run in input mode
  float *ss = chain && rows <= kInputModeRows ? s->ss_parts : nullptr;
  // a probe replay launches one kind only; the others' outputs stay as the
  // last step left them
  auto keep = [&](int kind) { return s->probe_only < 0 || s->probe_only == kind; };
  hipError_t e = hipSuccess;
  if (s->probe_only < 0) {
    e = gk::launch_gather_rows(m->embed, rp.tokens, rows, D, s->x_res, st, ss);
    if (e != hipSuccess) return e;
  }
  int ss_count = ss ? gk::gather_ss_parts(D) : 0;  // partial sums behind x_res
  bool x_planes = false;  // GEMM path: the previous down emitted this layer's QKV planes
  auto mark = [&](int kind) -> hipError_t {
    if (!s->probe_now || s->probe_kind != kind || s->probe_used >= s->probe_ev.size())
      return hipSuccess;
    return hipEventRecord(s->probe_ev[s->probe_used++], st);
  };
  for (uint32_t l = 0; l < c.num_layers; ++l) {
    const LayerDev &L = m->layers[l];
    q.layer = (int)l;
    const int Dq = layer_D(s, L.qkv->out_f, L.qkv->in_f);
    const int Do = layer_D(s, L.o->out_f, L.o->in_f);
    const int Dg = layer_D(s, L.gu->out_f / 2, L.gu->in_f);
    const int Dd = layer_D(s, L.down->out_f, L.down->in_f);
    // RMSNorm -> QKV (+RoPE, KV row write into the lane's page)
    ProjIn qin;
    if (x_planes) {
      qin.planes_q = s->act_q;
      qin.planes_m = s->act_meta;
    } else {
      qin.x = s->x_res;
      qin.norm_w = L.in_norm;
      qin.ss = ss;
      qin.ss_count = ss_count;
    }
    ProjOut qout;
    qout.bias = L.qkv_bias;
    qout.qkv = &q;
    if ((e = mark(GLACIER_HIP_PROBE_QKV)) != hipSuccess) return e;
    if (keep(GLACIER_HIP_PROBE_QKV)) e = run_proj(s, L.qkv, Dq, rows, gk::EPI_QKV, qin, qout, st);
    if (e != hipSuccess) return e;
    if ((e = mark(GLACIER_HIP_PROBE_QKV)) != hipSuccess) return e;
    ProjOut gout;
    if (fused) {
      // one lane: attention + the O projection (+ residual, partial sums of
      // h for gate/up's norm) in one launch, then gate/up as in the chain
      if ((e = mark(GLACIER_HIP_PROBE_ATTENTION)) != hipSuccess) return e;
      if (keep(GLACIER_HIP_PROBE_ATTENTION)) e = gk::launch_attn_o(attn_o_args(s, rp, l, ss), st);
      if (e != hipSuccess) return e;
      if ((e = mark(GLACIER_HIP_PROBE_ATTENTION)) != hipSuccess) return e;
      ss_count = gk::attn_o_groups((int)c.dim);
      ProjIn gin;
      gin.x = s->h;
      gin.norm_w = L.post_norm;
      gin.ss = ss;
      gin.ss_count = ss_count;
      gout.emit = gk::PlanesDst{s->act_q2, s->act_meta2, Dd};
      if ((e = mark(GLACIER_HIP_PROBE_GATE_UP)) != hipSuccess) return e;
      if (keep(GLACIER_HIP_PROBE_GATE_UP)) e = run_proj(s, L.gu, Dg, rows, gk::EPI_SWIGLU, gin, gout, st);
      if (e != hipSuccess) return e;
      if ((e = mark(GLACIER_HIP_PROBE_GATE_UP)) != hipSuccess) return e;
    } else {
      // attention: a prompt chunk of one lane past the GEMV size runs the
      // prefill kernel, other steps the decode kernel, which for up to 32 rows
      // also writes the O projection's planes
      const bool pf_attn = rows > kPrefillAttnRows && rp.chunk_lane >= 0 &&
                           s->opt.kv_dtype == GLACIER_HIP_F16;
      const bool o_planes = !pf_attn && rows <= 32 && (uint32_t)rows <= s->planes2_rows;
      const gk::PlanesDst opd = o_planes ? gk::PlanesDst{s->act_q2, s->act_meta2, Do}
                                         : gk::PlanesDst{nullptr, nullptr, 1};
      if ((e = mark(GLACIER_HIP_PROBE_ATTENTION)) != hipSuccess) return e;
      if (!keep(GLACIER_HIP_PROBE_ATTENTION))
        e = hipSuccess;
      else if (pf_attn)
        e = gk::launch_attention_prefill(s->q, s->kv_pool, s->page_table, (int)s->max_pages,
                                         rp.chunk_lane, rp.chunk_pos0, rows, (int)l,
                                         (int)c.num_layers, (int)c.num_heads, (int)c.num_kv_heads,
                                         (int)c.head_dim, s->attn, st);
      else
        e = gk::launch_attention(s->q, s->kv_pool, s->opt.kv_dtype == GLACIER_HIP_F16,
                                 s->page_table, (int)s->max_pages, rp.lane_of_row, rp.ctx_len, rows,
                                 (int)l, (int)c.num_layers, (int)c.num_heads, (int)c.num_kv_heads,
                                 (int)c.head_dim, (int)s->opt.max_positions, s->att_scratch,
                                 s->attn, st, opd);
      if (e != hipSuccess) return e;
      if ((e = mark(GLACIER_HIP_PROBE_ATTENTION)) != hipSuccess) return e;
      // O projection + residual (chain: partial sums of h for gate/up's norm)
      ProjIn oin;
      ProjOut oout;
      oout.y = s->h;
      oout.resid = s->x_res;
      oout.ss_out = ss;
      if (o_planes) {
        oin.planes_q = s->act_q2;
        oin.planes_m = s->act_meta2;
      } else {
        oin.x = s->attn;
      }
      if (ss) {
        ss_count = proj_grid(s, L.o, Do, rows, gk::EPI_RESID, oin, oout);
        if (ss_count <= 0) return hipErrorInvalidValue;
      }
      if (!chain) {  // GEMM: gate/up's planes from O's finishing pass
        oout.emit = gk::PlanesDst{s->act_q2, s->act_meta2, Dg};
        oout.emit_norm_w = L.post_norm;
        if (!gemm_emit_ok(s, L.o, Do, rows, gk::EPI_RESID, oin, oout)) {
          oout.emit = gk::PlanesDst{nullptr, nullptr, 1};
          oout.emit_norm_w = nullptr;
        }
      }
      if ((e = mark(GLACIER_HIP_PROBE_O)) != hipSuccess) return e;
      if (keep(GLACIER_HIP_PROBE_O)) e = run_proj(s, L.o, Do, rows, gk::EPI_RESID, oin, oout, st);
      if (e != hipSuccess) return e;
      if ((e = mark(GLACIER_HIP_PROBE_O)) != hipSuccess) return e;
      // gate/up + SwiGLU (decode sizes: emitted straight into down's planes)
      ProjIn gin;
      if (oout.emit.q) {
        gin.planes_q = s->act_q2;
        gin.planes_m = s->act_meta2;
      } else {
        gin.x = s->h;
        gin.norm_w = L.post_norm;
        gin.ss = ss;
        gin.ss_count = ss_count;
      }
      if (chain) {
        gout.emit = gk::PlanesDst{s->act_q2, s->act_meta2, Dd};
      } else {
        // GEMM: down's planes from gate/up's own tiles (the last K split of
        // each, or every tile without a split) or its finishing pass, else
        // the SwiGLU rows; into act_q when gate/up reads O's planes from
        // act_q2 (so no finished tile overwrites planes another still
        // reads), else into act_q2 up to the rows it holds (gate/up then
        // reads act_q: the conversion kernel's planes), else into act_q by
        // the finishing pass
        gout.emit = gin.planes_q == s->act_q2 ? gk::PlanesDst{s->act_q, s->act_meta, Dd}
                    : (uint32_t)rows <= s->planes2_rows
                        ? gk::PlanesDst{s->act_q2, s->act_meta2, Dd}
                        : gk::PlanesDst{s->act_q, s->act_meta, Dd};
        if (!gout.emit.q || !gemm_emit_ok(s, L.gu, Dg, rows, gk::EPI_SWIGLU, gin, gout)) {
          gout.emit = gk::PlanesDst{nullptr, nullptr, 1};
          gout.y = s->act;
        }
      }
      if ((e = mark(GLACIER_HIP_PROBE_GATE_UP)) != hipSuccess) return e;
      if (keep(GLACIER_HIP_PROBE_GATE_UP)) e = run_proj(s, L.gu, Dg, rows, gk::EPI_SWIGLU, gin, gout, st);
      if (e != hipSuccess) return e;
      if ((e = mark(GLACIER_HIP_PROBE_GATE_UP)) != hipSuccess) return e;
    }
    // down + residual (chain: partial sums of x_res for the next norm)
    ProjIn din;
    ProjOut dout;
    dout.y = s->x_res;
    dout.resid = s->h;
    const bool last = l + 1 == c.num_layers;  // the LM head converts x_res itself
    dout.ss_out = last ? nullptr : ss;
    if (gout.emit.q) {
      din.planes_q = gout.emit.q;
      din.planes_m = gout.emit.meta;
    } else {
      din.x = s->act;
    }
    if (ss && !last) {
      ss_count = proj_grid(s, L.down, Dd, rows, gk::EPI_RESID, din, dout);
      if (ss_count <= 0) return hipErrorInvalidValue;
    }
    x_planes = false;
    if (!chain && !last) {  // GEMM: the next layer's QKV planes from down's finishing pass
      const LayerDev &N = m->layers[l + 1];
      dout.emit = gk::PlanesDst{s->act_q, s->act_meta, layer_D(s, N.qkv->out_f, N.qkv->in_f)};
      dout.emit_norm_w = N.in_norm;
      x_planes = gemm_emit_ok(s, L.down, Dd, rows, gk::EPI_RESID, din, dout);
      if (!x_planes) {
        dout.emit = gk::PlanesDst{nullptr, nullptr, 1};
        dout.emit_norm_w = nullptr;
      }
    }
    if ((e = mark(GLACIER_HIP_PROBE_DOWN)) != hipSuccess) return e;
    if (keep(GLACIER_HIP_PROBE_DOWN)) e = run_proj(s, L.down, Dd, rows, gk::EPI_RESID, din, dout, st);
    if (e != hipSuccess) return e;
    if ((e = mark(GLACIER_HIP_PROBE_DOWN)) != hipSuccess) return e;
    if (s->tap_now) {
      e = hipMemcpyAsync(s->tap_x + (size_t)l * rows * D, s->x_res, (size_t)rows * D * 4,
                         hipMemcpyDeviceToDevice, st);
      if (e != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

// Final RMSNorm + LM head + (eligible) argmax for `rows` rows starting at x.
// Decode-
// sized row counts fuse the argmax into the head GEMV (each workgroup
// reduces its logits to one candidate per row) and finish with a
// one-block-per-row merge; longer row sets scan the logits afterwards.
hipError_t enqueue_head(glacier_hip_session *s, int rows, const float *x, bool elig, bool pre,
                        hipStream_t st) {
  glacier_hip_model *m = s->model;
  const auto &c = m->cfg;
  const long V = (long)c.vocab_size;
  const long W = (V + 63) / 64;
  const uint64_t *words = elig ? s->elig_words : nullptr;
  // The head converts its input with the separate kernel: in input mode
  // its ~1200 workgroups would each repeat the 3-digit quantisation of the
  // row, which measured slower than one extra launch.
  ProjIn in;
  in.x = x;
  in.norm_w = m->final_norm;
  ProjOut out;
  out.y = s->logits;
  if (rows <= gk::kGemvMaxRows) {
    out.arg_parts = (gk::ArgPartial *)s->arg_scratch;
    out.arg_words = words;
    out.arg_word_count = W;
    out.prehead = elig && pre;
    hipError_t e = run_proj(s, m->head, head_D(s), rows, gk::EPI_PLAIN, in, out, st);
    if (e != hipSuccess) return e;
    const int nparts = gk::gemv_argmax_parts((int)V, (int)c.dim, rows, head_D(s));
    return gk::launch_argmax_parts(out.arg_parts, nparts, V, rows, words, W, s->arg_result, st);
  }
  hipError_t e = run_proj(s, m->head, head_D(s), rows, gk::EPI_PLAIN, in, out, st);
  if (e != hipSuccess) return e;
  return gk::launch_argmax(s->logits, V, rows, words, W, s->arg_scratch, s->arg_counters,
                           s->arg_result, st);
}

// The full launch sequence of one decode step for `rows` lanes.
hipError_t enqueue_step(glacier_hip_session *s, int rows, bool head, bool elig, bool pre,
                        bool fused, hipStream_t st) {
  const RowPtrs rp{s->step_dev->tokens, s->step_dev->lane_of_row, s->step_dev->pos_of_row,
                   s->step_dev->ctx_len, s->step_dev->row0};
  hipError_t e = enqueue_layers(s, rows, rp, st, fused);
  if (e != hipSuccess || !head) return e;
  return enqueue_head(s, rows, s->x_res, elig, pre, st);
}

void destroy_session(glacier_hip_session *s) {
  if (s->prep.active && s->prep.cohort)  // a prepared wave's permit goes back to the bank
    (void)s->prep.cohort->lease.bank->abort_publication(s->prep.permit);
  for (Lane &ln : s->lanes)
    if (ln.lease) {  // the coordinator outlives the lane: every later call on it is refused
      ln.lease->lease.orphan();
      ln.lease->detach = nullptr;
      ln.lease = nullptr;
    }
  void *ptrs[] = {s->kv_pool, s->page_table, s->rope_cos, s->rope_sin, s->x_res, s->h, s->q,
                  s->attn, s->act, s->logits, s->act_q, s->act_meta, s->act_q2, s->act_meta2,
                  s->att_scratch, s->ss_parts, s->o_parts, s->o_counters, s->arg_scratch,
                  s->arg_counters,
                  s->arg_result,
                  s->elig_words, s->splitk_ws, s->splitk_counters,
                  s->step_dev, s->pf_dev, s->tap_x};
  for (void *p : ptrs) gh::dev_free(s->model->ctx, p);
  if (s->step_host) (void)hipHostFree(s->step_host);
  if (s->pf_host) (void)hipHostFree(s->pf_host);
  if (s->pt_host) (void)hipHostFree(s->pt_host);
  if (s->res_host) (void)hipHostFree(s->res_host);
  for (auto &g : s->graphs) {
    if (g.exec) (void)hipGraphExecDestroy(g.exec);
    if (g.graph) (void)hipGraphDestroy(g.graph);
  }
  for (hipEvent_t ev : s->probe_ev) (void)hipEventDestroy(ev);
  delete s;
}

void reset_lane(glacier_hip_session *s, Lane &ln, uint64_t seed) {
  ln.kv.start(s->pool);  // a new request: fresh cache instance, pages back to the pool
  ln.sampling_calls = 0;
  ln.prompt_len = 0;
  ln.first_pending = ln.chain_init = ln.retired = ln.chain_v3 = false;
  ln.v3_slot = -1;
  ln.first_token = 0;
  memset(ln.chain, 0, 32);
  // SplitMix64-seeded Xoshiro256 state (std.Random.DefaultPrng.init)
  uint64_t st = seed;
  for (int i = 0; i < 4; ++i) {
    st += 0x9e3779b97f4a7c15ull;
    uint64_t z = st;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    ln.rng[i] = z ^ (z >> 31);
  }
  ln.output.clear();
}

using gpk::RowTxn;

// Runs fn(lane, first, count) over the runs of consecutive rows of one lane.
template <class F>
int for_lane_runs(std::vector<RowTxn> &txns, F fn) {
  int rc = GLACIER_HIP_OK;
  for (size_t i = 0; i < txns.size();) {
    size_t j = i + 1;
    while (j < txns.size() && txns[j].lane == txns[i].lane) ++j;
    const int r = fn(txns[i].lane, &txns[i], j - i);
    if (r && !rc) rc = r;
    i = j;
  }
  return rc;
}

void abort_rows(glacier_hip_session *s, std::vector<RowTxn> &txns) {
  // abortRow per lane: installed pages lose their ownership generation, the
  // payloads stay with their logical pages and the consumed generations are
  // not handed back
  for_lane_runs(txns, [&](uint32_t lane, const RowTxn *t, size_t n) {
    if (s->lanes[lane].lease) s->lanes[lane].lease->lease.end_rows();
    return s->lanes[lane].kv.abort(t, n);
  });
  txns.clear();
}

// A lease refusing a step's new pages, in the session's status domain.
int lease_refusal(int rc) {
  return rc == GLACIER_HIP_LEASE_CAPACITY_EXCEEDED || rc == GLACIER_HIP_LEASE_INVALID_CLAIM ||
                 rc == GLACIER_HIP_LEASE_NODES_EXHAUSTED || rc == GLACIER_HIP_LEASE_CLAIM_OVERFLOW
             ? GLACIER_HIP_OUT_OF_MEMORY
             : GLACIER_HIP_INVALID_TRANSACTION;
}

void note_installs(glacier_hip_session *s, const std::vector<RowTxn> &txns) {
  for (const RowTxn &t : txns)
    if (t.installs) s->pt_host[(size_t)t.lane * s->max_pages + t.pos / 16] = t.page;
}

// beginRow (paged_kv_cache.zig:1006-1072) for every participating lane;
// nothing changes unless every lane can begin.
int begin_rows(glacier_hip_session *s, const uint32_t *lanes, uint32_t count,
               std::vector<RowTxn> &txns) {
  txns.clear();
  uint32_t need = 0;
  for (uint32_t i = 0; i < count; ++i) {
    const gpk::Cache &kv = s->lanes[lanes[i]].kv;
    if (kv.staged) return GLACIER_HIP_TRANSACTION_ACTIVE;
    if (kv.len + 1 > kv.max_seq) return GLACIER_HIP_CACHE_FULL;
    need += kv.pages_needed(1);
  }
  if (need > s->pool.free.size()) return GLACIER_HIP_CACHE_FULL;
  // lane by lane, as LeasedPagedKVCache.beginRowPlanned (leased_paged_kv_cache.zig:482-565):
  // a leased lane's new page is charged, the map takes it and the charge
  // settles before the next lane reserves, so lanes sharing one LeaseTree
  // never leave two allocation batches pending on it. A lane that cannot
  // begin aborts the rows begun before it (their pages stay charged with
  // their logical pages, as abortRowTxn leaves them).
  for (uint32_t i = 0; i < count; ++i) {
    glacier_hip_leased_kv *l = s->lanes[lanes[i]].lease;
    int rc = GLACIER_HIP_OK;
    if (l) {
      const int lrc = l->lease.reserve_rows(1);
      if (lrc) rc = lease_refusal(lrc);
    }
    if (!rc) {
      rc = s->lanes[lanes[i]].kv.begin(lanes[i], 1, s->pool, txns);
      if (l) l->lease.settle_rows(rc == GLACIER_HIP_OK);
    }
    if (rc) {
      note_installs(s, txns);  // installed pages stay with their logical pages
      abort_rows(s, txns);
      return rc;
    }
  }
  note_installs(s, txns);
  return GLACIER_HIP_OK;
}

// beginRow for `n` consecutive rows of one lane (a prompt chunk): row i's
// transaction starts from row i - 1's staged root, exactly as n sequential
// per-token transactions would (generate.zig:5080-5118 commits per token).
int begin_chunk(glacier_hip_session *s, uint32_t lane, uint32_t n, std::vector<RowTxn> &txns) {
  txns.clear();
  glacier_hip_leased_kv *l = s->lanes[lane].lease;
  if (l)
    if (int rc = l->lease.reserve_rows(n)) return lease_refusal(rc);
  const int rc = s->lanes[lane].kv.begin(lane, n, s->pool, txns);
  if (l) l->lease.settle_rows(rc == GLACIER_HIP_OK);
  if (rc) return rc;
  note_installs(s, txns);
  return GLACIER_HIP_OK;
}

int commit_rows(glacier_hip_session *s, std::vector<RowTxn> &txns) {
  const int rc = for_lane_runs(txns, [&](uint32_t lane, const RowTxn *t, size_t n) {
    if (s->lanes[lane].lease) s->lanes[lane].lease->lease.end_rows();
    return s->lanes[lane].kv.commit(t, n);
  });
  txns.clear();
  return rc;
}

// Copies the page-table entries installed by `txns` from the pinned host
// mirror (runs of consecutive logical pages of one lane go in one copy). The
// mirror is only rewritten after the step's stream synchronisation.
hipError_t upload_page_entries(glacier_hip_session *s, const std::vector<RowTxn> &txns,
                               hipStream_t st) {
  size_t i = 0;
  while (i < txns.size()) {
    if (!txns[i].installs) {
      ++i;
      continue;
    }
    const uint32_t lane = txns[i].lane;
    const uint64_t p0 = txns[i].pos / 16;
    uint64_t p1 = p0 + 1;
    size_t j = i + 1;
    for (; j < txns.size() && txns[j].lane == lane; ++j)
      if (txns[j].installs) {
        if (txns[j].pos / 16 != p1) break;
        ++p1;
      }
    const size_t off = (size_t)lane * s->max_pages + p0;
    hipError_t e = hipMemcpyAsync(s->page_table + off, s->pt_host + off, (p1 - p0) * 4,
                                  hipMemcpyHostToDevice, st);
    if (e != hipSuccess) return e;
    i = j;
  }
  return hipSuccess;
}

// The kernel launches of a captured step in dependency order (a chain for a
// one-stream capture); false if the graph holds any other kind of node.
bool record_launches(hipGraph_t g, std::vector<hipKernelNodeParams> &out) {
  size_t n = 0;
  if (hipGraphGetNodes(g, nullptr, &n) != hipSuccess || n == 0) return false;
  std::vector<hipGraphNode_t> nodes(n);
  if (hipGraphGetNodes(g, nodes.data(), &n) != hipSuccess) return false;
  std::map<hipGraphNode_t, size_t> indeg;
  std::vector<hipGraphNode_t> ready;
  for (hipGraphNode_t v : nodes) {
    hipGraphNodeType t;
    size_t d = 0;
    if (hipGraphNodeGetType(v, &t) != hipSuccess || t != hipGraphNodeTypeKernel ||
        hipGraphNodeGetDependencies(v, nullptr, &d) != hipSuccess)
      return false;
    indeg[v] = d;
    if (d == 0) ready.push_back(v);
  }
  out.clear();
  while (!ready.empty()) {
    hipGraphNode_t v = ready.front();
    ready.erase(ready.begin());
    hipKernelNodeParams p{};
    if (hipGraphKernelNodeGetParams(v, &p) != hipSuccess) return false;
    out.push_back(p);
    size_t m = 0;
    if (hipGraphNodeGetDependentNodes(v, nullptr, &m) != hipSuccess) return false;
    std::vector<hipGraphNode_t> next(m);
    if (m && hipGraphNodeGetDependentNodes(v, next.data(), &m) != hipSuccess) return false;
    for (hipGraphNode_t w : next)
      if (--indeg[w] == 0) ready.push_back(w);
  }
  return out.size() == n;
}

// Execute one step for `count` rows; on success results are in res_host.
int run_step(glacier_hip_session *s, const uint32_t *lanes, const uint32_t *tokens,
             uint32_t count, bool head, const uint64_t *elig_host, float *logits_host,
             std::vector<RowTxn> &txns) {
  glacier_hip_context *ctx = s->model->ctx;
  const auto &c = s->model->cfg;
  hipStream_t st = ctx->stream;
  // prehead never computes the logits of skipped rows
  // (generate.zig:423-426: full-vocabulary logits never exist)
  if (logits_host && elig_host && s->head_domain == GLACIER_HIP_HEAD_DOMAIN_PREHEAD)
    return GLACIER_HIP_INVALID_ARGUMENT;
  int rc = begin_rows(s, lanes, count, txns);
  if (rc) return rc;
  for (uint32_t i = 0; i < count; ++i) {
    s->step_host->tokens[i] = (int32_t)tokens[i];
    s->step_host->lane_of_row[i] = (int32_t)lanes[i];
    s->step_host->pos_of_row[i] = (int32_t)txns[i].pos;
    s->step_host->ctx_len[i] = (int32_t)txns[i].pos + 1;
  }
  {
    int32_t *r0 = s->step_host->row0;
    r0[0] = (int32_t)lanes[0];
    r0[1] = (int32_t)txns[0].pos + 1;
    r0[2] = (int32_t)txns[0].pos;
    r0[3] = 0;
    const uint32_t np = std::min<uint32_t>(kRow0Pages, s->max_pages);
    const int32_t *pr = s->pt_host + (size_t)lanes[0] * s->max_pages;
    for (uint32_t k = 0; k < np; ++k) r0[4 + k] = pr[k];
  }
  auto fail = [&](hipError_t e, const char *what) {
    (void)hipStreamSynchronize(st);
    abort_rows(s, txns);
    return hip_fail(ctx, e, what);
  };
  hipError_t e = hipMemcpyAsync(s->step_dev, s->step_host, sizeof(StepInputs),
                                hipMemcpyHostToDevice, st);
  if (e != hipSuccess) return fail(e, "step inputs");
  e = upload_page_entries(s, txns, st);
  if (e != hipSuccess) return fail(e, "page table");
  const uint64_t W = (c.vocab_size + 63) / 64;
  if (elig_host) {
    e = hipMemcpyAsync(s->elig_words, elig_host, (size_t)count * W * 8, hipMemcpyHostToDevice, st);
    if (e != hipSuccess) return fail(e, "eligibility words");
  }
  const bool elig = elig_host != nullptr;
  const bool pre = elig && s->head_domain == GLACIER_HIP_HEAD_DOMAIN_PREHEAD;
  const bool fused = count == 1 && txns[0].pos + 1 <= kFusedMaxCtx && attn_o_usable(s);
  s->tap_now = s->tap_x != nullptr;
  s->probe_now = s->probe_kind >= 0;
  s->probe_used = 0;
  if (s->tap_now || s->probe_now) {  // a traced or probed step launches directly
    if (s->tap_now) s->tap_rows = count;
    e = enqueue_step(s, (int)count, head, elig, pre, fused, st);
    s->tap_now = s->probe_now = false;
    if (e != hipSuccess) return fail(e, "enqueue traced step");
  } else if (s->opt.use_graph) {
    glacier_hip_session::GraphEntry *plan = nullptr;
    for (auto &g : s->graphs)
      if (g.rows == count && g.head == head && g.elig == elig && g.pre == pre && g.fused == fused)
        plan = &g;
    if (!plan) {
      glacier_hip_session::GraphEntry g{count, head, elig, pre, fused, nullptr, nullptr, {}};
      e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
      if (e != hipSuccess) return fail(e, "begin capture");
      hipError_t e2 = enqueue_step(s, (int)count, head, elig, pre, fused, st);
      e = hipStreamEndCapture(st, &g.graph);
      if (e2 != hipSuccess || e != hipSuccess) {
        if (g.graph) (void)hipGraphDestroy(g.graph);
        return fail(e2 != hipSuccess ? e2 : e, e2 != hipSuccess ? "capture step" : "end capture");
      }
      // replay the recorded launches (use_graph 1) unless the step holds a
      // node that is not a kernel launch; else the instantiated graph
      if (s->opt.use_graph != 1 || !record_launches(g.graph, g.launches)) {
        g.launches.clear();
        e = hipGraphInstantiate(&g.exec, g.graph, nullptr, nullptr, 0);
        if (e != hipSuccess) {
          (void)hipGraphDestroy(g.graph);
          return fail(e, "graph instantiate");
        }
      }
      s->graphs.push_back(std::move(g));
      plan = &s->graphs.back();
    }
    if (plan->exec) {
      e = hipGraphLaunch(plan->exec, st);
      if (e != hipSuccess) return fail(e, "graph launch");
    } else {
      for (const hipKernelNodeParams &p : plan->launches) {
        e = hipLaunchKernel(p.func, p.gridDim, p.blockDim, p.kernelParams, p.sharedMemBytes, st);
        if (e != hipSuccess) return fail(e, "plan launch");
      }
    }
  } else {
    e = enqueue_step(s, (int)count, head, elig, pre, fused, st);
    if (e != hipSuccess) return fail(e, "enqueue step");
  }
  s->last_rows = count;
  s->last_fused = fused;
  if (head) {
    e = hipMemcpyAsync(s->res_host, s->arg_result, count * sizeof(gk::ArgmaxResult),
                       hipMemcpyDeviceToHost, st);
    if (e != hipSuccess) return fail(e, "result copy");
    if (logits_host) {
      e = hipMemcpyAsync(logits_host, s->logits, (size_t)count * c.vocab_size * 4,
                         hipMemcpyDeviceToHost, st);
      if (e != hipSuccess) return fail(e, "logits copy");
    }
  }
  e = hipStreamSynchronize(st);
  if (e != hipSuccess) return fail(e, "step sync");
  for (uint32_t i = 0; i + 1 < s->probe_used; i += 2) {
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, s->probe_ev[i], s->probe_ev[i + 1]) == hipSuccess) {
      s->probe_ms += ms;
      s->probe_count++;
    }
  }
  s->probe_used = 0;
  if (s->inject_failure) {
    abort_rows(s, txns);
    return GLACIER_HIP_DEVICE_ERROR;
  }
  if (head)
    for (uint32_t i = 0; i < count; ++i)
      if (s->res_host[i].status != 0) {
        const int st_code = s->res_host[i].status;
        abort_rows(s, txns);
        return st_code;
      }
  return GLACIER_HIP_OK;
}

// One prompt chunk of `n` rows of one lane: all layers over the rows at
// once; with `head`, the last row's final norm, LM head and argmax.
int run_prefill_chunk(glacier_hip_session *s, uint32_t lane, const uint32_t *tokens, uint32_t n,
                      bool head, float *logits_host, std::vector<RowTxn> &txns) {
  glacier_hip_context *ctx = s->model->ctx;
  const auto &c = s->model->cfg;
  hipStream_t st = ctx->stream;
  int rc = begin_chunk(s, lane, n, txns);
  if (rc) return rc;
  const uint32_t C = s->prefill_chunk;
  int32_t *tok = s->pf_host, *lor = s->pf_host + C, *por = s->pf_host + 2 * C,
          *ctl = s->pf_host + 3 * C;
  for (uint32_t i = 0; i < n; ++i) {
    tok[i] = (int32_t)tokens[i];
    lor[i] = (int32_t)lane;
    por[i] = (int32_t)txns[i].pos;
    ctl[i] = (int32_t)txns[i].pos + 1;
  }
  auto fail = [&](hipError_t e, const char *what) {
    (void)hipStreamSynchronize(st);
    abort_rows(s, txns);
    return hip_fail(ctx, e, what);
  };
  hipError_t e = hipSuccess;
  for (int k = 0; k < 4 && e == hipSuccess; ++k)
    e = hipMemcpyAsync(s->pf_dev + (size_t)k * C, s->pf_host + (size_t)k * C, (size_t)n * 4,
                       hipMemcpyHostToDevice, st);
  if (e != hipSuccess) return fail(e, "prefill inputs");
  e = upload_page_entries(s, txns, st);
  if (e != hipSuccess) return fail(e, "page table");
  RowPtrs rp{s->pf_dev, s->pf_dev + C, s->pf_dev + 2 * C, s->pf_dev + 3 * C};
  bool consecutive = true;
  for (uint32_t i = 1; i < n; ++i) consecutive = consecutive && por[i] == por[0] + (int32_t)i;
  if (consecutive) {
    rp.chunk_lane = (int)lane;
    rp.chunk_pos0 = por[0];
  }
  e = enqueue_layers(s, (int)n, rp, st);
  if (e != hipSuccess) return fail(e, "prefill layers");
  if (head) {
    e = enqueue_head(s, 1, s->x_res + (size_t)(n - 1) * c.dim, false, false, st);
    if (e != hipSuccess) return fail(e, "prefill head");
    e = hipMemcpyAsync(s->res_host, s->arg_result, sizeof(gk::ArgmaxResult),
                       hipMemcpyDeviceToHost, st);
    if (e != hipSuccess) return fail(e, "result copy");
    if (logits_host) {
      e = hipMemcpyAsync(logits_host, s->logits, (size_t)c.vocab_size * 4, hipMemcpyDeviceToHost,
                         st);
      if (e != hipSuccess) return fail(e, "logits copy");
    }
  }
  e = hipStreamSynchronize(st);
  if (e != hipSuccess) return fail(e, "prefill sync");
  if (s->inject_failure) {
    abort_rows(s, txns);
    return GLACIER_HIP_DEVICE_ERROR;
  }
  if (head && s->res_host[0].status != 0) {
    const int st_code = s->res_host[0].status;
    abort_rows(s, txns);
    return st_code;
  }
  return GLACIER_HIP_OK;
}

// logicalKvPrefixSha256 (generate.zig:3150-3172; hashLogicalPrefix
// paged_kv_cache.zig:1532-1555) over the committed rows, K/V values widened to
// f32 bit patterns: each committed page is copied once, then hashed in the
// canonical layer / K-then-V / position order.
// `extra` = 1: the committed rows plus the lane's one staged row
// (logicalKvTxnSha256 paged_kv_cache.zig, the canonical digest after a row).
int logical_kv_sha256(glacier_hip_session *s, uint32_t lane, uint8_t out[32], uint64_t extra = 0) {
  const auto &c = s->model->cfg;
  const Lane &ln = s->lanes[lane];
  glacier_hip_context *ctx = s->model->ctx;
  const size_t kvd = (size_t)c.num_kv_heads * c.head_dim, L = c.num_layers;
  const size_t elem = s->opt.kv_dtype == GLACIER_HIP_F16 ? 2 : 4;
  const size_t page_elems = L * 2 * 16 * kvd;
  const uint64_t len = ln.kv.len + extra, pages = (len + 15) / 16;
  std::vector<uint8_t> raw(pages * page_elems * elem);
  for (uint64_t p = 0; p < pages; ++p) {
    const int32_t phys = ln.kv.page_of[p];
    if (phys < 0) return GLACIER_HIP_INVALID_TRANSACTION;
    GH_CHECK(ctx, hipMemcpy(raw.data() + p * page_elems * elem,
                            (char *)s->kv_pool + (size_t)phys * page_elems * elem,
                            page_elems * elem, hipMemcpyDeviceToHost));
  }
  gh::Sha256 h;
  h.update("glacier-logical-kv-state-v1\0", 28);
  h.u64(L);
  h.u64(kvd);
  h.u64(len);
  for (size_t l = 0; l < L; ++l)
    for (int v = 0; v < 2; ++v)
      for (uint64_t pos = 0; pos < len; ++pos) {
        const uint8_t *row = raw.data() +
                             ((((pos / 16) * L + l) * 2 + v) * 16 + pos % 16) * kvd * elem;
        for (size_t i = 0; i < kvd; ++i) {
          uint32_t b;
          if (elem == 4) {
            memcpy(&b, row + 4 * i, 4);
          } else {
            uint16_t hv;
            memcpy(&hv, row + 2 * i, 2);
            const float f = gh::f16_to_f32(hv);
            memcpy(&b, &f, 4);
          }
          h.u32(b);
        }
      }
  h.final(out);
  return GLACIER_HIP_OK;
}

// logicalRowTxnSha256 (paged_kv_cache.zig:1366-1384) of each staged row: the
// row's K and V of every layer (one strided copy), widened to f32 bits.
int row_payload_sha256(glacier_hip_session *s, const std::vector<RowTxn> &txns,
                       std::vector<std::array<uint8_t, 32>> &out) {
  const auto &c = s->model->cfg;
  glacier_hip_context *ctx = s->model->ctx;
  const size_t kvd = (size_t)c.num_kv_heads * c.head_dim, L = c.num_layers;
  const size_t elem = s->opt.kv_dtype == GLACIER_HIP_F16 ? 2 : 4;
  std::vector<uint8_t> raw(2 * L * kvd * elem);
  out.resize(txns.size());
  for (size_t i = 0; i < txns.size(); ++i) {
    const RowTxn &t = txns[i];
    // rows (layer l, K/V v) of the page sit 16 * kvd elements apart
    const size_t off = ((size_t)t.page * L * 2 * 16 + t.pos % 16) * kvd * elem;
    GH_CHECK(ctx, hipMemcpy2D(raw.data(), kvd * elem, (char *)s->kv_pool + off, 16 * kvd * elem,
                              kvd * elem, 2 * L, hipMemcpyDeviceToHost));
    gh::Sha256 h;
    h.update("glacier-paged-kv-row-v1", sizeof("glacier-paged-kv-row-v1"));
    h.u64(L);
    h.u64(kvd);
    h.u64(t.mark.base_len);
    for (size_t r = 0; r < 2 * L * kvd; ++r) {
      uint32_t b;
      if (elem == 4) {
        memcpy(&b, &raw[4 * r], 4);
      } else {
        uint16_t hv;
        memcpy(&hv, &raw[2 * r], 2);
        const float f = gh::f16_to_f32(hv);
        memcpy(&b, &f, 4);
      }
      h.u32(b);
    }
    h.final(out[i].data());
  }
  return GLACIER_HIP_OK;
}

// capacityLedger().allocation_capacity_bytes of a lane's cache
// (paged_kv_cache.zig capacity ledger: f32 page payloads + 16-byte entries).
uint64_t lane_capacity_bytes(const glacier_hip_session *s) {
  const auto &c = s->model->cfg;
  const uint64_t pages = (s->opt.max_positions + 15) / 16;
  const uint64_t payload = (uint64_t)c.num_layers * 2 * 16 * c.num_kv_heads * c.head_dim * 4;
  return pages * payload + pages * 16;
}

void copy_root(const glacier_hip_page_map_root_t &r, glacier_hip_root_transition_v1_t &t,
               bool before) {
  if (before) {
    t.root_before_generation = r.generation;
    t.root_before_len = r.committed_len;
    t.root_before_pages = r.committed_pages;
    memcpy(t.root_before_ownership_sha256, r.ownership_sha256, 32);
  } else {
    t.root_after_generation = r.generation;
    t.root_after_len = r.committed_len;
    t.root_after_pages = r.committed_pages;
    memcpy(t.root_after_ownership_sha256, r.ownership_sha256, 32);
  }
}

}  // namespace

// Creates the session, or with `quote` set only adds up the device bytes its
// allocations would take (requested and granularity-charged) and creates
// nothing: the quote and the allocation come from the same list.
static glacier_hip_session *session_create_impl(glacier_hip_model *m,
                                                const glacier_hip_session_options_t *opts,
                                                uint64_t *quote) {
  if (!m || !opts) return nullptr;
  glacier_hip_context *ctx = m->ctx;
  for (bool b : m->layer_set)
    if (!b) {
      ctx->last_error = "model layers not set";
      return nullptr;
    }
  if (!m->globals_set) {
    ctx->last_error = "model globals not set";
    return nullptr;
  }
  const auto &c = m->cfg;
  if (opts->max_lanes == 0 || opts->max_lanes > 32 || opts->max_positions == 0 ||
      opts->prefill_chunk < 0 || opts->prefill_chunk > 8192 ||
      (opts->kv_dtype != GLACIER_HIP_F32 && opts->kv_dtype != GLACIER_HIP_F16)) {
    ctx->last_error = "session options invalid";
    return nullptr;
  }
  auto *s = new glacier_hip_session();
  s->model = m;
  s->opt = *opts;
  s->max_pages = (opts->max_positions + 15) / 16;
  s->total_pages = opts->total_pages ? opts->total_pages : opts->max_lanes * s->max_pages;
  s->lanes.resize(opts->max_lanes);
  s->pool.init(s->total_pages);
  for (auto &ln : s->lanes)
    ln.kv.init(c.num_layers, (uint64_t)c.num_kv_heads * c.head_dim, opts->max_positions);
  for (auto &ln : s->lanes)
    ln.kv.page_payload_bytes = (uint64_t)c.num_layers * 2 * 16 * c.num_kv_heads * c.head_dim *
                               (opts->kv_dtype == GLACIER_HIP_F16 ? 2 : 4);
  s->prefill_chunk = opts->prefill_chunk ? (uint32_t)opts->prefill_chunk
                                         : std::min<uint32_t>(opts->max_positions, 2048);
  s->rows_cap = std::max(opts->max_lanes, s->prefill_chunk);
  const uint32_t L = opts->max_lanes;  // lanes: page tables, logits, masks
  const uint32_t M = s->rows_cap;      // activation rows: decode lanes or a prompt chunk
  const size_t kvd = (size_t)c.num_kv_heads * c.head_dim;
  const size_t elem = opts->kv_dtype == GLACIER_HIP_F16 ? 2 : 4;
  const size_t page_bytes = (size_t)c.num_layers * 2 * 16 * kvd * elem;
  const size_t Kmax = std::max(c.dim, c.hidden_dim);
  const size_t Gmax = Kmax / 32;
  const size_t W = (c.vocab_size + 63) / 64;
  const size_t att = gk::attention_scratch_floats((int)M, (int)c.num_heads, (int)c.num_kv_heads,
                                                  (int)c.head_dim, (int)opts->max_positions);
  bool ok = true;
  auto A = [&](void **p, size_t bytes) {
    if (quote) {
      quote[0] += bytes;
      quote[1] += gh::charged_bytes(bytes);
    } else if (ok && gh::dev_malloc(ctx, p, bytes) != hipSuccess) {
      ok = false;
    }
  };
  A(&s->kv_pool, page_bytes * s->total_pages);
  A((void **)&s->page_table, (size_t)L * s->max_pages * 4);
  A((void **)&s->rope_cos, (size_t)opts->max_positions * c.head_dim / 2 * 4);
  A((void **)&s->rope_sin, (size_t)opts->max_positions * c.head_dim / 2 * 4);
  A((void **)&s->x_res, (size_t)M * c.dim * 4);
  A((void **)&s->h, (size_t)M * c.dim * 4);
  A((void **)&s->q, (size_t)M * c.dim * 4);
  A((void **)&s->attn, (size_t)M * c.dim * 4);
  A((void **)&s->act, (size_t)M * c.hidden_dim * 4);
  A((void **)&s->logits, (size_t)L * c.vocab_size * 4);
  A((void **)&s->act_q, Gmax * 3 * M * 32);
  A((void **)&s->act_meta, Gmax * M * sizeof(gk::ActMeta));
  // the gate/up epilogue emits planes for every GEMV launch (up to
  // kGemvMaxRows rows) and attention the O projection's for every step of
  // up to 32 rows (decode lanes, or a prompt chunk that short); in GEMM
  // steps of any row count O's finishing pass emits gate/up's planes
  // (model width) here, so that gate/up can emit down's into act_q, which
  // none of its tiles read
  s->planes2_rows = std::min<uint32_t>(M, 32);
  // act_q2 also holds the O projection's planes, emitted by attention
  const size_t G2 = std::max<size_t>(c.hidden_dim, (size_t)c.num_heads * c.head_dim) / 32;
  const size_t q2_groups_rows = std::max(G2 * s->planes2_rows, (size_t)(c.dim / 32) * M);
  A((void **)&s->act_q2, q2_groups_rows * 3 * 32);
  A((void **)&s->act_meta2, q2_groups_rows * sizeof(gk::ActMeta));
  A((void **)&s->att_scratch, std::max<size_t>(att, 1) * 4);
  A((void **)&s->ss_parts, (size_t)32 * 1024 * sizeof(float));
  A((void **)&s->o_parts, (size_t)c.num_kv_heads * c.dim * sizeof(float));
  A((void **)&s->o_counters, (size_t)gk::attn_o_groups((int)c.dim) * sizeof(unsigned));
  size_t arg_bytes = gk::argmax_scratch_bytes((int)L, (long)c.vocab_size);
  for (uint32_t r = 1; r <= std::min<uint32_t>(L, gk::kGemvMaxRows); ++r)
    arg_bytes = std::max(arg_bytes, (size_t)r * sizeof(gk::ArgPartial) *
                                        std::max(0, gk::gemv_argmax_parts((int)c.vocab_size,
                                                                          (int)c.dim, (int)r,
                                                                          head_D(s))));
  A(&s->arg_scratch, arg_bytes);
  // GEMM split-K partial sums: the most any projection asks for at the row
  // counts past the GEMV (decode lanes up to 32, a full prompt chunk),
  // capped at 64 MiB (a smaller workspace only lowers a split)
  {
    size_t need = 0;
    const LayerDev &L0 = m->layers[0];  // every layer has the same shapes
    const glacier_hip_int4_weight *ws[] = {L0.qkv, L0.o, L0.gu, L0.down, m->head};
    for (uint32_t rows : {(uint32_t)gk::kGemvMaxRows + 1, 24u, 32u, M})
      if (rows > (uint32_t)gk::kGemvMaxRows && rows <= M)
        for (const auto *w : ws)
          for (int D : {1, 3}) {
            need = std::max(need, gk::gemm_splitk_floats((int)w->out_f, (int)rows, (int)w->in_f, D));
            // plane emission from the finishing pass needs the partial sums
            // even without a K split (decode lanes up to 32)
            if (rows <= 32) need = std::max(need, (size_t)rows * w->out_f);
          }
    s->splitk_floats = std::min<size_t>(need, 16u << 20);
    if (s->splitk_floats) A((void **)&s->splitk_ws, s->splitk_floats * sizeof(float));
    A((void **)&s->splitk_counters, (size_t)kSplitkCounters * sizeof(unsigned));
  }
  A((void **)&s->arg_counters, (size_t)L * 4);
  A((void **)&s->arg_result, (size_t)L * sizeof(gk::ArgmaxResult));
  A((void **)&s->elig_words, (size_t)L * W * 8);
  A((void **)&s->step_dev, sizeof(StepInputs));
  A((void **)&s->pf_dev, (size_t)4 * s->prefill_chunk * 4);
  if (quote) {  // host-pinned staging is not device memory
    delete s;
    return nullptr;
  }
  auto H = [&](void **p, size_t bytes) {
    if (ok && hipHostMalloc(p, bytes) != hipSuccess) ok = false;
  };
  H((void **)&s->step_host, sizeof(StepInputs));
  H((void **)&s->pf_host, (size_t)4 * s->prefill_chunk * 4);
  H((void **)&s->pt_host, (size_t)L * s->max_pages * 4);
  H((void **)&s->res_host, L * sizeof(gk::ArgmaxResult));
  if (ok) {
    ok = hipMemset(s->arg_counters, 0, (size_t)L * 4) == hipSuccess &&
         hipMemset(s->o_counters, 0,
                   (size_t)gk::attn_o_groups((int)c.dim) * sizeof(unsigned)) == hipSuccess &&
         hipMemset(s->splitk_counters, 0, (size_t)kSplitkCounters * sizeof(unsigned)) ==
             hipSuccess &&
         hipMemset(s->kv_pool, 0, page_bytes * s->total_pages) == hipSuccess;
    memset(s->pt_host, 0, (size_t)L * s->max_pages * 4);
    ok = ok && hipMemcpy(s->page_table, s->pt_host, (size_t)L * s->max_pages * 4,
                         hipMemcpyHostToDevice) == hipSuccess;
    // RopeTable.init (generate.zig:790-806), f32 libm on the host
    const size_t half = c.head_dim / 2;
    std::vector<float> cs(opts->max_positions * half), sn(opts->max_positions * half);
    for (size_t pos = 0; pos < opts->max_positions; ++pos)
      for (size_t pair = 0; pair < half; ++pair) {
        const float exponent = (float)(2 * pair) / (float)c.head_dim;
        const float freq = 1.0f / powf(c.rope_theta, exponent);
        const float angle = (float)pos * freq;
        cs[pos * half + pair] = cosf(angle);
        sn[pos * half + pair] = sinf(angle);
      }
    ok = ok && hipMemcpy(s->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(s->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice) == hipSuccess;
  }
  if (!ok) {
    (void)hipGetLastError();
    ctx->last_error = "session allocation failed";
    destroy_session(s);
    return nullptr;
  }
  return s;
}

extern "C" {

glacier_hip_session *glacier_hip_session_create(glacier_hip_model *m,
                                                const glacier_hip_session_options_t *opts) {
  return session_create_impl(m, opts, nullptr);
}

int glacier_hip_session_quote(glacier_hip_model *m, const glacier_hip_session_options_t *opts,
                              glacier_hip_allocation_quote_t *out) {
  if (!m || !opts || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  uint64_t q[2] = {0, 0};
  (void)session_create_impl(m, opts, q);
  if (q[0] == 0) return GLACIER_HIP_INVALID_ARGUMENT;  // options the session would refuse
  out->requested_bytes = q[0];
  out->charged_bytes = q[1];
  out->context_epoch = m->ctx->epoch;
  return GLACIER_HIP_OK;
}

void glacier_hip_session_destroy(glacier_hip_session *s) {
  if (!s) return;
  (void)hipStreamSynchronize(s->model->ctx->stream);
  destroy_session(s);
}

int glacier_hip_session_lane_begin(glacier_hip_session *s, uint32_t lane, uint64_t seed) {
  if (!s) return GLACIER_HIP_INVALID_HANDLE;
  if (lane >= s->lanes.size()) return GLACIER_HIP_INVALID_ARGUMENT;
  GH_SUBMISSION(s->model->ctx);
  if (s->prep.active) return GLACIER_HIP_TRANSACTION_ACTIVE;
  if (s->lanes[lane].lease) return GLACIER_HIP_INVALID_TRANSACTION;  // one request per lease
  reset_lane(s, s->lanes[lane], seed);
  return GLACIER_HIP_OK;
}

int glacier_hip_session_inject_failure(glacier_hip_session *s, int enable) {
  if (!s) return GLACIER_HIP_INVALID_HANDLE;
  s->inject_failure = enable != 0;
  return GLACIER_HIP_OK;
}

int glacier_hip_session_trace_layers(glacier_hip_session *s, int enable) {
  if (!s) return GLACIER_HIP_INVALID_HANDLE;
  GH_SUBMISSION(s->model->ctx);
  glacier_hip_context *ctx = s->model->ctx;
  if (enable && !s->tap_x) {
    const auto &c = s->model->cfg;
    const size_t n = (size_t)c.num_layers * s->lanes.size() * c.dim;
    GH_CHECK(ctx, gh::dev_malloc(ctx, (void **)&s->tap_x, n * 4));
  } else if (!enable && s->tap_x) {
    gh::dev_free(ctx, s->tap_x);
    s->tap_x = nullptr;
  }
  s->tap_rows = 0;
  return GLACIER_HIP_OK;
}

int glacier_hip_session_layer_trace(glacier_hip_session *s, float *out_host, uint32_t *rows_out) {
  if (!s || !out_host || !rows_out) return GLACIER_HIP_INVALID_ARGUMENT;
  GH_SUBMISSION(s->model->ctx);
  if (!s->tap_x || !s->tap_rows) return GLACIER_HIP_INVALID_TRANSACTION;
  const auto &c = s->model->cfg;
  GH_CHECK(s->model->ctx, hipMemcpy(out_host, s->tap_x, (size_t)c.num_layers * s->tap_rows * c.dim * 4,
                                    hipMemcpyDeviceToHost));
  *rows_out = s->tap_rows;
  return GLACIER_HIP_OK;
}

int glacier_hip_session_probe_kernel(glacier_hip_session *s, int kind) {
  if (!s) return GLACIER_HIP_INVALID_HANDLE;
  if (kind < -1 || kind > GLACIER_HIP_PROBE_DOWN) return GLACIER_HIP_INVALID_ARGUMENT;
  GH_SUBMISSION(s->model->ctx);
  glacier_hip_context *ctx = s->model->ctx;
  const size_t need = 2 * (size_t)s->model->cfg.num_layers;
  while (kind >= 0 && s->probe_ev.size() < need) {
    hipEvent_t ev;
    GH_CHECK(ctx, hipEventCreate(&ev));
    s->probe_ev.push_back(ev);
  }
  s->probe_kind = kind;
  s->probe_ms = 0.0;
  s->probe_count = 0;
  return GLACIER_HIP_OK;
}

int glacier_hip_session_probe_replay(glacier_hip_session *s, int kind, uint32_t reps, double *avg_us) {
  if (!s || !avg_us || reps == 0) return GLACIER_HIP_INVALID_ARGUMENT;
  // only launches whose outputs are step scratch (the next step rewrites them)
  if (kind != GLACIER_HIP_PROBE_GATE_UP && kind != GLACIER_HIP_PROBE_DOWN)
    return GLACIER_HIP_INVALID_ARGUMENT;
  GH_SUBMISSION(s->model->ctx);
  if (s->prep.active) return GLACIER_HIP_TRANSACTION_ACTIVE;
  if (s->last_rows == 0) return GLACIER_HIP_INVALID_TRANSACTION;  // no decode step yet
  glacier_hip_context *ctx = s->model->ctx;
  hipStream_t st = ctx->stream;
  hipEvent_t ev[2] = {nullptr, nullptr};
  GH_CHECK(ctx, hipEventCreate(&ev[0]));
  hipError_t e = hipEventCreate(&ev[1]);
  const RowPtrs rp{s->step_dev->tokens, s->step_dev->lane_of_row, s->step_dev->pos_of_row,
                   s->step_dev->ctx_len, s->step_dev->row0};
  s->probe_only = kind;
  if (e == hipSuccess) e = hipEventRecord(ev[0], st);
  for (uint32_t r = 0; r < reps && e == hipSuccess; ++r)
    e = enqueue_layers(s, (int)s->last_rows, rp, st, s->last_fused);
  if (e == hipSuccess) e = hipEventRecord(ev[1], st);
  s->probe_only = -1;
  const hipError_t es = hipStreamSynchronize(st);
  float ms = 0.0f;
  if (e == hipSuccess) e = es;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev[0], ev[1]);
  (void)hipEventDestroy(ev[0]);
  if (ev[1]) (void)hipEventDestroy(ev[1]);
  if (e != hipSuccess) return hip_fail(ctx, e, "probe replay");
  *avg_us = ms * 1000.0 / ((double)reps * s->model->cfg.num_layers);
  return GLACIER_HIP_OK;
}

int glacier_hip_session_probe_read(glacier_hip_session *s, double *total_us, uint64_t *launches) {
  if (!s || !total_us || !launches) return GLACIER_HIP_INVALID_ARGUMENT;
  *total_us = s->probe_ms * 1000.0;
  *launches = s->probe_count;
  return GLACIER_HIP_OK;
}

static int prefill_impl(glacier_hip_session *s, uint32_t lane, const uint32_t *tokens, uint32_t n,
                        uint32_t *first_token, float *logits_host, bool staged) {
  if (!s || !tokens || !first_token) return GLACIER_HIP_INVALID_ARGUMENT;
  if (lane >= s->lanes.size() || !s->lanes[lane].kv.active) return GLACIER_HIP_INVALID_ARGUMENT;
  const auto &c = s->model->cfg;
  Lane &ln = s->lanes[lane];
  if (n == 0) return GLACIER_HIP_SHAPE_MISMATCH;
  for (uint32_t i = 0; i < n; ++i)
    if (tokens[i] >= c.vocab_size) return GLACIER_HIP_SHAPE_MISMATCH;
  if (ln.kv.len + n > s->opt.max_positions) return GLACIER_HIP_CACHE_FULL;
  GH_SUBMISSION(s->model->ctx);
  if (s->prep.active) return GLACIER_HIP_TRANSACTION_ACTIVE;
  if (ln.first_pending || ln.retired || !ln.output.empty()) return GLACIER_HIP_INVALID_TRANSACTION;
  std::vector<RowTxn> txns;
  for (uint32_t done = 0; done < n;) {
    const uint32_t rows = std::min(n - done, s->prefill_chunk);
    const bool last = done + rows == n;
    int rc = run_prefill_chunk(s, lane, tokens + done, rows, last, last ? logits_host : nullptr,
                               txns);
    if (rc) return rc;  // rows of earlier chunks stay committed (cache.commit per token)
    if ((rc = commit_rows(s, txns))) return rc;  // staged under the lock: cannot fail
    done += rows;
  }
  *first_token = (uint32_t)s->res_host[0].index;
  ln.prompt_len = ln.kv.len;
  if (staged) {  // held for the first publication wave
    ln.first_pending = true;
    ln.first_token = *first_token;
  } else {
    ln.sampling_calls += 1;
    ln.output.push_back(*first_token);
  }
  return GLACIER_HIP_OK;
}

int glacier_hip_session_prefill(glacier_hip_session *s, uint32_t lane, const uint32_t *tokens,
                                uint32_t n, uint32_t *first_token, float *logits_host) {
  return prefill_impl(s, lane, tokens, n, first_token, logits_host, false);
}

int glacier_hip_session_prefill_staged(glacier_hip_session *s, uint32_t lane,
                                       const uint32_t *tokens, uint32_t n, uint32_t *first_token,
                                       float *logits_host) {
  return prefill_impl(s, lane, tokens, n, first_token, logits_host, true);
}

int glacier_hip_session_decode_step(glacier_hip_session *s, const uint32_t *lanes,
                                    const uint32_t *tokens, uint32_t count,
                                    const uint64_t *eligible_words_host, uint32_t *next_tokens,
                                    float *logits_host) {
  if (!s || !lanes || !tokens || !next_tokens) return GLACIER_HIP_INVALID_ARGUMENT;
  if (count == 0 || count > s->lanes.size()) return GLACIER_HIP_SHAPE_MISMATCH;
  const auto &c = s->model->cfg;
  for (uint32_t i = 0; i < count; ++i) {
    if (lanes[i] >= s->lanes.size() || !s->lanes[lanes[i]].kv.active) return GLACIER_HIP_INVALID_ARGUMENT;
    for (uint32_t j = 0; j < i; ++j)
      if (lanes[j] == lanes[i]) return GLACIER_HIP_INVALID_ARGUMENT;
    if (tokens[i] >= c.vocab_size) return GLACIER_HIP_SHAPE_MISMATCH;
    if (s->lanes[lanes[i]].kv.len + 1 > s->opt.max_positions) return GLACIER_HIP_CACHE_FULL;
  }
  GH_SUBMISSION(s->model->ctx);
  if (s->prep.active) return GLACIER_HIP_TRANSACTION_ACTIVE;
  for (uint32_t i = 0; i < count; ++i)  // a held first token publishes through a wave first
    if (s->lanes[lanes[i]].first_pending || s->lanes[lanes[i]].retired)
      return GLACIER_HIP_INVALID_TRANSACTION;
  std::vector<RowTxn> txns;
  int rc = run_step(s, lanes, tokens, count, true, eligible_words_host, logits_host, txns);
  if (rc) return rc;
  // publish: KV root + length, sampler counter, output word (all or nothing)
  if ((rc = commit_rows(s, txns))) return rc;  // staged under the lock: cannot fail
  for (uint32_t i = 0; i < count; ++i) next_tokens[i] = (uint32_t)s->res_host[i].index;
  for (uint32_t i = 0; i < count; ++i) {
    Lane &ln = s->lanes[lanes[i]];
    // the eligible (posthead) branch does not count a sampler call
    // (generate.zig:5574-5598); the greedy sampler does (:5593)
    if (!eligible_words_host) ln.sampling_calls += 1;
    ln.output.push_back(next_tokens[i]);
  }
  return GLACIER_HIP_OK;
}

int glacier_hip_session_lane_root(glacier_hip_session *s, uint32_t lane,
                                  glacier_hip_page_map_root_t *out) {
  if (!s || !out || lane >= s->lanes.size()) return GLACIER_HIP_INVALID_ARGUMENT;
  *out = s->lanes[lane].kv.root;
  return GLACIER_HIP_OK;
}

int glacier_hip_session_lane_state(glacier_hip_session *s, uint32_t lane,
                                   glacier_hip_lane_state_t *out) {
  if (!s || !out || lane >= s->lanes.size()) return GLACIER_HIP_INVALID_ARGUMENT;
  const Lane &ln = s->lanes[lane];
  out->kv_positions = ln.kv.len;
  out->published_tokens = ln.output.size();
  out->sampling_calls = ln.sampling_calls;
  memcpy(out->rng_state, ln.rng, sizeof ln.rng);
  gh::token_sequence_sha256(ln.output.data(), ln.output.size(), out->output_sha256);
  return GLACIER_HIP_OK;
}

int glacier_hip_session_read_kv_row(glacier_hip_session *s, uint32_t lane, uint32_t layer,
                                    int value, uint32_t position, float *out_host) {
  if (!s || !out_host || lane >= s->lanes.size()) return GLACIER_HIP_INVALID_ARGUMENT;
  const auto &c = s->model->cfg;
  const Lane &ln = s->lanes[lane];
  if (layer >= c.num_layers || position >= ln.kv.len) return GLACIER_HIP_SHAPE_MISMATCH;
  const int32_t page = ln.kv.page_of[position / 16];
  if (page < 0) return GLACIER_HIP_INVALID_TRANSACTION;
  const size_t kvd = (size_t)c.num_kv_heads * c.head_dim;
  const size_t elem = s->opt.kv_dtype == GLACIER_HIP_F16 ? 2 : 4;
  const size_t off = ((((size_t)page * c.num_layers + layer) * 2 + (value ? 1 : 0)) * 16 +
                      position % 16) * kvd;
  glacier_hip_context *ctx = s->model->ctx;
  std::vector<uint8_t> raw(kvd * elem);
  GH_CHECK(ctx, hipMemcpy(raw.data(), (char *)s->kv_pool + off * elem, kvd * elem,
                          hipMemcpyDeviceToHost));
  for (size_t i = 0; i < kvd; ++i) {
    if (elem == 4) memcpy(&out_host[i], &raw[4 * i], 4);
    else {
      uint16_t hv;
      memcpy(&hv, &raw[2 * i], 2);
      out_host[i] = gh::f16_to_f32(hv);
    }
  }
  return GLACIER_HIP_OK;
}

int glacier_hip_session_lane_kv_sha256(glacier_hip_session *s, uint32_t lane, uint8_t out[32]) {
  if (!s || !out || lane >= s->lanes.size()) return GLACIER_HIP_INVALID_ARGUMENT;
  return logical_kv_sha256(s, lane, out);
}

int glacier_hip_session_page_of(glacier_hip_session *s, uint32_t lane, uint32_t logical_page,
                                int32_t *physical_out) {
  if (!s || !physical_out || lane >= s->lanes.size()) return GLACIER_HIP_INVALID_ARGUMENT;
  const Lane &ln = s->lanes[lane];
  if (logical_page >= ln.kv.page_of.size()) return GLACIER_HIP_SHAPE_MISMATCH;
  *physical_out = ln.kv.page_of[logical_page];
  return GLACIER_HIP_OK;
}

int glacier_hip_session_set_head_domain(glacier_hip_session *s, int mode) {
  if (!s || (mode != GLACIER_HIP_HEAD_DOMAIN_POSTHEAD && mode != GLACIER_HIP_HEAD_DOMAIN_PREHEAD))
    return GLACIER_HIP_INVALID_ARGUMENT;
  GH_SUBMISSION(s->model->ctx);
  s->head_domain = mode;
  return GLACIER_HIP_OK;
}

int glacier_hip_session_page_generation(glacier_hip_session *s, uint32_t lane,
                                        uint32_t logical_page, uint64_t *ownership_generation_out) {
  if (!s || !ownership_generation_out || lane >= s->lanes.size()) return GLACIER_HIP_INVALID_ARGUMENT;
  const Lane &ln = s->lanes[lane];
  if (logical_page >= ln.kv.page_gen.size()) return GLACIER_HIP_SHAPE_MISMATCH;
  *ownership_generation_out = ln.kv.page_gen[logical_page];
  return GLACIER_HIP_OK;
}


// ---- checkpoint page images (continuation_paged_kv_restore.zig) ----------

int glacier_hip_session_encode_page_image(glacier_hip_session *s, uint32_t lane,
                                          uint32_t logical_page,
                                          const uint8_t challenge_sha256[32], uint8_t *out,
                                          uint64_t out_capacity, uint64_t *out_len,
                                          glacier_hip_page_image_v1_t *info) {
  if (!s) return GLACIER_HIP_INVALID_HANDLE;
  if (!challenge_sha256 || !out || !out_len || lane >= s->lanes.size())
    return GLACIER_HIP_INVALID_ARGUMENT;
  GH_SUBMISSION(s->model->ctx);
  const auto &c = s->model->cfg;
  const Lane &ln = s->lanes[lane];
  glacier_hip_page_image_v1_t tmp{};
  glacier_hip_page_image_v1_t &hd = info ? *info : tmp;
  memset(&hd, 0, sizeof hd);
  auto reject = [&](uint32_t e) {
    hd.error = e;
    return GLACIER_HIP_INVALID_CHECKPOINT;
  };
  // encodePageImageV1 (:174-261): a committed page of the current root
  bool zero = true;
  for (int i = 0; i < 32; ++i) zero = zero && challenge_sha256[i] == 0;
  if (zero || !ln.kv.active) return reject(GLACIER_HIP_PAGE_IMAGE_INVALID_PAGE_IMAGE);
  const gpk::Root root = ln.kv.root;
  if (logical_page >= root.committed_pages) return reject(GLACIER_HIP_PAGE_IMAGE_INVALID_PAGE_IMAGE);
  const uint64_t start = (uint64_t)logical_page * 16;
  if (start >= root.committed_len) return reject(GLACIER_HIP_PAGE_IMAGE_INVALID_PAGE_IMAGE);
  const uint64_t rows = std::min<uint64_t>(16, root.committed_len - start);
  const uint64_t L = c.num_layers, kvd = (uint64_t)c.num_kv_heads * c.head_dim;
  const uint64_t need = gpi::encoded_bytes(L, kvd, rows);
  if (!need) return reject(GLACIER_HIP_PAGE_IMAGE_INVALID_PAGE_IMAGE);
  if (out_capacity < need) return reject(GLACIER_HIP_PAGE_IMAGE_CAPACITY_EXCEEDED);
  const int32_t phys = ln.kv.page_of[logical_page];
  if (phys < 0 || ln.kv.page_gen[logical_page] == 0)
    return reject(GLACIER_HIP_PAGE_IMAGE_INVALID_PAGE_IMAGE);
  // read the page back, then lay its committed rows out canonically:
  // (layer, K then V, row, dim) little-endian f32; fp16 widens exactly
  const size_t elem = s->opt.kv_dtype == GLACIER_HIP_F16 ? 2 : 4;
  const size_t page_elems = L * 2 * 16 * kvd;
  std::vector<uint8_t> raw(page_elems * elem);
  glacier_hip_context *ctx = s->model->ctx;
  GH_CHECK(ctx, hipMemcpy(raw.data(), (char *)s->kv_pool + (size_t)phys * page_elems * elem,
                          page_elems * elem, hipMemcpyDeviceToHost));
  std::vector<uint8_t> canon(L * 2 * rows * kvd * 4);
  size_t w = 0;
  for (uint64_t l = 0; l < L; ++l)
    for (int v = 0; v < 2; ++v)
      for (uint64_t r = 0; r < rows; ++r) {
        const uint8_t *src = raw.data() + (((l * 2 + v) * 16 + r) * kvd) * elem;
        for (uint64_t i = 0; i < kvd; ++i, w += 4) {
          float f;
          if (elem == 4) {
            memcpy(&f, src + 4 * i, 4);
          } else {
            uint16_t hv;
            memcpy(&hv, src + 2 * i, 2);
            f = gh::f16_to_f32(hv);
          }
          uint32_t b;
          memcpy(&b, &f, 4);
          for (int k = 0; k < 4; ++k) canon[w + k] = (uint8_t)(b >> (8 * k));
        }
      }
  glacier_hip_page_ref_t ref{gpk::kPageRefAbi, ln.kv.instance, logical_page,
                             ln.kv.page_gen[logical_page]};
  const uint32_t e = gpi::encode(root, L, kvd, ln.kv.max_seq, ref, rows, canon.data(),
                                 canon.size(), challenge_sha256, out, out_capacity, out_len);
  if (e) return reject(e);
  gpi::decode(out, *out_len, challenge_sha256, &hd);
  return GLACIER_HIP_OK;
}

int glacier_hip_session_restore_checkpoint(glacier_hip_session *s, uint32_t lane,
                                           const uint8_t *const *images,
                                           const uint64_t *image_lens, uint32_t count,
                                           const uint8_t challenge_sha256[32], uint64_t seed,
                                           glacier_hip_checkpoint_restore_v1_t *out,
                                           glacier_hip_page_ref_t *target_refs) {
  if (!s) return GLACIER_HIP_INVALID_HANDLE;
  if (!images || !image_lens || !challenge_sha256 || !out || lane >= s->lanes.size() ||
      count == 0)
    return GLACIER_HIP_INVALID_ARGUMENT;
  for (uint32_t i = 0; i < count; ++i)
    if (!images[i]) return GLACIER_HIP_INVALID_ARGUMENT;
  GH_SUBMISSION(s->model->ctx);
  if (s->prep.active) return GLACIER_HIP_TRANSACTION_ACTIVE;
  memset(out, 0, sizeof *out);
  out->abi_version = gpi::kCheckpointRestoreAbi;
  const auto &c = s->model->cfg;
  const uint64_t L = c.num_layers, kvd = (uint64_t)c.num_kv_heads * c.head_dim;
  Lane &ln = s->lanes[lane];
  if (ln.lease) return GLACIER_HIP_INVALID_TRANSACTION;
  // the restore target is a fresh request (PagedKVCache.initForCheckpoint)
  reset_lane(s, ln, seed);
  auto reject = [&](uint32_t e) {
    out->error = e;
    return GLACIER_HIP_INVALID_CHECKPOINT;
  };
  // ---- decode every image (restoreAndCommitV1's loop, :405-447) ----
  std::vector<glacier_hip_page_image_v1_t> hd(count);
  for (uint32_t i = 0; i < count; ++i) {
    const uint32_t e = gpi::decode(images[i], image_lens[i], challenge_sha256, &hd[i]);
    if (e) return reject(e);
    if (hd[i].source_ref.logical_page != i) return reject(GLACIER_HIP_PAGE_IMAGE_INVALID_RESTORE_PLAN);
    if (i > 0 && (memcmp(&hd[i].source_root, &hd[0].source_root, sizeof hd[0].source_root) != 0 ||
                  hd[i].num_layers != hd[0].num_layers || hd[i].dim != hd[0].dim ||
                  hd[i].max_seq != hd[0].max_seq))
      return reject(GLACIER_HIP_PAGE_IMAGE_FOREIGN_CHECKPOINT);
  }
  const glacier_hip_page_map_root_t src = hd[0].source_root;
  out->source_root = src;
  // ---- restoreCheckpointV1 validation (paged_kv_cache.zig:614-684) ----
  if (hd[0].num_layers != L || hd[0].dim != kvd || hd[0].max_seq != ln.kv.max_seq)
    return reject(GLACIER_HIP_PAGE_IMAGE_INVALID_CHECKPOINT);
  if (ln.kv.instance == src.cache_instance) {  // initForCheckpoint: a different instance
    ln.kv.instance = gpk::next_cache_instance();
    ln.kv.root.cache_instance = ln.kv.instance;
    gpk::empty_ownership_digest(ln.kv.instance, L, kvd, ln.kv.max_seq, ln.kv.root.ownership_sha256);
  }
  if (src.committed_len > ln.kv.max_seq || src.committed_pages > ln.kv.page_of.size() ||
      src.committed_pages != count)
    return reject(GLACIER_HIP_PAGE_IMAGE_INVALID_CHECKPOINT);
  uint8_t own[32];
  gpk::empty_ownership_digest(src.cache_instance, L, kvd, ln.kv.max_seq, own);
  for (uint32_t i = 0; i < count; ++i) {
    const glacier_hip_page_ref_t &f = hd[i].source_ref;
    const uint64_t rows = std::min<uint64_t>(16, src.committed_len - (uint64_t)i * 16);
    if (f.cache_instance != src.cache_instance || f.ownership_generation == 0 ||
        hd[i].committed_rows != rows)
      return reject(GLACIER_HIP_PAGE_IMAGE_INVALID_CHECKPOINT);
    gpk::append_ownership_digest(own, f.cache_instance, f.logical_page, f.ownership_generation, own);
  }
  if (memcmp(own, src.ownership_sha256, 32) != 0)
    return reject(GLACIER_HIP_PAGE_IMAGE_INVALID_CHECKPOINT);
  // ---- build the device pages (an fp16 pool takes only exact values) ----
  const bool f16 = s->opt.kv_dtype == GLACIER_HIP_F16;
  const size_t elem = f16 ? 2 : 4;
  const size_t page_elems = L * 2 * 16 * kvd;
  std::vector<uint8_t> pages((size_t)count * page_elems * elem, 0);
  for (uint32_t i = 0; i < count; ++i) {
    const uint8_t *rd = images[i] + hd[i].payload_offset;
    uint8_t *dst = pages.data() + (size_t)i * page_elems * elem;
    for (uint64_t l = 0; l < L; ++l)
      for (int v = 0; v < 2; ++v)
        for (uint64_t r = 0; r < hd[i].committed_rows; ++r)
          for (uint64_t k = 0; k < kvd; ++k, rd += 4) {
            const uint32_t b = (uint32_t)rd[0] | ((uint32_t)rd[1] << 8) | ((uint32_t)rd[2] << 16) |
                               ((uint32_t)rd[3] << 24);
            const size_t at = ((l * 2 + v) * 16 + r) * kvd + k;
            if (!f16) {
              memcpy(dst + 4 * at, &b, 4);
            } else {
              float f;
              memcpy(&f, &b, 4);
              const uint16_t hv = gh::f32_to_f16(f);
              const float back = gh::f16_to_f32(hv);
              if (memcmp(&back, &f, 4) != 0 && !(back != back && f != f))
                return reject(GLACIER_HIP_PAGE_IMAGE_INVALID_CHECKPOINT);
              memcpy(dst + 2 * at, &hv, 2);
            }
          }
  }
  if (s->pool.free.size() < count) return GLACIER_HIP_CACHE_FULL;
  // ---- install: pool pages, HBM rows, page table, page map ----
  glacier_hip_context *ctx = s->model->ctx;
  std::vector<int32_t> phys(count);
  for (uint32_t i = 0; i < count; ++i) {
    phys[i] = s->pool.free.back();
    s->pool.free.pop_back();
  }
  auto undo = [&]() {
    for (uint32_t i = 0; i < count; ++i) s->pool.free.push_back(phys[count - 1 - i]);
  };
  for (uint32_t i = 0; i < count; ++i) {
    if (hipMemcpy((char *)s->kv_pool + (size_t)phys[i] * page_elems * elem,
                  pages.data() + (size_t)i * page_elems * elem, page_elems * elem,
                  hipMemcpyHostToDevice) != hipSuccess) {
      undo();
      ctx->last_error = "restore: page upload failed";
      return GLACIER_HIP_DEVICE_ERROR;
    }
    s->pt_host[(size_t)lane * s->max_pages + i] = phys[i];
  }
  if (hipMemcpy(s->page_table + (size_t)lane * s->max_pages, s->pt_host + (size_t)lane * s->max_pages,
                (size_t)count * 4, hipMemcpyHostToDevice) != hipSuccess) {
    undo();
    ctx->last_error = "restore: page table upload failed";
    return GLACIER_HIP_DEVICE_ERROR;
  }
  uint8_t tgt[32];
  memcpy(tgt, ln.kv.root.ownership_sha256, 32);
  for (uint32_t i = 0; i < count; ++i) {
    ln.kv.page_of[i] = phys[i];
    ln.kv.page_gen[i] = (uint64_t)i + 1;
    gpk::append_ownership_digest(tgt, ln.kv.instance, i, (uint64_t)i + 1, tgt);
    if (target_refs) target_refs[i] = {gpk::kPageRefAbi, ln.kv.instance, i, (uint64_t)i + 1};
  }
  ln.kv.len = src.committed_len;
  ln.kv.next_page_generation = (uint64_t)count + 1;
  ln.kv.root.cache_instance = ln.kv.instance;
  ln.kv.root.generation = 2;
  ln.kv.root.committed_len = src.committed_len;
  ln.kv.root.committed_pages = src.committed_pages;
  memcpy(ln.kv.root.ownership_sha256, tgt, 32);
  ln.kv.next_root_generation = 3;
  ln.prompt_len = src.committed_len;
  out->target_root = ln.kv.root;
  out->restored_pages = count;
  out->restored_payload_bytes = (uint64_t)count * L * 2 * 16 * kvd * 4;
  return GLACIER_HIP_OK;
}

}  // extern "C"

// abortPublication of a staged wave's permit (the sequence stays for the retry)
static void release_permit(PreparedWave &P) {
  if (!P.cohort) return;
  (void)P.cohort->lease.bank->abort_publication(P.permit);
  P.cohort = nullptr;
}

// Leased lanes of the cohort `c` in this session (lanes whose coordinator
// shares its bank, tree and publication sequence).
static bool same_cohort(const glb::Leased &a, const glb::Leased &b) {
  return a.bank == b.bank && a.tree == b.tree && a.sequence == b.sequence &&
         a.request_epoch == b.request_epoch && a.session_id == b.session_id;
}

// A v3 resource commitment's default slot (ResourceCommitmentV3 .{}, :141-160).
static void empty_resource_v3(glacier_hip_resource_commitment_v3_t &r, uint32_t slot) {
  memset(&r, 0, sizeof r);
  r.abi_version = gpub::kResourceCommitmentAbi;
  r.lane_index = slot;
  r.lifecycle = GLACIER_HIP_LIFECYCLE_RECLAIMED;
  r.allocation_set.abi_version = gpub::kAllocationSetAbi;
}

// collectResourceSnapshot's commitment of a cohort lane that is not in the
// wave because an earlier wave published its terminal token (:834-860): its
// sealed root and digest while its pages stay charged, the seal's root only
// once they are reclaimed.
static int retired_resource_v3(const Lane &ln, glacier_hip_leased_kv *l, uint32_t slot,
                               glacier_hip_resource_commitment_v3_t &r) {
  glb::Leased &a = l->lease;
  empty_resource_v3(r, slot);
  uint32_t life = 0;
  if (a.lifecycle(&life)) return GLACIER_HIP_INVALID_TRANSACTION;
  r.lifecycle = life;
  r.coordinator_instance = a.instance;
  r.cache_instance = ln.kv.root.cache_instance;
  r.scope_index = a.scope.node_index;
  r.scope_generation = a.scope.generation;
  memcpy(r.kv_state_chain_after, ln.chain, 32);
  glacier_hip_terminal_seal_t seal;
  const bool sealed = a.terminal_seal(&seal, nullptr, nullptr) == GLACIER_HIP_LEASE_OK;
  if (life == GLACIER_HIP_LIFECYCLE_TERMINAL_RETAINED) {
    if (!sealed) return GLACIER_HIP_INVALID_TRANSACTION;
    r.root = seal.root;
    r.has_canonical_after = 1;
    memcpy(r.canonical_after_sha256, seal.logical_kv_sha256, 32);
    r.has_binding_summary = 1;
    if (a.binding_summary(GLACIER_HIP_BINDING_LIVE, &r.binding_summary) ||
        a.allocation_set(GLACIER_HIP_BINDING_LIVE, &r.allocation_set) ||
        memcmp(&r.binding_summary, &seal.bindings, sizeof seal.bindings) != 0)
      return GLACIER_HIP_INVALID_TRANSACTION;
  } else if (life == GLACIER_HIP_LIFECYCLE_RECLAIMED) {
    if (sealed) r.root = seal.root;
  } else {
    return GLACIER_HIP_INVALID_TRANSACTION;  // live without a wave, or mid-reclaim
  }
  return GLACIER_HIP_OK;
}

// Batch.begin (paged_token_txn.zig:346-471 for v1 waves,
// paged_lease_token_txn.zig:1117-1250 for v3 waves): validate the lanes, run
// the wave's device step privately, take the cohort's publication permit and
// seal the proposal into s->prep.
static int step_prepare_impl(glacier_hip_session *s, const uint32_t *lanes, const uint32_t *tokens,
                             uint32_t count, const uint64_t *eligible_words_host,
                             const glacier_hip_publication_binding_t *binding, bool v3,
                             const uint32_t *terminal_reason, uint32_t *next_tokens,
                             float *logits_host) {
  if (!s || !lanes || !binding || !next_tokens) return GLACIER_HIP_INVALID_ARGUMENT;
  if (count == 0 || count > GLACIER_HIP_PUBLICATION_WIDTH || count > s->lanes.size())
    return GLACIER_HIP_SHAPE_MISMATCH;
  const auto &c = s->model->cfg;
  uint32_t mask = 0;
  int first = -1;
  glacier_hip_leased_kv *cohort = nullptr;
  for (uint32_t i = 0; i < count; ++i) {
    // validateAndBuildLane's checks (:832-944; v3 :663-733)
    if (lanes[i] >= s->lanes.size() || !s->lanes[lanes[i]].kv.active) return GLACIER_HIP_INVALID_ARGUMENT;
    for (uint32_t j = 0; j < i; ++j)
      if (lanes[j] == lanes[i]) return GLACIER_HIP_INVALID_ARGUMENT;
    const uint32_t slot = binding->lane_index[i];
    if (slot >= GLACIER_HIP_PUBLICATION_WIDTH || (mask >> slot & 1)) return GLACIER_HIP_INVALID_ARGUMENT;
    mask |= 1u << slot;
    const Lane &ln = s->lanes[lanes[i]];
    if (ln.retired) return GLACIER_HIP_INVALID_TRANSACTION;
    const int kind = ln.first_pending ? 1 : 0;
    if (!kind && !ln.chain_init) return GLACIER_HIP_INVALID_TRANSACTION;  // no first wave yet
    if (first >= 0 && first != kind) return GLACIER_HIP_INVALID_TRANSACTION;  // one kind per wave
    first = kind;
    if (!kind) {
      if (!tokens || tokens[i] >= c.vocab_size) return GLACIER_HIP_SHAPE_MISMATCH;
      if (ln.kv.len + 1 > s->opt.max_positions) return GLACIER_HIP_CACHE_FULL;
      if (ln.kv.len + 1 != ln.prompt_len + ln.output.size()) return GLACIER_HIP_INVALID_TRANSACTION;
    }
    // a lane's chain runs under one ABI's domains for its whole request
    if (ln.chain_init && ln.chain_v3 != v3) return GLACIER_HIP_INVALID_TRANSACTION;
    // leased lanes publish under their cohort's permit for the binding's
    // sequence: every leased lane of the wave shares one bank, tree and
    // sequence cell, and the permit generation goes into the proposal
    if (ln.lease) {
      if (cohort && !same_cohort(ln.lease->lease, cohort->lease)) return GLACIER_HIP_INVALID_ARGUMENT;
      if (!cohort) cohort = ln.lease;
    } else if (v3) {
      return GLACIER_HIP_INVALID_ARGUMENT;  // v3 waves publish leased lanes only
    }
    if (v3) {
      if (ln.v3_slot >= 0 && (uint32_t)ln.v3_slot != slot) return GLACIER_HIP_INVALID_ARGUMENT;
      if (terminal_reason && terminal_reason[i] > 1 + GLACIER_HIP_TERMINAL_CANCELLED)
        return GLACIER_HIP_INVALID_ARGUMENT;
    }
  }
  if (v3) {
    // the cohort's slots are fixed, and every cohort lane that is not
    // retired joins every wave (Batch.begin's activeMask rule, :1127-1131)
    for (uint32_t l = 0; l < s->lanes.size(); ++l) {
      const Lane &o = s->lanes[l];
      if (!o.lease || !same_cohort(o.lease->lease, cohort->lease) || o.v3_slot < 0) continue;
      const bool in_wave = std::find(lanes, lanes + count, l) != lanes + count;
      if (in_wave) continue;
      if (mask >> o.v3_slot & 1) return GLACIER_HIP_INVALID_ARGUMENT;  // slot of another lane
      if (!o.retired) return GLACIER_HIP_INVALID_TRANSACTION;
    }
  }
  GH_SUBMISSION(s->model->ctx);
  if (s->prep.active) return GLACIER_HIP_TRANSACTION_ACTIVE;
  PreparedWave &P = s->prep;
  P.txns.clear();
  P.lanes.assign(lanes, lanes + count);
  P.slots.assign(binding->lane_index, binding->lane_index + count);
  P.tokens.assign(count, 0);
  P.first = first == 1;
  P.elig = eligible_words_host != nullptr;
  P.v3 = v3;
  P.reasons.assign(count, 0);
  for (uint32_t i = 0; i < count; ++i)
    P.reasons[i] = v3 ? (terminal_reason ? terminal_reason[i] : 0)
                      : (binding->terminal[i] ? 1 + GLACIER_HIP_TERMINAL_EOS : 0);
  std::vector<std::array<uint8_t, 32>> digests;
  if (!P.first) {
    int rc = run_step(s, lanes, tokens, count, true, eligible_words_host, logits_host, P.txns);
    if (rc) return rc;
    rc = row_payload_sha256(s, P.txns, digests);
    if (rc) {
      abort_rows(s, P.txns);
      return rc;
    }
    for (uint32_t i = 0; i < count; ++i) P.tokens[i] = (uint32_t)s->res_host[i].index;
  } else {
    for (uint32_t i = 0; i < count; ++i) P.tokens[i] = s->lanes[lanes[i]].first_token;
  }
  auto fail = [&](int rc) {
    if (!P.first) abort_rows(s, P.txns);
    release_permit(P);
    return rc;
  };
  P.cohort = nullptr;
  if (cohort) {
    glb::Leased &a = cohort->lease;
    if (binding->transaction_sequence != *a.sequence || binding->request_epoch != a.request_epoch)
      return fail(GLACIER_HIP_INVALID_TRANSACTION);
    if (v3) {
      // collectResourceSnapshot's tree checks (:765-776): a live tree whose
      // parent is the session's receipt and which charges KV bytes only
      glb::Claim other = a.tree->ceiling, cur = a.tree->current;
      other.kv_bytes = cur.kv_bytes = 0;
      if (a.bank->validate_tree(*a.tree) != GLACIER_HIP_LEASE_OK ||
          memcmp(&a.tree->parent, &binding->receipt, sizeof binding->receipt) != 0 ||
          !glb::claim_zero(other) || !glb::claim_zero(cur))
        return fail(GLACIER_HIP_INVALID_TRANSACTION);
    }
    if (a.bank->begin_publication(*a.tree, a.request_epoch, a.session_id, *a.sequence, &P.permit))
      return fail(GLACIER_HIP_INVALID_TRANSACTION);
    P.cohort = cohort;
  }
  glacier_hip_token_proposal_v1_t &pr = P.proposal;
  gpub::empty_proposal(pr);
  pr.execution_abi = binding->execution_abi;
  pr.request_epoch = binding->request_epoch;
  pr.transaction_sequence = binding->transaction_sequence;
  pr.resource_permit_generation =
      P.cohort ? P.permit.generation : binding->resource_permit_generation;
  pr.live_mask = mask;
  pr.live_lane_count = count;
  pr.kv_capacity_bytes = binding->kv_capacity_bytes;
  pr.receipt = binding->receipt;
  std::vector<std::array<uint8_t, 32>> canonical(count);
  for (uint32_t i = 0; i < count; ++i) {
    Lane &ln = s->lanes[lanes[i]];
    glacier_hip_lane_proposal_v1_t &lp = pr.lanes[P.slots[i]];
    glacier_hip_root_transition_v1_t &t = lp.kv_transition;
    lp.lane_index = P.slots[i];
    lp.step_index = ln.output.size();
    lp.prompt_len = ln.prompt_len;
    lp.kv_capacity_bytes = lane_capacity_bytes(s);
    // the canonical logical-KV digest after the wave's row: a first wave's
    // committed rows, a terminal row's committed rows plus its staged row
    // (prepareTokenRow's require_canonical_after, :579-625)
    if (P.first || (v3 && P.reasons[i])) {
      if (int rc = logical_kv_sha256(s, lanes[i], canonical[i].data(), P.first ? 0 : 1))
        return fail(rc);
    }
    if (P.first) {  // initialRootTransition (:790-811; v3 :579-606)
      const glacier_hip_page_map_root_t &r = ln.kv.root;
      lp.has_kv_transition = 0;
      lp.kv_before = lp.kv_after = ln.kv.len;
      t.cache_instance = r.cache_instance;
      copy_root(r, t, true);
      copy_root(r, t, false);
      memcpy(t.initial_logical_kv_sha256, canonical[i].data(), 32);
      if (v3)
        gpub::initial_state_chain_v3(canonical[i].data(), r, t.state_chain_before);
      else
        gpub::initial_state_chain(canonical[i].data(), r, t.state_chain_before);
      memcpy(t.state_chain_after, t.state_chain_before, 32);
    } else {  // rootTransition (:813-872; v3 :608-661)
      const RowTxn &rt = P.txns[i];
      lp.has_kv_transition = 1;
      lp.kv_before = rt.mark.base_len;
      lp.kv_after = rt.mark.base_len + 1;
      t.cache_instance = rt.mark.cache_instance;
      t.row_txn_generation = rt.mark.generation;
      copy_root(rt.before, t, true);
      copy_root(rt.after, t, false);
      t.logical_page = rt.mark.page_ref.logical_page;
      t.page_ownership_generation = rt.mark.page_ref.ownership_generation;
      t.installs_new_page = rt.installs ? 1 : 0;
      memcpy(t.row_payload_sha256, digests[i].data(), 32);
      memcpy(t.state_chain_before, ln.chain, 32);
      if (v3)
        gpub::appended_state_chain_v3(ln.chain, rt.before, rt.after, rt.mark, digests[i].data(),
                                      t.state_chain_after);
      else
        gpub::appended_state_chain(ln.chain, rt.before, rt.after, rt.mark, digests[i].data(),
                                   t.state_chain_after);
    }
    lp.output_before = ln.output.size();
    lp.output_after = ln.output.size() + 1;
    memcpy(lp.rng_before, ln.rng, sizeof ln.rng);
    memcpy(lp.rng_after, ln.rng, sizeof ln.rng);  // greedy: the RNG never advances
    lp.sampling_calls_before = ln.sampling_calls;
    // the greedy sampler counts a call (generate.zig:5593), the eligible
    // posthead branch does not (:5574-5598); the first token is greedy
    lp.sampling_calls_after = ln.sampling_calls + ((P.first || !P.elig) ? 1 : 0);
    lp.token_id = P.tokens[i];
    lp.terminal = P.reasons[i] ? 1 : 0;
  }
  if (!v3) {
    gpub::proposal_sha256(pr, P.sha);
  } else {
    // ProposalV3 (:162-180): the v1 lanes' fields plus each lane's output
    // digest and terminal reason, the redacted tree commitment and one
    // resource commitment per slot (collectResourceSnapshot :765-896)
    glacier_hip_token_proposal_v3_t &q = P.proposal_v3;
    memset(&q, 0, sizeof q);
    q.abi_version = gpub::kProposalV3Abi;
    q.resource_bank_abi = gpub::kResourceBankAbi;
    q.resource_lease_tree_abi = gpub::kLeaseTreeAbi;
    q.resource_publication_fence_abi = gpub::kPublicationFenceAbi;
    q.leased_paged_kv_abi = gpub::kLeasedPagedKvAbi;
    q.paged_kv_abi = gpk::kPagedKvAbi;
    q.page_transition_abi = gpub::kPageTransitionV3Abi;
    q.execution_abi = pr.execution_abi;
    q.request_epoch = pr.request_epoch;
    q.transaction_sequence = pr.transaction_sequence;
    q.resource_permit_generation = pr.resource_permit_generation;
    q.live_mask = mask;
    q.live_lane_count = count;
    q.parent_receipt = binding->receipt;
    const glacier_hip_lease_tree_t &tree = *P.cohort->lease.tree;  // treeCommitment (:751-763)
    q.tree.abi_version = gpub::kTreeCommitmentAbi;
    q.tree.tree_key = tree.tree_key;
    q.tree.identity_generation = tree.identity_generation;
    q.tree.generation = tree.generation;
    q.tree.structural_revision = tree.structural_revision;
    q.tree.ceiling = tree.ceiling;
    q.tree.current = tree.current;
    q.tree.active_nodes = tree.active_nodes;
    q.tree.state_digest = tree.state_digest;
    q.tree.token_integrity = tree.integrity;
    for (uint32_t l = 0; l < GLACIER_HIP_PUBLICATION_WIDTH; ++l) {
      empty_resource_v3(q.resources[l], l);
      glacier_hip_lane_proposal_v3_t &d = q.lanes[l];
      const glacier_hip_lane_proposal_v1_t &sl = pr.lanes[l];
      d.lane_index = sl.lane_index;
      d.has_kv_transition = sl.has_kv_transition;
      d.step_index = sl.step_index;
      d.prompt_len = sl.prompt_len;
      d.kv_before = sl.kv_before;
      d.kv_after = sl.kv_after;
      d.kv_transition = sl.kv_transition;
      d.kv_transition.abi_version = gpub::kPageTransitionV3Abi;
      d.output_before = sl.output_before;
      d.output_after = sl.output_after;
      memcpy(d.rng_before, sl.rng_before, sizeof d.rng_before);
      memcpy(d.rng_after, sl.rng_after, sizeof d.rng_after);
      d.sampling_calls_before = sl.sampling_calls_before;
      d.sampling_calls_after = sl.sampling_calls_after;
      d.token_id = sl.token_id;
    }
    for (uint32_t i = 0; i < count; ++i) {
      Lane &ln = s->lanes[lanes[i]];
      glb::Leased &a = ln.lease->lease;
      const uint32_t slot = P.slots[i];
      glacier_hip_lane_proposal_v3_t &d = q.lanes[slot];
      d.terminal_reason = P.reasons[i];
      {  // outputAfterSha256 (:566-577): the output with this token appended
        std::vector<uint32_t> out(ln.output);
        out.push_back(P.tokens[i]);
        gh::token_sequence_sha256(out.data(), out.size(), d.output_sha256);
      }
      glacier_hip_resource_commitment_v3_t &r = q.resources[slot];
      uint32_t life = 0;
      if (a.lifecycle(&life) || life != GLACIER_HIP_LIFECYCLE_LIVE) return fail(GLACIER_HIP_INVALID_TRANSACTION);
      r.lifecycle = life;
      r.coordinator_instance = a.instance;
      r.cache_instance = ln.kv.root.cache_instance;
      r.scope_index = a.scope.node_index;
      r.scope_generation = a.scope.generation;
      r.root = P.first ? ln.kv.root : P.txns[i].after;
      memcpy(r.kv_state_chain_after, d.kv_transition.state_chain_after, 32);
      if (P.first || P.reasons[i]) {
        r.has_canonical_after = 1;
        memcpy(r.canonical_after_sha256, canonical[i].data(), 32);
      }
      if (P.reasons[i]) {
        // the generation the lane's terminal seal takes (TerminalPlanV3)
        r.has_terminal_generation = 1;
        r.terminal_generation = a.next_generation;
      }
      r.has_binding_summary = 1;
      if (a.binding_summary(GLACIER_HIP_BINDING_LIVE, &r.binding_summary) ||
          a.allocation_set(GLACIER_HIP_BINDING_LIVE, &r.allocation_set))
        return fail(GLACIER_HIP_INVALID_TRANSACTION);
    }
    for (uint32_t l = 0; l < s->lanes.size(); ++l) {  // retired cohort lanes
      const Lane &o = s->lanes[l];
      if (!o.lease || !same_cohort(o.lease->lease, P.cohort->lease) || o.v3_slot < 0 || !o.retired)
        continue;
      if (int rc = retired_resource_v3(o, o.lease, (uint32_t)o.v3_slot, q.resources[o.v3_slot]))
        return fail(rc);
    }
    for (const auto &r : q.resources) {  // the snapshot's cross-checks (:862-882)
      if (r.has_binding_summary != (r.allocation_set.count != 0) ||
          (r.has_binding_summary && (r.binding_summary.count != r.allocation_set.count ||
                                     r.binding_summary.payload_bytes != r.allocation_set.payload_bytes)))
        return fail(GLACIER_HIP_INVALID_TRANSACTION);
    }
    gpub::proposal_v3_sha256(q, P.sha);
  }
  P.active = true;
  for (uint32_t i = 0; i < count; ++i) next_tokens[i] = P.tokens[i];
  return GLACIER_HIP_OK;
}

extern "C" {

int glacier_hip_session_step_prepare(glacier_hip_session *s, const uint32_t *lanes,
                                     const uint32_t *tokens, uint32_t count,
                                     const uint64_t *eligible_words_host,
                                     const glacier_hip_publication_binding_t *binding,
                                     glacier_hip_token_proposal_v1_t *proposal_out,
                                     uint8_t proposal_sha256_out[32], uint32_t *next_tokens,
                                     float *logits_host) {
  if (!proposal_out || !proposal_sha256_out) return GLACIER_HIP_INVALID_ARGUMENT;
  const int rc = step_prepare_impl(s, lanes, tokens, count, eligible_words_host, binding, false,
                                   nullptr, next_tokens, logits_host);
  if (rc) return rc;
  *proposal_out = s->prep.proposal;
  memcpy(proposal_sha256_out, s->prep.sha, 32);
  return GLACIER_HIP_OK;
}

int glacier_hip_session_step_prepare_v3(glacier_hip_session *s, const uint32_t *lanes,
                                        const uint32_t *tokens, uint32_t count,
                                        const uint64_t *eligible_words_host,
                                        const glacier_hip_publication_binding_t *binding,
                                        const uint32_t *terminal_reason,
                                        glacier_hip_token_proposal_v3_t *proposal_out,
                                        uint8_t proposal_sha256_out[32], uint32_t *next_tokens) {
  if (!proposal_out || !proposal_sha256_out) return GLACIER_HIP_INVALID_ARGUMENT;
  const int rc = step_prepare_impl(s, lanes, tokens, count, eligible_words_host, binding, true,
                                   terminal_reason, next_tokens, nullptr);
  if (rc) return rc;
  *proposal_out = s->prep.proposal_v3;
  memcpy(proposal_sha256_out, s->prep.sha, 32);
  return GLACIER_HIP_OK;
}

int glacier_hip_session_step_abort(glacier_hip_session *s) {
  // Batch.abort / rollback (:565-600): every staged row aborts; nothing else
  // was touched
  if (!s) return GLACIER_HIP_INVALID_ARGUMENT;
  GH_SUBMISSION(s->model->ctx);
  if (!s->prep.active) return GLACIER_HIP_INVALID_TRANSACTION;
  if (!s->prep.first) abort_rows(s, s->prep.txns);
  release_permit(s->prep);
  s->prep.active = false;
  return GLACIER_HIP_OK;
}

int glacier_hip_session_step_commit(glacier_hip_session *s, const glacier_hip_prepare_ack_v1_t *ack,
                                    glacier_hip_commit_receipt_v1_t *receipt_out) {
  // Batch.prepare's ack checks (:503-515) then Batch.commit (:519-563)
  if (!s || !ack) return GLACIER_HIP_INVALID_ARGUMENT;
  GH_SUBMISSION(s->model->ctx);
  PreparedWave &P = s->prep;
  if (!P.active) return GLACIER_HIP_INVALID_TRANSACTION;
  if (ack->abi_version != (P.v3 ? gpub::kPrepareAckV3Abi : gpub::kPrepareAckAbi) ||
      ack->sink_epoch == 0 || ack->reservation_id == 0 ||
      memcmp(ack->proposal_sha256, P.sha, 32) != 0) {
    if (!P.first) abort_rows(s, P.txns);
    release_permit(P);
    P.active = false;
    return GLACIER_HIP_INVALID_TRANSACTION;
  }
  // the cohort's permit must still be the bank's live one before anything
  // is published (commitPublicationAssumeValid may not fail after commit)
  if (P.cohort && P.cohort->lease.bank->validate_publication(P.permit) != GLACIER_HIP_LEASE_OK) {
    if (!P.first) abort_rows(s, P.txns);
    P.cohort = nullptr;  // the bank no longer holds this permit
    P.active = false;
    s->model->ctx->last_error = "the wave's publication permit is no longer the bank's live permit";
    return GLACIER_HIP_INVALID_TRANSACTION;
  }
  if (P.v3) {  // each terminal lane's seal still takes the generation the proposal names
    for (size_t i = 0; i < P.lanes.size(); ++i) {
      const glacier_hip_resource_commitment_v3_t &r = P.proposal_v3.resources[P.slots[i]];
      const glacier_hip_leased_kv *l = s->lanes[P.lanes[i]].lease;
      if (r.has_terminal_generation && (!l || l->lease.next_generation != r.terminal_generation)) {
        if (!P.first) abort_rows(s, P.txns);
        release_permit(P);
        P.active = false;
        s->model->ctx->last_error = "a terminal lane's coordinator moved after the wave was proposed";
        return GLACIER_HIP_INVALID_TRANSACTION;
      }
    }
  }
  if (!P.first) {
    const int rc = commit_rows(s, P.txns);  // staged under the session's rule: cannot fail
    if (rc) {
      release_permit(P);
      P.active = false;
      return rc;
    }
  }
  for (size_t i = 0; i < P.lanes.size(); ++i) {
    Lane &ln = s->lanes[P.lanes[i]];
    const glacier_hip_lane_proposal_v1_t &lp = P.proposal.lanes[P.slots[i]];
    memcpy(ln.rng, lp.rng_after, sizeof ln.rng);
    ln.sampling_calls = lp.sampling_calls_after;
    ln.output.push_back(lp.token_id);
    memcpy(ln.chain, lp.kv_transition.state_chain_after, 32);
    ln.chain_init = true;
    ln.chain_v3 = P.v3;
    if (P.v3) ln.v3_slot = (int)P.slots[i];
    ln.first_pending = false;
    if (lp.terminal) ln.retired = true;
  }
  uint8_t commit_sha[32];
  if (P.v3)
    gpub::commit_v3_sha256(P.sha, *ack, commit_sha);
  else
    gpub::commit_sha256(P.sha, *ack, commit_sha);
  int status = GLACIER_HIP_OK;
  if (P.cohort) {
    // the wave's permit commits once (the cohort's sequence advances), then
    // every leased lane whose terminal token this wave published is sealed.
    // The rows are published by now: a bank or seal refusal here is drift
    // between the bank and the lanes (the reference traps), reported as
    // GLACIER_HIP_SCHEDULER_POISONED after the wave's bookkeeping completes.
    glb::Leased &a = P.cohort->lease;
    if (a.bank->commit_publication(P.permit) == GLACIER_HIP_LEASE_OK) {
      *a.sequence = P.permit.sequence + 1;
    } else {
      status = GLACIER_HIP_SCHEDULER_POISONED;
      s->model->ctx->last_error = "the bank refused a validated publication permit at commit";
    }
    for (size_t i = 0; i < P.lanes.size(); ++i) {
      const glacier_hip_lane_proposal_v1_t &lp = P.proposal.lanes[P.slots[i]];
      glacier_hip_leased_kv *l = s->lanes[P.lanes[i]].lease;
      if (l && lp.terminal && status == GLACIER_HIP_OK &&
          l->lease.finalize_wave_terminal(P.permit.sequence, P.reasons[i] - 1, lp.token_id, P.sha,
                                          commit_sha) !=
              GLACIER_HIP_LEASE_OK) {
        status = GLACIER_HIP_SCHEDULER_POISONED;
        s->model->ctx->last_error = "a published terminal token's lane could not be sealed";
      }
    }
    P.cohort = nullptr;
  }
  if (receipt_out) {
    memset(receipt_out, 0, sizeof *receipt_out);
    receipt_out->abi_version = P.v3 ? gpub::kCommitReceiptV3Abi : gpub::kCommitReceiptAbi;
    memcpy(receipt_out->proposal_sha256, P.sha, 32);
    receipt_out->prepare_ack = *ack;
    memcpy(receipt_out->commit_sha256, commit_sha, 32);
  }
  P.active = false;
  return status;
}

}  // extern "C"

namespace {

// One LaneWeave wave (lane_weave_run_wave): the device step of the planned
// lanes runs privately, an optional sink acknowledges the wave's stages, then
// each quantum's row, sampler counter and output word publish under its
// service permit.
int lane_weave_wave_impl(glacier_hip_session *s, glacier_hip_lane_weave *lw,
                         const uint32_t *lane_of_slot, uint32_t slot_count,
                         uint32_t *tokens_by_lane, const uint64_t *eligible_by_lane,
                         uint32_t max_count, glacier_hip_wave_sink_fn sink, void *sink_ctx,
                         uint32_t *slots_out, glacier_hip_lane_event_t *events_out,
                         uint32_t *count_out) {
  if (!s || !lw || !lane_of_slot || !tokens_by_lane || !count_out)
    return GLACIER_HIP_INVALID_ARGUMENT;
  *count_out = 0;
  const uint32_t L = (uint32_t)s->lanes.size();
  if (max_count == 0 || max_count > L) return GLACIER_HIP_SHAPE_MISMATCH;
  const auto &c = s->model->cfg;
  const uint64_t W = (c.vocab_size + 63) / 64;
  GH_SUBMISSION(s->model->ctx);
  if (s->prep.active) return GLACIER_HIP_TRANSACTION_ACTIVE;
  std::vector<uint32_t> lanes, toks, next, slots;
  std::vector<RowTxn> txns;
  std::vector<uint8_t> published;
  const bool elig = eligible_by_lane != nullptr;
  gh::WaveOps ops;
  ops.run = [&](const uint32_t *plan, uint32_t n) -> int {
    lanes.resize(n);
    toks.resize(n);
    next.assign(n, 0);
    slots.assign(plan, plan + n);
    for (uint32_t i = 0; i < n; ++i) {
      if (plan[i] >= slot_count || lane_of_slot[plan[i]] >= L) return GLACIER_HIP_SHAPE_MISMATCH;
      lanes[i] = lane_of_slot[plan[i]];
      toks[i] = tokens_by_lane[lanes[i]];
      const Lane &ln = s->lanes[lanes[i]];
      if (!ln.kv.active) return GLACIER_HIP_INVALID_ARGUMENT;
      for (uint32_t j = 0; j < i; ++j)
        if (lanes[j] == lanes[i]) return GLACIER_HIP_INVALID_ARGUMENT;
      if (toks[i] >= c.vocab_size) return GLACIER_HIP_SHAPE_MISMATCH;
      if (ln.kv.len + 1 > s->opt.max_positions) return GLACIER_HIP_CACHE_FULL;
      if (ln.first_pending || ln.retired) return GLACIER_HIP_INVALID_TRANSACTION;
    }
    std::vector<uint64_t> words;
    if (elig) {
      words.resize((size_t)n * W);
      for (uint32_t i = 0; i < n; ++i)
        memcpy(&words[(size_t)i * W], eligible_by_lane + (size_t)lanes[i] * W, W * 8);
    }
    const int rc = run_step(s, lanes.data(), toks.data(), n, true, elig ? words.data() : nullptr,
                            nullptr, txns);
    if (rc) return rc;  // run_step aborted its rows
    for (uint32_t i = 0; i < n; ++i) next[i] = (uint32_t)s->res_host[i].index;
    published.assign(n, 0);
    return GLACIER_HIP_OK;
  };
  if (sink) {
    ops.sink = [&]() -> int {
      std::vector<std::array<uint8_t, 32>> digests;
      if (int rc = row_payload_sha256(s, txns, digests)) return rc;
      std::vector<glacier_hip_wave_stage_v1_t> stages(lanes.size());
      for (size_t i = 0; i < lanes.size(); ++i) {
        glacier_hip_wave_stage_v1_t &w = stages[i];
        memset(&w, 0, sizeof w);
        w.slot = slots[i];
        w.lane = lanes[i];
        const Lane &ln = s->lanes[lanes[i]];
        glacier_hip_lane_proposal_v1_t &lp = w.stage;
        gpub::empty_transition(lp.kv_transition);
        const RowTxn &rt = txns[i];
        glacier_hip_root_transition_v1_t &t = lp.kv_transition;
        lp.lane_index = (uint32_t)i;
        lp.step_index = ln.output.size();
        lp.prompt_len = ln.prompt_len;
        lp.kv_capacity_bytes = lane_capacity_bytes(s);
        lp.has_kv_transition = 1;
        lp.kv_before = rt.mark.base_len;
        lp.kv_after = rt.mark.base_len + 1;
        t.cache_instance = rt.mark.cache_instance;
        t.row_txn_generation = rt.mark.generation;
        copy_root(rt.before, t, true);
        copy_root(rt.after, t, false);
        t.logical_page = rt.mark.page_ref.logical_page;
        t.page_ownership_generation = rt.mark.page_ref.ownership_generation;
        t.installs_new_page = rt.installs ? 1 : 0;
        memcpy(t.row_payload_sha256, digests[i].data(), 32);
        if (ln.chain_init) {
          memcpy(t.state_chain_before, ln.chain, 32);
          gpub::appended_state_chain(ln.chain, rt.before, rt.after, rt.mark, digests[i].data(),
                                     t.state_chain_after);
        }
        lp.output_before = ln.output.size();
        lp.output_after = ln.output.size() + 1;
        memcpy(lp.rng_before, ln.rng, sizeof ln.rng);
        memcpy(lp.rng_after, ln.rng, sizeof ln.rng);  // greedy: the RNG never advances
        lp.sampling_calls_before = ln.sampling_calls;
        lp.sampling_calls_after = ln.sampling_calls + (elig ? 0 : 1);
        lp.token_id = next[i];
      }
      return sink(sink_ctx, stages.data(), (uint32_t)stages.size()) ? GLACIER_HIP_SINK_REJECTED
                                                                     : GLACIER_HIP_OK;
    };
  }
  ops.publish = [&](uint32_t i) -> int {
    // this quantum's KV row (root + length), sampler counter and output word
    Lane &ln = s->lanes[lanes[i]];
    if (ln.lease) ln.lease->lease.end_rows();
    if (int rc = ln.kv.commit(&txns[i], 1)) return rc;
    published[i] = 1;
    // the eligible (posthead) branch does not count a sampler call
    // (generate.zig:5574-5598); the greedy sampler does (:5593)
    if (!elig) ln.sampling_calls += 1;
    ln.output.push_back(next[i]);
    tokens_by_lane[lanes[i]] = next[i];
    return GLACIER_HIP_OK;
  };
  ops.abort = [&](uint32_t from) {
    for (uint32_t i = from; i < (uint32_t)txns.size(); ++i) {
      if (published[i]) continue;
      Lane &ln = s->lanes[lanes[i]];
      if (ln.lease) ln.lease->lease.end_rows();
      (void)ln.kv.abort(&txns[i], 1);
    }
  };
  return gh::lane_weave_run_wave(lw, max_count, ops, slots_out, events_out, count_out);
}

}  // namespace

extern "C" int glacier_hip_session_lane_weave_wave(
    glacier_hip_session *s, glacier_hip_lane_weave *lw, const uint32_t *lane_of_slot,
    uint32_t slot_count, uint32_t *tokens_by_lane, const uint64_t *eligible_by_lane,
    uint32_t max_count, uint32_t *slots_out, glacier_hip_lane_event_t *events_out,
    uint32_t *count_out) {
  return lane_weave_wave_impl(s, lw, lane_of_slot, slot_count, tokens_by_lane, eligible_by_lane,
                              max_count, nullptr, nullptr, slots_out, events_out, count_out);
}

extern "C" int glacier_hip_session_lane_weave_wave_staged(
    glacier_hip_session *s, glacier_hip_lane_weave *lw, const uint32_t *lane_of_slot,
    uint32_t slot_count, uint32_t *tokens_by_lane, const uint64_t *eligible_by_lane,
    uint32_t max_count, glacier_hip_wave_sink_fn sink, void *sink_ctx, uint32_t *slots_out,
    glacier_hip_lane_event_t *events_out, uint32_t *count_out) {
  if (!sink) return GLACIER_HIP_INVALID_ARGUMENT;
  return lane_weave_wave_impl(s, lw, lane_of_slot, slot_count, tokens_by_lane, eligible_by_lane,
                              max_count, sink, sink_ctx, slots_out, events_out, count_out);
}

// ---------------------------------------------------------------------------
// Leased lanes (leased_paged_kv_cache.zig over a device session lane)
// ---------------------------------------------------------------------------
namespace {
void detach_lane(glacier_hip_leased_kv *c) {
  auto *s = (glacier_hip_session *)c->owner;
  if (!s || c->lane >= s->lanes.size()) return;
  Lane &ln = s->lanes[c->lane];
  if (ln.lease != c) return;
  PreparedWave &P = s->prep;
  if (P.active && std::find(P.lanes.begin(), P.lanes.end(), c->lane) != P.lanes.end()) {
    // the lane's coordinator goes away inside a prepared wave: the wave aborts
    if (!P.first) abort_rows(s, P.txns);
    if (P.cohort) (void)P.cohort->lease.bank->abort_publication(P.permit);
    P.cohort = nullptr;
    P.active = false;
  }
  ln.lease = nullptr;
  ln.kv.leased_instance = 0;  // the lane may start a new request
  ln.kv.leased_owner = 0;
}
}  // namespace

extern "C" int glacier_hip_leased_kv_create_for_lane(
    glacier_hip_lease_bank *b, glacier_hip_lease_tree_t *tree, const glacier_hip_lease_node_t *scope,
    glacier_hip_session *s, uint32_t lane, glacier_hip_page_lease_binding_t *bindings,
    uint32_t binding_count, uint64_t request_epoch, uint64_t session_id, uint64_t *sequence,
    glacier_hip_leased_kv **out) {
  if (!b || !tree || !scope || !s || !bindings || !sequence || !out || lane >= s->lanes.size())
    return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  GH_SUBMISSION(s->model->ctx);
  Lane &ln = s->lanes[lane];
  if (s->prep.active || ln.lease || !ln.kv.active) return GLACIER_HIP_LEASE_INVALID_COORDINATOR;
  auto *c = new (std::nothrow) glacier_hip_leased_kv();
  if (!c) return GLACIER_HIP_LEASE_INVALID_CONFIGURATION;
  glb::Target t;
  t.cache = &ln.kv;
  t.pool = &s->pool;
  t.kv_sha256 = [s, lane](uint8_t o[32]) {
    if (s->lanes[lane].kv.retired) return (int)GLACIER_HIP_LEASE_CACHE_RETIRED;
    return logical_kv_sha256(s, lane, o) ? (int)GLACIER_HIP_LEASE_DEVICE_ERROR
                                         : (int)GLACIER_HIP_LEASE_OK;
  };
  const int rc = c->lease.init(&b->bank, tree, *scope, t, bindings, binding_count, request_epoch,
                               session_id, sequence);
  if (rc) {
    delete c;
    return rc;
  }
  c->owner = s;
  c->lane = lane;
  c->detach = detach_lane;
  ln.lease = c;
  *out = c;
  return GLACIER_HIP_LEASE_OK;
}
