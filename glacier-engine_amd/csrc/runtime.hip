// runtime.hip — C ABI: context, buffers and allocation lease, device
// capability, persistent INT4 weights, and the stand-alone kernel entry
// points (GEMV, RMSNorm, paged attention, argmax). The model/session token
// loop lives in session.hip.
#include <math.h>
#include <cmath>
#include <string.h>

#include <algorithm>
#include <cstdio>

#include "host_util.h"
#include "runtime.h"

using gh::hip_fail;

// Scratch of glacier_hip_int4_gemv_noalloc: activation planes, then the
// GEMM's split-K partial sums. One array per GPU for the life of the
// process; host code reaches it only through the address
// hipGetSymbolAddress returns on that device (glacier_hip_init).
static constexpr size_t kNoAllocPlanesBytes = 4u << 20;
static constexpr size_t kNoAllocSplitkBytes = 12u << 20;
static constexpr uint32_t kNoAllocMaxRows = 64;
static __device__ __align__(256) uint8_t scratch[kNoAllocPlanesBytes + kNoAllocSplitkBytes];

namespace gh {

int hip_fail(glacier_hip_context *ctx, hipError_t e, const char *what) {
  if (ctx) {
    ctx->last_error = std::string(what) + ": " + hipGetErrorString(e);
  }
  // the failure is reported through the status code; clear the thread's last
  // error so that the launch checks (hipGetLastError) of later calls do not
  // report it again
  (void)hipGetLastError();
  if (e == hipErrorOutOfMemory) return GLACIER_HIP_OUT_OF_MEMORY;
  return GLACIER_HIP_DEVICE_ERROR;
}

hipError_t dev_malloc(glacier_hip_context *ctx, void **p, size_t bytes) {
  *p = nullptr;
  const hipError_t e = hipMalloc(p, bytes);
  if (e != hipSuccess) {
    *p = nullptr;
    (void)hipGetLastError();  // handled here: later launch checks must not see it
    return e;
  }
  std::lock_guard<std::mutex> lk(ctx->dev_mu);
  ctx->dev_allocs[*p] = bytes;
  ctx->dev_requested += bytes;
  ctx->dev_charged += charged_bytes(bytes);
  return hipSuccess;
}

void dev_free(glacier_hip_context *ctx, void *p) {
  if (!p) return;
  {
    std::lock_guard<std::mutex> lk(ctx->dev_mu);
    auto it = ctx->dev_allocs.find(p);
    if (it != ctx->dev_allocs.end()) {
      ctx->dev_requested -= it->second;
      ctx->dev_charged -= charged_bytes(it->second);
      ctx->dev_allocs.erase(it);
    }
  }
  (void)hipFree(p);
}

int resolve_activation(int activation, uint32_t out_f, uint32_t in_f) {
  if (activation == GLACIER_HIP_ACT_AUTO)
    // int4_matmul.zig:461-463 (vocabulary head) and :372-374 (wide input)
    return (out_f > 65536 || in_f > 16384) ? GLACIER_HIP_ACT_F32 : GLACIER_HIP_ACT_Q8;
  return activation;
}

void repack_tiles(const std::vector<RowSrc> &rows, uint32_t K, std::vector<uint32_t> &codes,
                  std::vector<uint16_t> &scales) {
  // Tile layout of kernels.h: lane 16*j + n holds group 4*kq + j of row n.
  const size_t N = rows.size();
  const size_t NB = N / 16, KQ = K / 128, G = K / 32;
  codes.assign(NB * KQ * 64 * 4, 0u);
  scales.assign(NB * KQ * 64, 0u);
  parallel_for(NB, [&](size_t b0, size_t b1) {
    for (size_t nb = b0; nb < b1; ++nb)
      for (int nl = 0; nl < 16; ++nl) {
        const RowSrc &src = rows[nb * 16 + nl];
        const uint8_t *rp = src.packed ? src.packed + src.row * (K / 2) : nullptr;
        for (size_t g = 0; g < G; ++g) {
          const size_t kq = g / 4, j = g % 4;
          const size_t lane = j * 16 + (size_t)nl;
          uint16_t sh = 0;
          if (src.scales_f16) sh = src.scales_f16[src.row * G + g];
          else if (src.scales_f32) sh = f32_to_f16(src.scales_f32[src.row * G + g]);
          scales[(nb * KQ + kq) * 64 + lane] = sh;
          for (int w = 0; w < 4; ++w) {
            uint32_t word = 0x77777777u;  // code 7 decodes to 0 for absent rows
            if (rp) {
              const uint8_t *b = rp + g * 16 + w * 4;  // columns 32g + 8w .. +8
              uint8_t code[8];
              for (int t = 0; t < 8; ++t) code[t] = (b[t / 2] >> (4 * (t & 1))) & 0xF;
              word = 0;
              for (int bb = 0; bb < 4; ++bb)
                word |= (uint32_t)(code[bb] | (code[bb + 4] << 4)) << (8 * bb);
            }
            codes[((nb * KQ + kq) * 64 + lane) * 4 + w] = word;
          }
        }
      }
  }, 4);
}

glacier_hip_int4_weight *upload_weight(glacier_hip_context *ctx, uint32_t out_f, uint32_t in_f,
                                       const std::vector<uint32_t> &codes,
                                       const std::vector<uint16_t> &scales) {
  auto *w = new glacier_hip_int4_weight();
  w->ctx = ctx;
  w->out_f = out_f;
  w->in_f = in_f;
  const size_t cb = codes.size() * 4, sb = scales.size() * 2;
  if (gh::dev_malloc(ctx, (void **)&w->codes, cb) != hipSuccess ||
      gh::dev_malloc(ctx, (void **)&w->scales, sb) != hipSuccess ||
      hipMemcpy(w->codes, codes.data(), cb, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(w->scales, scales.data(), sb, hipMemcpyHostToDevice) != hipSuccess) {
    ctx->last_error = "int4 weight upload failed";
    gh::dev_free(ctx, w->codes);
    gh::dev_free(ctx, w->scales);
    delete w;
    return nullptr;
  }
  w->device_bytes = cb + sb;
  ctx->live_weights++;
  return w;
}

int ensure_scratch(glacier_hip_context *ctx, glacier_hip_context::StreamScratch &ss, size_t bytes,
                   size_t counters) {
  if (bytes > ss.scratch_bytes) {
    gh::dev_free(ctx, ss.scratch);
    ss.scratch = nullptr;
    ss.scratch_bytes = 0;
    GH_CHECK(ctx, gh::dev_malloc(ctx, &ss.scratch, bytes));
    ss.scratch_bytes = bytes;
  }
  if (counters > ss.counter_count) {
    gh::dev_free(ctx, ss.counters);
    ss.counters = nullptr;
    ss.counter_count = 0;
    GH_CHECK(ctx, gh::dev_malloc(ctx, (void **)&ss.counters, counters * sizeof(uint32_t)));
    GH_CHECK(ctx, hipMemset(ss.counters, 0, counters * sizeof(uint32_t)));
    ss.counter_count = counters;
  }
  return GLACIER_HIP_OK;
}

}  // namespace gh

extern "C" {

uint64_t glacier_hip_abi_version(void) { return 0x4748495000000001ull; }

static std::string g_init_error;

glacier_hip_context *glacier_hip_init(int device_ordinal) {
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || device_ordinal < 0 || device_ordinal >= count) {
    g_init_error = std::string("hipGetDeviceCount: ") + hipGetErrorString(e) +
                   " count=" + std::to_string(count);
    return nullptr;
  }
  if ((e = hipSetDevice(device_ordinal)) != hipSuccess) {
    g_init_error = std::string("hipSetDevice: ") + hipGetErrorString(e);
    return nullptr;
  }
  auto *ctx = new glacier_hip_context();
  ctx->device = device_ordinal;
  const char *what = "hipGetDeviceProperties";
  e = hipGetDeviceProperties(&ctx->props, device_ordinal);
  if (e == hipSuccess) {
    what = "hipStreamCreateWithFlags";
    e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  }
  if (e == hipSuccess) {
    what = "hipHostMalloc";
    e = hipHostMalloc((void **)&ctx->results_host, sizeof(gk::ArgmaxResult) * 64);
  }
  if (e == hipSuccess) {
    // the no-allocation GEMV's scratch on this (current) device
    static std::mutex sym_mu;
    static void *sym_ptr[64] = {};
    std::lock_guard<std::mutex> lk(sym_mu);
    if (device_ordinal < 64 && !sym_ptr[device_ordinal]) {
      void *p = nullptr;
      if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) == hipSuccess) sym_ptr[device_ordinal] = p;
      else (void)hipGetLastError();  // reported by the entry point
    }
    if (device_ordinal < 64) ctx->noalloc_scratch = sym_ptr[device_ordinal];
  }
  if (e == hipSuccess) {
    what = "identity rows";
    int32_t h[64];
    for (int i = 0; i < 64; ++i) h[i] = i;
    e = gh::dev_malloc(ctx, (void **)&ctx->ident, sizeof h);
    if (e == hipSuccess) e = hipMemcpy(ctx->ident, h, sizeof h, hipMemcpyHostToDevice);
  }
  if (e != hipSuccess) {
    g_init_error = std::string(what) + ": " + hipGetErrorString(e);
    delete ctx;
    return nullptr;
  }
  static uint64_t epoch_counter = 0x6c61636965720000ull;
  ctx->epoch = ++epoch_counter;
  {  // command tokens carry a nonce of this context
    gh::Sha256 h;
    h.update("glacier-hip-command-nonce-v1", 28);
    h.u64(ctx->epoch);
    h.u64((uint64_t)(uintptr_t)ctx);
    h.u64((uint64_t)device_ordinal);
    uint8_t d[32];
    h.final(d);
    memcpy(ctx->nonce, d, 32);
  }
  if (hipEventCreate(&ctx->origin) != hipSuccess ||
      hipEventRecord(ctx->origin, ctx->stream) != hipSuccess) {
    g_init_error = "origin event";
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return nullptr;
  }
  return ctx;
}

int glacier_hip_deinit(glacier_hip_context *ctx) {
  if (!ctx) return GLACIER_HIP_INVALID_HANDLE;
  if (!ctx->buffers.empty() || ctx->live_weights != 0 || !ctx->commands.empty())
    return GLACIER_HIP_BUSY;
  (void)hipDeviceSynchronize();
  for (auto &kv : ctx->per_stream) {
    auto &ss = kv.second;
    gh::dev_free(ctx, ss.scratch);
    gh::dev_free(ctx, ss.planes);
    gh::dev_free(ctx, ss.splitk);
    gh::dev_free(ctx, ss.counters);
  }
  if (ctx->results_host) (void)hipHostFree(ctx->results_host);
  gh::dev_free(ctx, ctx->ident);
  if (ctx->origin) (void)hipEventDestroy(ctx->origin);
  (void)hipStreamDestroy(ctx->stream);
  delete ctx;
  return GLACIER_HIP_OK;
}

const char *glacier_hip_last_error(glacier_hip_context *ctx) {
  return ctx ? ctx->last_error.c_str() : g_init_error.c_str();
}

int glacier_hip_synchronize(glacier_hip_context *ctx) {
  if (!ctx) return GLACIER_HIP_INVALID_HANDLE;
  GH_CHECK(ctx, hipStreamSynchronize(ctx->stream));
  return GLACIER_HIP_OK;
}

int glacier_hip_device_info(glacier_hip_context *ctx, glacier_hip_device_info_t *out) {
  if (!ctx || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  memset(out, 0, sizeof *out);
  const hipDeviceProp_t &p = ctx->props;
  snprintf(out->name, sizeof out->name, "%s", p.name);
  snprintf(out->arch, sizeof out->arch, "%s", p.gcnArchName);
  out->compute_units = (uint32_t)p.multiProcessorCount;
  out->wavefront_size = (uint32_t)p.warpSize;
  out->total_global_bytes = p.totalGlobalMem;
  out->max_single_allocation_bytes = p.totalGlobalMem;
  out->lds_bytes_per_block = (uint32_t)p.sharedMemPerBlock;
  out->l2_bytes = (uint32_t)p.l2CacheSize;
  out->clock_khz = (uint32_t)p.clockRate;
  out->memory_clock_khz = (uint32_t)p.memoryClockRate;
  out->memory_bus_width_bits = (uint32_t)p.memoryBusWidth;
  out->device_ordinal = (uint32_t)ctx->device;
  return GLACIER_HIP_OK;
}

using gh::kGranularity;
static uint64_t charged_size(uint64_t requested) { return gh::charged_bytes(requested); }

int glacier_hip_live_device_bytes(glacier_hip_context *ctx, uint64_t *requested_out,
                                  uint64_t *charged_out) {
  if (!ctx) return GLACIER_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lk(ctx->dev_mu);
  if (requested_out) *requested_out = ctx->dev_requested;
  if (charged_out) *charged_out = ctx->dev_charged;
  return GLACIER_HIP_OK;
}

int glacier_hip_allocation_limits(glacier_hip_context *ctx, glacier_hip_allocation_limits_t *out) {
  if (!ctx || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  out->max_single_allocation_bytes = ctx->props.totalGlobalMem;
  out->max_total_device_bytes = ctx->props.totalGlobalMem;
  out->allocation_granularity_bytes = kGranularity;
  out->max_queue_slots = 1;
  return GLACIER_HIP_OK;
}

// device_capability_contract.zig:331-350 capabilityRootV1
static void capability_root(const glacier_hip_device_capability_v1_t &c, uint8_t out[32]) {
  gh::Sha256 h;
  h.update("glacier-device-capability-v1\0", 29);
  h.u64(c.abi_version);
  h.u64(c.backend_kind);
  h.u64(c.device_class);
  h.u64(c.operation_profile_bits);
  h.u64(c.operator_bits);
  h.u64(c.element_type_bits);
  h.u64(c.numerical_policy_bits);
  h.u64(c.feature_bits);
  h.u64(c.max_single_allocation_bytes);
  h.u64(c.max_total_device_bytes);
  h.u64(c.max_queue_slots);
  h.update(c.backend_sha256, 32);
  h.update(c.device_sha256, 32);
  h.update(c.driver_sha256, 32);
  h.update(c.placement_sha256, 32);
  h.final(out);
}

int glacier_hip_device_capability_v1(glacier_hip_context *ctx,
                                     glacier_hip_device_capability_v1_t *out) {
  if (!ctx || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  memset(out, 0, sizeof *out);
  out->abi_version = 0x4744434100000001ull;
  out->backend_kind = 3;  // portable_compute
  out->device_class = 2;  // accelerator
  // matvec_int4_f32_bounded profile: operator matvec_int4_f32, element
  // types packed_int4 + float32, numerical policy bounded_float32.
  out->operation_profile_bits = 1ull << 2;
  out->operator_bits = 1ull << 2;
  out->element_type_bits = (1ull << 0) | (1ull << 2);
  out->numerical_policy_bits = 1ull << 1;
  // allocation | dispatch | completion_fence | persistent_weights
  out->feature_bits = (1ull << 0) | (1ull << 1) | (1ull << 2) | (1ull << 3) | (1ull << 4) |
                     (1ull << 5);  // allocation, dispatch, completion fence, persistent
                                   // weights, command GPU times, allocated bytes
  out->max_single_allocation_bytes = ctx->props.totalGlobalMem;
  out->max_total_device_bytes = ctx->props.totalGlobalMem;
  out->max_queue_slots = 1;
  {
    gh::Sha256 h;
    h.update("glacier-hip-backend-gfx950-v1", 29);
    h.final(out->backend_sha256);
  }
  {
    gh::Sha256 h;
    h.update(ctx->props.name, strnlen(ctx->props.name, sizeof ctx->props.name));
    h.update(ctx->props.gcnArchName, strnlen(ctx->props.gcnArchName, sizeof ctx->props.gcnArchName));
    h.u64((uint64_t)ctx->props.multiProcessorCount);
    h.u64((uint64_t)ctx->props.totalGlobalMem);
    h.final(out->device_sha256);
  }
  {
    int rt = 0, drv = 0;
    (void)hipRuntimeGetVersion(&rt);
    (void)hipDriverGetVersion(&drv);
    gh::Sha256 h;
    h.u64((uint64_t)rt);
    h.u64((uint64_t)drv);
    h.final(out->driver_sha256);
  }
  {
    gh::Sha256 h;
    h.update("hip-device-ordinal", 18);
    h.u64((uint64_t)ctx->device);
    h.u64((uint64_t)ctx->props.pciBusID);
    h.final(out->placement_sha256);
  }
  capability_root(*out, out->capability_sha256);
  return GLACIER_HIP_OK;
}

int glacier_hip_buffer_create(glacier_hip_context *ctx, uint64_t requested_length,
                              glacier_hip_buffer_token_t *out) {
  glacier_hip_allocation_quote_t q;
  int rc = glacier_hip_allocation_quote(ctx, requested_length, &q);
  if (rc) return rc;
  return glacier_hip_allocation_allocate(ctx, &q, out);
}

int glacier_hip_allocation_quote(glacier_hip_context *ctx, uint64_t requested_bytes,
                                 glacier_hip_allocation_quote_t *out) {
  if (!ctx || !out || requested_bytes == 0) return GLACIER_HIP_INVALID_ARGUMENT;
  if (requested_bytes > ctx->props.totalGlobalMem) return GLACIER_HIP_OUT_OF_MEMORY;
  out->requested_bytes = requested_bytes;
  out->charged_bytes = charged_size(requested_bytes);
  out->context_epoch = ctx->epoch;
  return GLACIER_HIP_OK;
}

int glacier_hip_allocation_allocate(glacier_hip_context *ctx,
                                    const glacier_hip_allocation_quote_t *quote,
                                    glacier_hip_buffer_token_t *out) {
  if (!ctx || !quote || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  if (quote->context_epoch != ctx->epoch || quote->requested_bytes == 0 ||
      quote->charged_bytes != charged_size(quote->requested_bytes))
    return GLACIER_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lk(ctx->buf_mu);
  void *p = nullptr;
  hipError_t e = gh::dev_malloc(ctx, &p, quote->requested_bytes);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipMalloc");  // nothing was created
  const uint64_t id = ctx->next_buffer_id++;
  ctx->buffers[id] = {p, quote->requested_bytes, quote->charged_bytes};
  out->id = id;
  out->requested_bytes = quote->requested_bytes;
  out->charged_bytes = quote->charged_bytes;
  return GLACIER_HIP_OK;
}

int glacier_hip_allocation_free(glacier_hip_context *ctx, const glacier_hip_buffer_token_t *token) {
  return glacier_hip_buffer_release(ctx, token);
}

int glacier_hip_buffer_info(glacier_hip_context *ctx, const glacier_hip_buffer_token_t *token,
                            glacier_hip_buffer_info_t *out) {
  if (!ctx || !token || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lk(ctx->buf_mu);
  auto it = ctx->buffers.find(token->id);
  if (it == ctx->buffers.end() || it->second.requested != token->requested_bytes)
    return GLACIER_HIP_INVALID_HANDLE;
  out->id = token->id;
  out->requested_bytes = it->second.requested;
  out->charged_bytes = it->second.charged;
  out->device_address = (uint64_t)(uintptr_t)it->second.ptr;
  return GLACIER_HIP_OK;
}

int glacier_hip_buffer_release(glacier_hip_context *ctx, const glacier_hip_buffer_token_t *token) {
  if (!ctx || !token) return GLACIER_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lk(ctx->buf_mu);
  auto it = ctx->buffers.find(token->id);
  if (it == ctx->buffers.end() || it->second.requested != token->requested_bytes)
    return GLACIER_HIP_INVALID_HANDLE;
  for (const auto &kv : ctx->commands)  // a live command still uses it
    for (uint64_t id : kv.second.buf)
      if (id == token->id) return GLACIER_HIP_BUSY;
  gh::dev_free(ctx, it->second.ptr);
  ctx->buffers.erase(it);
  return GLACIER_HIP_OK;
}

int glacier_hip_live_buffer_count(glacier_hip_context *ctx, uint64_t *out) {
  if (!ctx || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lk(ctx->buf_mu);
  *out = ctx->buffers.size();
  return GLACIER_HIP_OK;
}

int glacier_hip_live_weight_count(glacier_hip_context *ctx, uint64_t *out) {
  if (!ctx || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  *out = ctx->live_weights;
  return GLACIER_HIP_OK;
}

// ---- INT4 weights ---------------------------------------------------------
static glacier_hip_int4_weight *weight_create(glacier_hip_context *ctx, const uint8_t *packed,
                                              uint64_t packed_bytes, const float *s32,
                                              const uint16_t *s16, uint64_t scale_count,
                                              uint32_t group, uint32_t in_f, uint32_t out_f) {
  if (!ctx || !packed || (!s32 && !s16)) return nullptr;
  if (group != 32 || out_f == 0 || in_f == 0 || out_f % 16 != 0 || in_f % 128 != 0) {
    ctx->last_error = "int4 weight: need group 32, out_f % 16 == 0, in_f % 128 == 0";
    return nullptr;
  }
  const uint64_t n = (uint64_t)out_f * in_f;
  if (packed_bytes < n / 2 || scale_count < n / group) {
    ctx->last_error = "int4 weight: truncated packed bytes or scales";
    return nullptr;
  }
  std::vector<gh::RowSrc> rows(out_f);
  for (uint32_t r = 0; r < out_f; ++r) rows[r] = {packed, s32, s16, r};
  std::vector<uint32_t> codes;
  std::vector<uint16_t> scales;
  gh::repack_tiles(rows, in_f, codes, scales);
  auto *w = gh::upload_weight(ctx, out_f, in_f, codes, scales);
  if (w) w->group = group;
  return w;
}

glacier_hip_int4_weight *glacier_hip_int4_weight_create(glacier_hip_context *ctx,
                                                        const uint8_t *packed,
                                                        uint64_t packed_bytes,
                                                        const float *scales, uint64_t scale_count,
                                                        uint32_t group_size, uint32_t in_features,
                                                        uint32_t out_features) {
  return weight_create(ctx, packed, packed_bytes, scales, nullptr, scale_count, group_size,
                       in_features, out_features);
}

glacier_hip_int4_weight *glacier_hip_int4_weight_create_f16scales(
    glacier_hip_context *ctx, const uint8_t *packed, uint64_t packed_bytes,
    const uint16_t *scales_f16, uint64_t scale_count, uint32_t group_size, uint32_t in_features,
    uint32_t out_features) {
  return weight_create(ctx, packed, packed_bytes, nullptr, scales_f16, scale_count, group_size,
                       in_features, out_features);
}

void glacier_hip_int4_weight_destroy(glacier_hip_int4_weight *w) {
  if (!w) return;
  gh::dev_free(w->ctx, w->codes);
  gh::dev_free(w->ctx, w->scales);
  if (w->ctx && w->ctx->live_weights) w->ctx->live_weights--;
  delete w;
}

uint64_t glacier_hip_int4_weight_device_bytes(const glacier_hip_int4_weight *w) {
  return w ? w->device_bytes : 0;
}

// Activation planes: int8 [G][D][m][32] followed (256-aligned) by ActMeta [G][m].
static size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }
static size_t planes_q_bytes(uint32_t m, uint32_t in_f, int D) { return (size_t)(in_f / 32) * D * m * 32; }
static size_t planes_bytes(uint32_t m, uint32_t in_f, int D) {
  return al256(planes_q_bytes(m, in_f, D)) + (size_t)(in_f / 32) * m * sizeof(gk::ActMeta);
}

static int act_digits(int activation) {
  if (activation == GLACIER_HIP_ACT_Q8) return 1;
  if (activation == GLACIER_HIP_ACT_F32) return 3;
  return 0;
}

// ws == null: the stream's split-K workspace, grown on demand; else the
// caller's (ws_floats floats; a smaller workspace only lowers the K split).
static int gemv_launch(glacier_hip_context *ctx, glacier_hip_int4_weight *w, const void *planes,
                       uint32_t m, int D, const float *bias_dev, float *y_dev, hipStream_t st,
                       float *ws = nullptr, size_t ws_floats = 0) {
  const int N = (int)w->out_f, K = (int)w->in_f;
  gk::GemvArgs a{};
  a.codes = w->codes;
  a.scales = w->scales;
  a.N = N;
  a.K = K;
  a.act_q = (const int8_t *)planes;
  a.act_meta = (const gk::ActMeta *)((const char *)planes + al256(planes_q_bytes(m, (uint32_t)K, D)));
  a.M = (int)m;
  a.D = D;
  a.bias = bias_dev;
  a.y = y_dev;
  a.epi = gk::EPI_PLAIN;
  // up to kGemvMaxRows rows: the decode GEMV (K1); more: the MFMA GEMM (K2),
  // with a workspace for its K split (grown on demand, capped at 64 MiB;
  // a smaller one only lowers the split)
  if (m <= (uint32_t)gk::kGemvMaxRows) {
    GH_CHECK(ctx, gk::launch_gemv(a, st));
    return GLACIER_HIP_OK;
  }
  if (ws) {
    a.splitk_ws = ws;
    a.splitk_ws_floats = ws_floats;
  } else {
    auto &ss = ctx->per_stream[st];
    const size_t need = std::min<size_t>(gk::gemm_splitk_floats(N, (int)m, K, D), 16u << 20);
    if (need > ss.splitk_floats) {
      gh::dev_free(ctx, ss.splitk);
      ss.splitk = nullptr;
      ss.splitk_floats = 0;
      GH_CHECK(ctx, gh::dev_malloc(ctx, (void **)&ss.splitk, need * sizeof(float)));
      ss.splitk_floats = need;
    }
    a.splitk_ws = ss.splitk;
    a.splitk_ws_floats = ss.splitk_floats;
  }
  GH_CHECK(ctx, gk::launch_gemm(a, st));
  return GLACIER_HIP_OK;
}

static int prepare_launch(glacier_hip_context *ctx, const void *x_dev, int x_dtype, uint32_t m,
                          uint32_t in_f, int D, void *planes, hipStream_t st) {
  GH_CHECK(ctx, gk::launch_prep_act(x_dev, x_dtype == GLACIER_HIP_BF16, nullptr, 0.0f, (int)m,
                                    (int)in_f, D, (int8_t *)planes,
                                    (gk::ActMeta *)((char *)planes + al256(planes_q_bytes(m, in_f, D))),
                                    nullptr, st));
  return GLACIER_HIP_OK;
}

static int gemv_common(glacier_hip_context *ctx, glacier_hip_int4_weight *w, const void *x_dev,
                       int x_dtype, uint32_t m, const float *bias_dev, float *y_dev,
                       int activation, hipStream_t st) {
  if (!ctx || !w || !x_dev || !y_dev) return GLACIER_HIP_INVALID_ARGUMENT;
  if (w->ctx != ctx) return GLACIER_HIP_INVALID_HANDLE;
  if (m == 0 || m > GLACIER_HIP_MAX_ROWS) return GLACIER_HIP_SHAPE_MISMATCH;
  if (x_dtype != GLACIER_HIP_F32 && x_dtype != GLACIER_HIP_BF16) return GLACIER_HIP_DTYPE_UNSUPPORTED;
  const int D = act_digits(gh::resolve_activation(activation, w->out_f, w->in_f));
  if (!D) return GLACIER_HIP_INVALID_ARGUMENT;
  auto &ss = ctx->per_stream[st];
  const size_t pb = planes_bytes(m, w->in_f, D);
  if (pb > ss.planes_bytes) {
    gh::dev_free(ctx, ss.planes);
    ss.planes = nullptr;
    ss.planes_bytes = 0;
    GH_CHECK(ctx, gh::dev_malloc(ctx, &ss.planes, pb));
    ss.planes_bytes = pb;
  }
  int rc = prepare_launch(ctx, x_dev, x_dtype, m, w->in_f, D, ss.planes, st);
  if (rc) return rc;
  return gemv_launch(ctx, w, ss.planes, m, D, bias_dev, y_dev, st);
}

int glacier_hip_int4_gemv(glacier_hip_context *ctx, glacier_hip_int4_weight *w, const void *x_dev,
                          int x_dtype, uint32_t m, const float *bias_dev, float *y_dev,
                          int activation, void *stream) {
  if (!ctx) return GLACIER_HIP_INVALID_HANDLE;
  GH_SUBMISSION(ctx);
  return gemv_common(ctx, w, x_dev, x_dtype, m, bias_dev, y_dev, activation,
                     stream ? (hipStream_t)stream : ctx->stream);
}

int glacier_hip_int4_gemv_noalloc(glacier_hip_context *ctx, glacier_hip_int4_weight *w,
                                  const void *x_dev, int x_dtype, uint32_t m, const float *bias_dev,
                                  float *y_dev, int activation, void *stream) {
  if (!ctx) return GLACIER_HIP_INVALID_HANDLE;
  if (!w || !x_dev || !y_dev) return GLACIER_HIP_INVALID_ARGUMENT;
  if (w->ctx != ctx) return GLACIER_HIP_INVALID_HANDLE;
  if (x_dtype != GLACIER_HIP_F32 && x_dtype != GLACIER_HIP_BF16) return GLACIER_HIP_DTYPE_UNSUPPORTED;
  const int D = act_digits(gh::resolve_activation(activation, w->out_f, w->in_f));
  if (!D) return GLACIER_HIP_INVALID_ARGUMENT;
  GH_SUBMISSION(ctx);
  if (m == 0 || m > kNoAllocMaxRows || planes_bytes(m, w->in_f, D) > kNoAllocPlanesBytes) {
    ctx->last_error = "int4_gemv_noalloc: more rows than its fixed scratch holds (at most 64 "
                      "rows and 4 MiB of activation planes)";
    return GLACIER_HIP_SHAPE_MISMATCH;
  }
  if (!ctx->noalloc_scratch) {
    ctx->last_error = "int4_gemv_noalloc: no scratch address on this device";
    return GLACIER_HIP_DEVICE_ERROR;
  }
  hipStream_t st = stream ? (hipStream_t)stream : ctx->stream;
  uint8_t *planes = (uint8_t *)ctx->noalloc_scratch;
  int rc = prepare_launch(ctx, x_dev, x_dtype, m, w->in_f, D, planes, st);
  if (rc) return rc;
  return gemv_launch(ctx, w, planes, m, D, bias_dev, y_dev, st,
                     (float *)(planes + kNoAllocPlanesBytes), kNoAllocSplitkBytes / sizeof(float));
}

uint64_t glacier_hip_activation_bytes(uint32_t m, uint32_t in_f, int activation) {
  const int D = act_digits(activation);
  if (!D || in_f % 128 != 0 || m == 0) return 0;
  return planes_bytes(m, in_f, D);
}

int glacier_hip_activation_prepare(glacier_hip_context *ctx, const void *x_dev, int x_dtype,
                                   uint32_t m, uint32_t in_f, int activation, void *act_dev,
                                   void *stream) {
  if (!ctx || !x_dev || !act_dev) return GLACIER_HIP_INVALID_ARGUMENT;
  const int D = act_digits(activation);
  if (!D) return GLACIER_HIP_INVALID_ARGUMENT;
  if (m == 0 || m > GLACIER_HIP_MAX_ROWS || in_f == 0 || in_f % 128 != 0) return GLACIER_HIP_SHAPE_MISMATCH;
  if (x_dtype != GLACIER_HIP_F32 && x_dtype != GLACIER_HIP_BF16) return GLACIER_HIP_DTYPE_UNSUPPORTED;
  GH_SUBMISSION(ctx);
  return prepare_launch(ctx, x_dev, x_dtype, m, in_f, D, act_dev,
                        stream ? (hipStream_t)stream : ctx->stream);
}

int glacier_hip_int4_gemv_prepared(glacier_hip_context *ctx, glacier_hip_int4_weight *w,
                                   const void *act_dev, uint32_t m, int activation,
                                   const float *bias_dev, float *y_dev, void *stream) {
  if (!ctx || !w || !act_dev || !y_dev) return GLACIER_HIP_INVALID_ARGUMENT;
  if (w->ctx != ctx) return GLACIER_HIP_INVALID_HANDLE;
  const int D = act_digits(activation);
  if (!D) return GLACIER_HIP_INVALID_ARGUMENT;
  if (m == 0 || m > GLACIER_HIP_MAX_ROWS) return GLACIER_HIP_SHAPE_MISMATCH;
  GH_SUBMISSION(ctx);
  return gemv_launch(ctx, w, act_dev, m, D, bias_dev, y_dev,
                     stream ? (hipStream_t)stream : ctx->stream);
}

int glacier_hip_int4_matvec_dispatch(glacier_hip_context *ctx, glacier_hip_int4_weight *w,
                                     const float *input, uint64_t input_count, float *output,
                                     uint64_t output_count) {
  if (!ctx || !w || !input || !output) return GLACIER_HIP_INVALID_ARGUMENT;
  if (input_count != w->in_f || output_count != w->out_f) return GLACIER_HIP_SHAPE_MISMATCH;
  GH_SUBMISSION(ctx);
  float *xd = nullptr, *yd = nullptr;
  GH_CHECK(ctx, gh::dev_malloc(ctx, (void **)&xd, input_count * 4));
  hipError_t e = gh::dev_malloc(ctx, (void **)&yd, output_count * 4);
  if (e != hipSuccess) {
    gh::dev_free(ctx, xd);
    return hip_fail(ctx, e, "hipMalloc");
  }
  int rc = GLACIER_HIP_OK;
  e = hipMemcpyAsync(xd, input, input_count * 4, hipMemcpyHostToDevice, ctx->stream);
  if (e != hipSuccess) rc = hip_fail(ctx, e, "copy in");
  if (!rc) rc = gemv_common(ctx, w, xd, GLACIER_HIP_F32, 1, nullptr, yd, GLACIER_HIP_ACT_F32, ctx->stream);
  if (!rc) {
    e = hipMemcpyAsync(output, yd, output_count * 4, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) rc = hip_fail(ctx, e, "copy out");
  }
  gh::dev_free(ctx, xd);
  gh::dev_free(ctx, yd);
  return rc;
}

// ---- asynchronous registered-buffer dispatch --------------------------------
static const uint64_t kAsyncSubmissionAbi = 0x474d415300000001ull;  // backend.zig:26
static const uint64_t kAsyncCompletionAbi = 0x474d414300000001ull;  // backend.zig:27

static bool binding_zero(const uint8_t b[32]) {
  for (int i = 0; i < 32; ++i)
    if (b[i]) return false;
  return true;
}

static uint64_t live_buffer_bytes(const glacier_hip_context *ctx) {
  uint64_t n = 0;
  for (const auto &kv : ctx->buffers) n += kv.second.charged;
  return n;
}

// The command of `token` + `binding` (held under ctx->buf_mu), or null.
static glacier_hip_context::AsyncCmd *find_command(glacier_hip_context *ctx,
                                                   const glacier_hip_command_token_t *t,
                                                   const uint8_t binding[32]) {
  if (memcmp(t->context_nonce, ctx->nonce, sizeof ctx->nonce) != 0) return nullptr;
  auto it = ctx->commands.find(t->generation);
  if (it == ctx->commands.end() || memcmp(it->second.binding, binding, 32) != 0) return nullptr;
  return &it->second;
}

// The completion record of a command; once the command has ended the record
// is fixed (every later poll returns the same bytes, as finalize compares).
static void completion_of(glacier_hip_context *ctx, uint64_t gen,
                          glacier_hip_context::AsyncCmd &c, bool wait,
                          glacier_hip_async_completion_t *out) {
  if (c.observed) {
    *out = c.final;
    return;
  }
  glacier_hip_async_completion_t r;
  memset(&r, 0, sizeof r);
  r.abi_version = kAsyncCompletionAbi;
  memcpy(r.token.context_nonce, ctx->nonce, sizeof ctx->nonce);
  r.token.generation = gen;
  memcpy(r.submission_binding, c.binding, 32);
  r.current_allocated_before = c.alloc_before;
  const hipError_t e = wait ? hipEventSynchronize(c.end) : hipEventQuery(c.end);
  if (e != hipSuccess) (void)hipGetLastError();  // reported in the record, not later
  if (e == hipErrorNotReady) {
    r.state = GLACIER_HIP_COMMAND_PENDING;
    r.current_allocated_after = c.alloc_before;
    *out = r;
    return;
  }
  r.current_allocated_after = live_buffer_bytes(ctx);
  if (e != hipSuccess) {
    r.state = GLACIER_HIP_COMMAND_ERROR;
    r.error_code = (int64_t)e;
    r.error_present = 1;
    r.error_domain_kind = 2;  // other
  } else {
    float ms0 = 0.0f, ms1 = 0.0f;
    if (hipEventElapsedTime(&ms0, ctx->origin, c.start) == hipSuccess &&
        hipEventElapsedTime(&ms1, ctx->origin, c.end) == hipSuccess) {
      r.gpu_start_time = ms0 * 1e-3;
      r.gpu_end_time = ms1 * 1e-3;
    }
    r.state = GLACIER_HIP_COMMAND_COMPLETED;
  }
  c.final = r;
  c.observed = true;
  *out = r;
}

int glacier_hip_int4_registered_buffers_submit_async(
    glacier_hip_context *ctx, const glacier_hip_buffer_token_t *ptok,
    const glacier_hip_buffer_token_t *stok, const glacier_hip_buffer_token_t *itok,
    const glacier_hip_buffer_token_t *otok, const uint8_t *packed, uint64_t packed_bytes,
    const float *scales, uint64_t scale_count, const float *input, uint64_t input_count,
    uint32_t group_size, uint32_t in_f, uint32_t out_f, const uint8_t binding[32],
    glacier_hip_async_submission_t *sub) {
  if (sub) {
    memset(sub, 0, sizeof *sub);
    sub->abi_version = kAsyncSubmissionAbi;
    sub->disposition = 2;  // submitted_or_ambiguous until the queue accepted it
  }
  if (!ctx || !ptok || !stok || !itok || !otok || !packed || !scales || !input || !binding ||
      !sub || binding_zero(binding))
    return GLACIER_HIP_INVALID_ARGUMENT;
  if (group_size != 32 || out_f == 0 || in_f == 0 || out_f % 16 || in_f % 128)
    return GLACIER_HIP_SHAPE_MISMATCH;
  const uint64_t n = (uint64_t)out_f * in_f;
  if (packed_bytes < n / 2 || scale_count < n / 32 || input_count != in_f)
    return GLACIER_HIP_SHAPE_MISMATCH;
  GH_SUBMISSION(ctx);
  std::lock_guard<std::mutex> bl(ctx->buf_mu);
  const glacier_hip_buffer_token_t *toks[4] = {ptok, stok, itok, otok};
  const uint64_t need[4] = {n / 2, scale_count * 4, (uint64_t)in_f * 4, (uint64_t)out_f * 4};
  void *ptr[4];
  for (int i = 0; i < 4; ++i) {
    auto it = ctx->buffers.find(toks[i]->id);
    if (it == ctx->buffers.end() || it->second.requested != toks[i]->requested_bytes)
      return GLACIER_HIP_INVALID_HANDLE;
    if (it->second.requested < need[i]) return GLACIER_HIP_SHAPE_MISMATCH;
    for (int j = 0; j < i; ++j)
      if (toks[j]->id == toks[i]->id) return GLACIER_HIP_INVALID_ARGUMENT;
    ptr[i] = it->second.ptr;
  }
  // the registered weight buffers receive the device tile layout (codes,
  // then fp16 scales: half the f32 scale buffer)
  std::vector<gh::RowSrc> rows(out_f);
  for (uint32_t r = 0; r < out_f; ++r) rows[r] = {packed, scales, nullptr, r};
  std::vector<uint32_t> codes;
  std::vector<uint16_t> sc16;
  gh::repack_tiles(rows, in_f, codes, sc16);
  GH_CHECK(ctx, hipMemcpy(ptr[0], codes.data(), codes.size() * 4, hipMemcpyHostToDevice));
  GH_CHECK(ctx, hipMemcpy(ptr[1], sc16.data(), sc16.size() * 2, hipMemcpyHostToDevice));
  GH_CHECK(ctx, hipMemcpy(ptr[2], input, (size_t)in_f * 4, hipMemcpyHostToDevice));
  glacier_hip_int4_weight view;
  view.ctx = ctx;
  view.out_f = out_f;
  view.in_f = in_f;
  view.codes = (uint4 *)ptr[0];
  view.scales = (uint2 *)ptr[1];
  glacier_hip_context::AsyncCmd c;
  memcpy(c.binding, binding, 32);
  for (int i = 0; i < 4; ++i) c.buf[i] = toks[i]->id;
  c.alloc_before = live_buffer_bytes(ctx);
  GH_CHECK(ctx, hipEventCreate(&c.start));
  hipError_t e = hipEventCreate(&c.end);
  if (e != hipSuccess) {
    (void)hipEventDestroy(c.start);
    return hip_fail(ctx, e, "hipEventCreate");
  }
  int rc = GLACIER_HIP_OK;
  if ((e = hipEventRecord(c.start, ctx->stream)) != hipSuccess) rc = hip_fail(ctx, e, "record");
  if (!rc) rc = gemv_common(ctx, &view, ptr[2], GLACIER_HIP_F32, 1, nullptr, (float *)ptr[3],
                            GLACIER_HIP_ACT_F32, ctx->stream);
  if (!rc && (e = hipEventRecord(c.end, ctx->stream)) != hipSuccess) rc = hip_fail(ctx, e, "record");
  if (rc) {  // nothing was queued that outlives this call
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipEventDestroy(c.start);
    (void)hipEventDestroy(c.end);
    return rc;
  }
  const uint64_t gen = ctx->next_command_generation++;
  ctx->commands[gen] = c;
  memcpy(sub->token.context_nonce, ctx->nonce, sizeof ctx->nonce);
  sub->token.generation = gen;
  memcpy(sub->submission_binding, binding, 32);
  sub->disposition = 1;  // submitted
  return GLACIER_HIP_OK;
}

static int poll_or_wait(glacier_hip_context *ctx, const glacier_hip_command_token_t *t,
                        const uint8_t binding[32], glacier_hip_async_completion_t *out, bool wait) {
  if (!ctx || !t || !binding || !out || t->generation == 0 || binding_zero(binding))
    return GLACIER_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> bl(ctx->buf_mu);
  auto *c = find_command(ctx, t, binding);
  if (!c) return GLACIER_HIP_INVALID_HANDLE;
  completion_of(ctx, t->generation, *c, wait, out);
  return GLACIER_HIP_OK;
}

int glacier_hip_registered_dispatch_poll(glacier_hip_context *ctx,
                                         const glacier_hip_command_token_t *t,
                                         const uint8_t binding[32],
                                         glacier_hip_async_completion_t *out) {
  return poll_or_wait(ctx, t, binding, out, false);
}

int glacier_hip_registered_dispatch_wait(glacier_hip_context *ctx,
                                         const glacier_hip_command_token_t *t,
                                         const uint8_t binding[32],
                                         glacier_hip_async_completion_t *out) {
  return poll_or_wait(ctx, t, binding, out, true);
}

static bool expected_ok(const glacier_hip_command_token_t *t, const uint8_t binding[32],
                        const glacier_hip_async_completion_t *x) {
  return x && x->abi_version == kAsyncCompletionAbi && x->reserved == 0 &&
         memcmp(&x->token, t, sizeof *t) == 0 && memcmp(x->submission_binding, binding, 32) == 0;
}

int glacier_hip_registered_dispatch_finalize(glacier_hip_context *ctx,
                                             const glacier_hip_command_token_t *t,
                                             const uint8_t binding[32],
                                             const glacier_hip_async_completion_t *expected) {
  if (!ctx || !t || !binding || t->generation == 0 || binding_zero(binding) ||
      !expected_ok(t, binding, expected))
    return GLACIER_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> bl(ctx->buf_mu);
  auto *c = find_command(ctx, t, binding);
  if (!c) return GLACIER_HIP_INVALID_HANDLE;
  glacier_hip_async_completion_t exact;
  completion_of(ctx, t->generation, *c, false, &exact);
  if ((exact.state != GLACIER_HIP_COMMAND_COMPLETED && exact.state != GLACIER_HIP_COMMAND_ERROR) ||
      memcmp(&exact, expected, sizeof exact) != 0)
    return GLACIER_HIP_INVALID_TRANSACTION;
  (void)hipEventDestroy(c->start);
  (void)hipEventDestroy(c->end);
  ctx->commands.erase(t->generation);
  return GLACIER_HIP_OK;
}

int glacier_hip_int4_registered_output_read(glacier_hip_context *ctx,
                                            const glacier_hip_command_token_t *t,
                                            const uint8_t binding[32],
                                            const glacier_hip_async_completion_t *expected,
                                            const glacier_hip_buffer_token_t *otok,
                                            float *output, uint64_t output_count) {
  if (!ctx || !t || !binding || t->generation == 0 || binding_zero(binding) ||
      !expected_ok(t, binding, expected) || !otok || !output || output_count == 0 ||
      output_count > UINT64_MAX / 4)
    return GLACIER_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> bl(ctx->buf_mu);
  auto *c = find_command(ctx, t, binding);
  if (!c) return GLACIER_HIP_INVALID_HANDLE;
  glacier_hip_async_completion_t exact;
  completion_of(ctx, t->generation, *c, false, &exact);
  if (exact.state != GLACIER_HIP_COMMAND_COMPLETED || memcmp(&exact, expected, sizeof exact) != 0)
    return GLACIER_HIP_INVALID_TRANSACTION;
  auto it = ctx->buffers.find(otok->id);
  if (otok->id != c->buf[3] || it == ctx->buffers.end() ||
      it->second.requested != otok->requested_bytes || output_count * 4 > it->second.requested)
    return GLACIER_HIP_SHAPE_MISMATCH;
  GH_CHECK(ctx, hipMemcpy(output, it->second.ptr, output_count * 4, hipMemcpyDeviceToHost));
  return GLACIER_HIP_OK;
}

int glacier_hip_live_command_count(glacier_hip_context *ctx, uint64_t *out) {
  if (!ctx || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> bl(ctx->buf_mu);
  *out = ctx->commands.size();
  return GLACIER_HIP_OK;
}

int glacier_hip_rmsnorm(glacier_hip_context *ctx, const float *x_dev, const float *w_dev,
                        uint32_t rows, uint32_t dim, float eps, float *out_dev, void *stream) {
  if (!ctx || !x_dev || !w_dev || !out_dev) return GLACIER_HIP_INVALID_ARGUMENT;
  if (rows == 0 || dim == 0) return GLACIER_HIP_SHAPE_MISMATCH;
  GH_CHECK(ctx, gk::launch_rmsnorm(x_dev, w_dev, (int)rows, (int)dim, eps, out_dev,
                                   stream ? (hipStream_t)stream : ctx->stream));
  return GLACIER_HIP_OK;
}

int glacier_hip_paged_attention(glacier_hip_context *ctx, const float *q_dev,
                                const void *kv_pool_dev, int kv_dtype,
                                const int32_t *page_table_dev, uint32_t max_pages_per_lane,
                                const int32_t *ctx_lens_dev, uint32_t lanes, uint32_t layer,
                                uint32_t num_layers, uint32_t num_heads, uint32_t num_kv_heads,
                                uint32_t head_dim, uint32_t max_ctx, float *out_dev,
                                void *stream) {
  if (!ctx || !q_dev || !kv_pool_dev || !page_table_dev || !ctx_lens_dev || !out_dev)
    return GLACIER_HIP_INVALID_ARGUMENT;
  if (kv_dtype != GLACIER_HIP_F32 && kv_dtype != GLACIER_HIP_F16) return GLACIER_HIP_DTYPE_UNSUPPORTED;
  if (lanes == 0 || lanes > 64 || num_kv_heads == 0 || num_heads % num_kv_heads != 0 ||
      num_heads / num_kv_heads > 8 || (head_dim != 64 && head_dim != 128) ||
      layer >= num_layers || max_ctx == 0 || (max_ctx + 15) / 16 > max_pages_per_lane)
    return GLACIER_HIP_SHAPE_MISMATCH;
  GH_SUBMISSION(ctx);
  hipStream_t st = stream ? (hipStream_t)stream : ctx->stream;
  // lane_of_row = identity: row i attends with page-table row i
  const size_t sc = gk::attention_scratch_floats((int)lanes, (int)num_heads, (int)num_kv_heads,
                                                 (int)head_dim, (int)max_ctx);
  auto &ss = ctx->per_stream[st];
  int rc = gh::ensure_scratch(ctx, ss, sc * 4, 1);
  if (rc) return rc;
  GH_CHECK(ctx, gk::launch_attention(q_dev, kv_pool_dev, kv_dtype == GLACIER_HIP_F16, page_table_dev,
                                     (int)max_pages_per_lane, ctx->ident, ctx_lens_dev, (int)lanes,
                                     (int)layer, (int)num_layers, (int)num_heads,
                                     (int)num_kv_heads, (int)head_dim, (int)max_ctx,
                                     (float *)ss.scratch, out_dev, st));
  return GLACIER_HIP_OK;
}

int glacier_hip_paged_attention_o(glacier_hip_context *ctx, const float *q_dev,
                                  const void *kv_pool_dev, const int32_t *page_table_dev,
                                  uint32_t max_pages, const int32_t *ctx_len_dev, uint32_t layer,
                                  uint32_t num_layers, uint32_t num_heads, uint32_t num_kv_heads,
                                  uint32_t head_dim, uint32_t max_ctx,
                                  const glacier_hip_int4_weight *o_weight, float *parts_dev,
                                  void *stream) {
  if (!ctx || !q_dev || !kv_pool_dev || !page_table_dev || !ctx_len_dev || !o_weight ||
      !parts_dev)
    return GLACIER_HIP_INVALID_ARGUMENT;
  if (o_weight->ctx != ctx) return GLACIER_HIP_INVALID_HANDLE;
  gk::AttnOArgs a{};
  a.q = q_dev;
  a.kv_pool = kv_pool_dev;
  a.page_table = page_table_dev;
  a.max_pages = (int)max_pages;
  a.lane_of_row = ctx->ident;  // row 0 attends with page-table row 0
  a.ctx_len = ctx_len_dev;
  a.layer = (int)layer;
  a.num_layers = (int)num_layers;
  a.num_heads = (int)num_heads;
  a.num_kv_heads = (int)num_kv_heads;
  a.head_dim = (int)head_dim;
  a.max_ctx = (int)max_ctx;
  a.codes = o_weight->codes;
  a.scales = o_weight->scales;
  a.N = (int)o_weight->out_f;
  a.K = (int)o_weight->in_f;
  a.parts = parts_dev;
  if (layer >= num_layers || max_ctx == 0 || max_pages == 0 || (max_ctx + 15) / 16 > max_pages ||
      max_ctx > (1u << 24) || num_heads > 1024 || !gk::attn_o_ok(a))
    return GLACIER_HIP_SHAPE_MISMATCH;
  GH_SUBMISSION(ctx);
  hipStream_t st = stream ? (hipStream_t)stream : ctx->stream;
  GH_CHECK(ctx, gk::launch_attn_o(a, st));
  return GLACIER_HIP_OK;
}

int glacier_hip_paged_attention_prefill(glacier_hip_context *ctx, const float *q_dev,
                                        const void *kv_pool_dev, const int32_t *page_table_dev,
                                        uint32_t max_pages, uint32_t pos0, uint32_t T,
                                        uint32_t layer, uint32_t num_layers, uint32_t num_heads,
                                        uint32_t num_kv_heads, uint32_t head_dim, float *out_dev,
                                        void *stream) {
  if (!ctx || !q_dev || !kv_pool_dev || !page_table_dev || !out_dev)
    return GLACIER_HIP_INVALID_ARGUMENT;
  if (T == 0 || num_kv_heads == 0 || num_heads % num_kv_heads != 0 ||
      num_heads / num_kv_heads > 8 || (head_dim != 64 && head_dim != 128) ||
      layer >= num_layers || (uint64_t)pos0 + T > (uint64_t)max_pages * 16 || pos0 > (1u << 30))
    return GLACIER_HIP_SHAPE_MISMATCH;
  GH_SUBMISSION(ctx);
  GH_CHECK(ctx, gk::launch_attention_prefill(q_dev, kv_pool_dev, page_table_dev, (int)max_pages, 0,
                                             (int)pos0, (int)T, (int)layer, (int)num_layers,
                                             (int)num_heads, (int)num_kv_heads, (int)head_dim,
                                             out_dev, stream ? (hipStream_t)stream : ctx->stream));
  return GLACIER_HIP_OK;
}

static int argmax_common(glacier_hip_context *ctx, const float *logits_dev, uint64_t n,
                         const uint64_t *words_dev, uint64_t word_count, uint32_t rows,
                         glacier_hip_argmax_result_t *out, hipStream_t st) {
  if (!ctx || !logits_dev || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  if (rows == 0 || rows > 64) return GLACIER_HIP_SHAPE_MISMATCH;
  if (words_dev) {
    const uint64_t wc = n / 64 + (n % 64 != 0);
    if (wc == 0 || word_count != wc) {
      for (uint32_t r = 0; r < rows; ++r) out[r] = {0, 0, GLACIER_HIP_INVALID_MASK, 0};
      return GLACIER_HIP_INVALID_MASK;
    }
  } else if (n == 0) {
    return GLACIER_HIP_SHAPE_MISMATCH;
  }
  GH_SUBMISSION(ctx);
  const size_t sb = gk::argmax_scratch_bytes((int)rows, (long)n);
  auto &ss = ctx->per_stream[st];
  int rc = gh::ensure_scratch(ctx, ss, sb + 256 + rows * sizeof(gk::ArgmaxResult), rows);
  if (rc) return rc;
  auto *res_dev = (gk::ArgmaxResult *)((char *)ss.scratch + ((sb + 255) & ~(size_t)255));
  GH_CHECK(ctx, gk::launch_argmax(logits_dev, (long)n, (int)rows, words_dev, (long)word_count,
                                  ss.scratch, ss.counters, res_dev, st));
  GH_CHECK(ctx, hipMemcpyAsync(ctx->results_host, res_dev, rows * sizeof(gk::ArgmaxResult),
                               hipMemcpyDeviceToHost, st));
  GH_CHECK(ctx, hipStreamSynchronize(st));
  int status = GLACIER_HIP_OK;
  for (uint32_t r = 0; r < rows; ++r) {
    const gk::ArgmaxResult &g = ctx->results_host[r];
    out[r].token_index = g.index;
    out[r].eligible_rows = g.eligible_rows;
    out[r].status = g.status;
    out[r].reserved = 0;
    if (g.status && !status) status = g.status;
  }
  return status;
}

int glacier_hip_argmax(glacier_hip_context *ctx, const float *logits_dev, uint64_t n,
                       uint32_t rows, uint64_t *index_host, void *stream) {
  if (!index_host) return GLACIER_HIP_INVALID_ARGUMENT;
  std::vector<glacier_hip_argmax_result_t> r(rows ? rows : 1);
  int rc = argmax_common(ctx, logits_dev, n, nullptr, 0, rows, r.data(),
                         stream ? (hipStream_t)stream : (ctx ? ctx->stream : nullptr));
  if (rc) return rc;
  for (uint32_t i = 0; i < rows; ++i) index_host[i] = r[i].token_index;
  return GLACIER_HIP_OK;
}

int glacier_hip_eligible_argmax(glacier_hip_context *ctx, const float *logits_dev, uint64_t n,
                                const uint64_t *words_dev, uint64_t word_count, uint32_t rows,
                                glacier_hip_argmax_result_t *results_host, void *stream) {
  if (!words_dev) return GLACIER_HIP_INVALID_ARGUMENT;
  return argmax_common(ctx, logits_dev, n, words_dev, word_count, rows, results_host,
                       stream ? (hipStream_t)stream : (ctx ? ctx->stream : nullptr));
}

// The reference's eligible-greedy counts (EligibleGreedyContext.run,
// int4_executor.zig:986-1150, totals :1939-1966): per 64-row tile, a fully
// eligible tile is one run of all its rows; otherwise each maximal run of
// 4-row groups holding an eligible row is one run of 4 rows per group.
// device_rows: the 16-row blocks this device streams (any eligible row).
static void eligible_counts(const uint64_t *words, uint64_t out_f,
                            glacier_hip_eligible_greedy_result_t &r) {
  r.eligible_rows = r.producer_rows = r.producer_runs = r.device_rows = 0;
  const uint64_t tiles = (out_f + 63) / 64;
  for (uint64_t t = 0; t < tiles; ++t) {
    const uint64_t row_count = std::min<uint64_t>(64, out_f - 64 * t);
    const uint64_t valid = row_count == 64 ? ~0ull : (1ull << row_count) - 1;
    const uint64_t e = words[t] & valid;
    r.eligible_rows += (uint64_t)__builtin_popcountll(e);
    if (!e) continue;
    if (e == valid) {
      r.producer_rows += row_count;
      r.producer_runs += 1;
      continue;
    }
    bool in_run = false;
    for (uint64_t g = 0; g < row_count / 4; ++g) {
      if ((e >> (4 * g)) & 0xFull) {
        r.producer_rows += 4;
        if (!in_run) r.producer_runs += 1;
        in_run = true;
      } else {
        in_run = false;
      }
    }
  }
  for (uint64_t b = 0; b < out_f / 16; ++b)
    if ((words[b / 4] >> ((b % 4) * 16)) & 0xFFFFull) r.device_rows += 16;
  r.skipped_rows = out_f - r.producer_rows;
  r.overcomputed_rows = r.producer_rows - r.eligible_rows;
}

int glacier_hip_int4_eligible_greedy(glacier_hip_context *ctx, glacier_hip_int4_weight *w,
                                     const float *x_dev, uint32_t in_f,
                                     const uint64_t *words_host, uint64_t word_count,
                                     int activation, glacier_hip_eligible_greedy_result_t *out,
                                     void *stream) {
  if (!ctx || !w || !x_dev || !words_host || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  if (w->ctx != ctx) return GLACIER_HIP_INVALID_HANDLE;
  int D;
  if (activation == GLACIER_HIP_ACT_AUTO || activation == GLACIER_HIP_ACT_Q8) D = 1;
  else if (activation == GLACIER_HIP_ACT_F32) D = 3;
  else return GLACIER_HIP_INVALID_ARGUMENT;
  // validation before any write (int4_executor.zig:1870-1890): geometry,
  // eligibility words (validateEligibleWords), a finite input
  const uint64_t V = w->out_f;
  if (in_f != w->in_f || V % 4) return GLACIER_HIP_SHAPE_MISMATCH;
  const uint64_t W = V / 64 + (V % 64 != 0);
  if (word_count != W) return GLACIER_HIP_SHAPE_MISMATCH;
  if (V % 64 && (words_host[W - 1] >> (V % 64)) != 0) return GLACIER_HIP_SHAPE_MISMATCH;
  glacier_hip_eligible_greedy_result_t r{};
  eligible_counts(words_host, V, r);
  if (r.eligible_rows == 0) return GLACIER_HIP_SHAPE_MISMATCH;
  GH_SUBMISSION(ctx);
  hipStream_t st = stream ? (hipStream_t)stream : ctx->stream;
  {
    std::vector<float> xh(in_f);
    GH_CHECK(ctx, hipMemcpyAsync(xh.data(), x_dev, (size_t)in_f * 4, hipMemcpyDeviceToHost, st));
    GH_CHECK(ctx, hipStreamSynchronize(st));
    for (float v : xh)
      if (!std::isfinite(v)) return GLACIER_HIP_SHAPE_MISMATCH;
  }
  const int nparts = gk::gemv_argmax_parts((int)V, (int)in_f, 1, D);
  if (nparts <= 0) return GLACIER_HIP_SHAPE_MISMATCH;
  auto &ss = ctx->per_stream[st];
  const size_t pb = planes_bytes(1, in_f, D);
  if (pb > ss.planes_bytes) {
    gh::dev_free(ctx, ss.planes);
    ss.planes = nullptr;
    ss.planes_bytes = 0;
    GH_CHECK(ctx, gh::dev_malloc(ctx, &ss.planes, pb));
    ss.planes_bytes = pb;
  }
  // scratch: eligibility words | candidates | merged result
  const size_t wb = al256(W * 8), cb = al256((size_t)nparts * sizeof(gk::ArgPartial));
  int rc = gh::ensure_scratch(ctx, ss, wb + cb + sizeof(gk::ArgmaxResult), 1);
  if (rc) return rc;
  auto *words_dev = (uint64_t *)ss.scratch;
  auto *parts = (gk::ArgPartial *)((char *)ss.scratch + wb);
  auto *res_dev = (gk::ArgmaxResult *)((char *)ss.scratch + wb + cb);
  GH_CHECK(ctx, hipMemcpyAsync(words_dev, words_host, W * 8, hipMemcpyHostToDevice, st));
  rc = prepare_launch(ctx, x_dev, GLACIER_HIP_F32, 1, in_f, D, ss.planes, st);
  if (rc) return rc;
  gk::GemvArgs a{};
  a.codes = w->codes;
  a.scales = w->scales;
  a.N = (int)V;
  a.K = (int)in_f;
  a.act_q = (const int8_t *)ss.planes;
  a.act_meta = (const gk::ActMeta *)((const char *)ss.planes + al256(planes_q_bytes(1, in_f, D)));
  a.M = 1;
  a.D = D;
  a.epi = gk::EPI_PLAIN;
  a.arg_parts = parts;
  a.arg_words = words_dev;
  a.arg_word_count = (long)W;
  a.prehead = 1;
  GH_CHECK(ctx, gk::launch_gemv(a, st));
  GH_CHECK(ctx, gk::launch_argmax_parts(parts, nparts, (long)V, 1, words_dev, (long)W, res_dev, st));
  GH_CHECK(ctx, hipMemcpyAsync(ctx->results_host, res_dev, sizeof(gk::ArgmaxResult),
                               hipMemcpyDeviceToHost, st));
  GH_CHECK(ctx, hipStreamSynchronize(st));
  const gk::ArgmaxResult &g = ctx->results_host[0];
  // an eligible NaN (or any mask the host checks missed) is the reference's
  // ShapeMismatch (int4_executor.zig:1933-1938)
  if (g.status != GLACIER_HIP_OK || g.index >= V || g.eligible_rows != r.eligible_rows)
    return GLACIER_HIP_SHAPE_MISMATCH;
  r.token_index = g.index;
  *out = r;
  return GLACIER_HIP_OK;
}

// ---- synthetic generator ----------------------------------------------------
static inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
static inline uint64_t stream_key(uint64_t seed, uint64_t tensor_id) {
  return mix64(seed ^ mix64(tensor_id + 0x632be59bd9b4e019ull));
}
static inline uint64_t stream_at(uint64_t key, uint64_t i) {
  return mix64(key + (i + 1) * 0x9e3779b97f4a7c15ull);
}
// Box-Muller pair from stream values 2i and 2i+1, in double precision.
static inline void normal_pair(uint64_t key, uint64_t i, double *z0, double *z1) {
  const double u1 = (double)((stream_at(key, 2 * i) >> 11) + 1) * 0x1.0p-53;
  const double u2 = (double)(stream_at(key, 2 * i + 1) >> 11) * 0x1.0p-53;
  const double r = sqrt(-2.0 * log(u1));
  const double a = 6.283185307179586 * u2;
  *z0 = r * cos(a);
  *z1 = r * sin(a);
}

void glacier_hip_synth_int4(uint64_t seed, uint64_t tensor_id, uint8_t *packed, uint64_t bytes) {
  const uint64_t key = stream_key(seed, tensor_id);
  const uint64_t words = bytes / 8;
  gh::parallel_for(words, [&](size_t b, size_t e) {
    for (size_t i = b; i < e; ++i) {
      const uint64_t v = stream_at(key, i);
      memcpy(packed + 8 * i, &v, 8);
    }
  }, 1 << 16);
  if (bytes % 8) {
    const uint64_t v = stream_at(key, words);
    memcpy(packed + 8 * words, &v, bytes % 8);
  }
}

void glacier_hip_synth_scales_f16(uint64_t seed, uint64_t tensor_id, float sigma, uint16_t *out,
                                  uint64_t count) {
  const uint64_t key = stream_key(seed, tensor_id);
  gh::parallel_for((count + 1) / 2, [&](size_t b, size_t e) {
    for (size_t i = b; i < e; ++i) {
      double z0, z1;
      normal_pair(key, i, &z0, &z1);
      out[2 * i] = gh::f32_to_f16(fabsf((float)(sigma * z0)));
      if (2 * i + 1 < count) out[2 * i + 1] = gh::f32_to_f16(fabsf((float)(sigma * z1)));
    }
  }, 1 << 14);
}

void glacier_hip_synth_normal_f32(uint64_t seed, uint64_t tensor_id, float sigma, float *out,
                                  uint64_t count) {
  const uint64_t key = stream_key(seed, tensor_id);
  gh::parallel_for((count + 1) / 2, [&](size_t b, size_t e) {
    for (size_t i = b; i < e; ++i) {
      double z0, z1;
      normal_pair(key, i, &z0, &z1);
      out[2 * i] = (float)(sigma * z0);
      if (2 * i + 1 < count) out[2 * i + 1] = (float)(sigma * z1);
    }
  }, 1 << 14);
}

void glacier_hip_synth_tokens(uint64_t seed, uint64_t tensor_id, uint32_t vocab, uint32_t *out,
                              uint64_t count) {
  const uint64_t key = stream_key(seed, tensor_id);
  for (uint64_t i = 0; i < count; ++i) out[i] = (uint32_t)(stream_at(key, i) % vocab);
}

uint64_t glacier_hip_synth_tensor_id(uint32_t layer, uint32_t which) {
  return ((uint64_t)layer + 1) << 8 | which;
}

float glacier_hip_f16_to_f32(uint16_t h) { return gh::f16_to_f32(h); }

}  // extern "C"
