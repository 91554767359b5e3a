// runtime.h — internal structures shared by the C-ABI implementation files.
#pragma once
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/glacier_hip.h"
#include "kernels.h"

struct glacier_hip_context {
  int device = 0;
  hipStream_t stream = nullptr;
  hipDeviceProp_t props{};
  uint64_t epoch = 0;  // binds allocation quotes to this context
  std::mutex mu;       // one submission at a time (int4_executor.zig:2267)
  std::mutex buf_mu;   // buffer table (backend.zig:1682-1684 buffer mutex)
  std::string last_error;
  struct Buf {
    void *ptr;
    uint64_t requested, charged;
  };
  std::map<uint64_t, Buf> buffers;
  uint64_t next_buffer_id = 1;
  uint64_t live_weights = 0;
  // Scratch of the stand-alone kernel entry points, one set per stream: the
  // host lock only orders the calls, so work queued on two streams must not
  // share a buffer.
  struct StreamScratch {
    void *scratch = nullptr;  // attention partials / argmax candidates
    size_t scratch_bytes = 0;
    void *planes = nullptr;  // activation planes of glacier_hip_int4_gemv
    size_t planes_bytes = 0;
    float *splitk = nullptr;  // GEMM split-K partial sums of glacier_hip_int4_gemv
    size_t splitk_floats = 0;
    uint32_t *counters = nullptr;  // zeroed once, self-resetting
    size_t counter_count = 0;
  };
  std::map<hipStream_t, StreamScratch> per_stream;
  gk::ArgmaxResult *results_host = nullptr;  // pinned
  int32_t *ident = nullptr;  // device 0..63: row i -> page-table row i
  // asynchronous registered dispatches, by command generation
  struct AsyncCmd {
    uint8_t binding[32];
    uint64_t buf[4];  // packed, scales, input, output buffer ids
    hipEvent_t start = nullptr, end = nullptr;
    uint64_t alloc_before = 0;
    bool observed = false;  // the final completion record is fixed once seen
    glacier_hip_async_completion_t final{};
  };
  // every device allocation of the product (buffers, weights, sessions,
  // scratch): requested and granularity-charged bytes
  std::mutex dev_mu;
  std::map<void *, uint64_t> dev_allocs;
  uint64_t dev_requested = 0, dev_charged = 0;
  std::map<uint64_t, AsyncCmd> commands;
  uint64_t next_command_generation = 1;
  uint64_t nonce[4] = {0, 0, 0, 0};
  hipEvent_t origin = nullptr;  // recorded at init: the zero of the GPU times
  // device address of this device's no-allocation GEMV scratch (null when
  // hipGetSymbolAddress failed at init; the entry point then refuses)
  void *noalloc_scratch = nullptr;
};

struct glacier_hip_int4_weight {
  glacier_hip_context *ctx = nullptr;
  uint32_t out_f = 0, in_f = 0, group = 32;
  uint4 *codes = nullptr;
  uint2 *scales = nullptr;
  uint64_t device_bytes = 0;
};

namespace gh {

// Allocation granularity the lease adapter charges (hipMalloc rounds large
// buffers to 2 MiB pages).
constexpr uint64_t kGranularity = 2ull << 20;
inline uint64_t charged_bytes(uint64_t requested) {
  return requested == 0 ? 0 : (requested + kGranularity - 1) / kGranularity * kGranularity;
}
// hipMalloc / hipFree with the context's device-byte accounting.
hipError_t dev_malloc(glacier_hip_context *ctx, void **p, size_t bytes);
void dev_free(glacier_hip_context *ctx, void *p);

// Record a HIP failure on the context and map it to a status code.
int hip_fail(glacier_hip_context *ctx, hipError_t e, const char *what);
#define GH_CHECK(ctx, expr)                                   \
  do {                                                        \
    hipError_t _e = (expr);                                   \
    if (_e != hipSuccess) return gh::hip_fail((ctx), _e, #expr); \
  } while (0)

// Device row source for the tile repack: row `row` of a reference-layout
// matrix (packed codes + f32 scales), or an all-zero row when packed == null.
struct RowSrc {
  const uint8_t *packed;
  const float *scales_f32;
  const uint16_t *scales_f16;
  uint64_t row;
};

// Build the device tile layout (kernels.h) for rows[0..N) of width K.
void repack_tiles(const std::vector<RowSrc> &rows, uint32_t K, std::vector<uint32_t> &codes,
                  std::vector<uint16_t> &scales);

glacier_hip_int4_weight *upload_weight(glacier_hip_context *ctx, uint32_t out_f, uint32_t in_f,
                                       const std::vector<uint32_t> &codes,
                                       const std::vector<uint16_t> &scales);

// Ensure the stream's scratch holds at least `bytes` and its counters `count`.
int ensure_scratch(glacier_hip_context *ctx, glacier_hip_context::StreamScratch &ss, size_t bytes,
                   size_t counters);

// The host side of a submission: one at a time per context, a second one
// (from another thread) is rejected with GLACIER_HIP_BUSY rather than queued
// (acquireSubmission, int4_executor.zig:2267-2270).
#define GH_SUBMISSION(ctx)                                        \
  std::unique_lock<std::mutex> _submission((ctx)->mu, std::try_to_lock); \
  if (!_submission.owns_lock()) return GLACIER_HIP_BUSY

// Run one projection on the device: prep (+ optional norm) then GEMV.
struct ProjBuffers {
  int8_t *act_q;
  gk::ActMeta *meta;
  float *partial;
  uint32_t *counters;
};
int resolve_activation(int activation, uint32_t out_f, uint32_t in_f);

}  // namespace gh
