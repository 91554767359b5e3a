// Host-side exerciser for the runtime's host C++ (LaneWeave scheduler,
// paged-KV page map and row transactions, publication digests, page-image
// codec, prepared runtime image reader, SHA-256 and fp16 helpers). It is
// compiled together with those sources under AddressSanitizer +
// UndefinedBehaviorSanitizer (and the concurrent mode under
// ThreadSanitizer) by tests/test_host_sanitizers.py and run on the CPU; it
// calls the same C ABI the device library exports. Every mode checks the
// module's own invariants and exits non-zero on a violation; the sanitizers
// abort on the first memory or undefined-behaviour error.
//
// Modes:
//   sha <n>                 SHA-256 of lengths 0..n-1 (one shot and chunked), hex per line
//   f16 <out.bin>           f16->f32 of every half and f32->f16 of a fixed sample, to a file
//   laneweave <seed> <ops>  random admit / plan / wave / serve / cancel / retire / close trace
//   pagedkv <seed> <ops>    random begin / commit / abort / reset, page images of every
//                           committed page, decode of mutated and truncated images
//   glrt <seed> <tmp> <nvalid> <image>...  open and walk each image, then mutated copies
//   threads <seed> <ops>    two threads driving one scheduler (waves vs admit / cancel)
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <random>
#include <string>
#include <atomic>
#include <thread>
#include <vector>

#include "glacier_hip.h"
#include "host_util.h"
#include "lane_weave.h"
#include "page_image.h"
#include "runtime_image.h"

namespace {

int g_fail = 0;
struct Counts {
  long admitted = 0, served = 0, waves = 0, failed_waves = 0, commits = 0, aborts = 0, resets = 0;
  long images = 0, decoded = 0, refused = 0;
} g_n;
#define CHECK(c)                                                              \
  do {                                                                        \
    if (!(c)) {                                                               \
      fprintf(stderr, "%s:%d check failed: %s\n", __FILE__, __LINE__, #c);    \
      ++g_fail;                                                               \
      return;                                                                 \
    }                                                                         \
  } while (0)

void hex(const uint8_t *d, size_t n, char *out) {
  static const char *k = "0123456789abcdef";
  for (size_t i = 0; i < n; ++i) {
    out[2 * i] = k[d[i] >> 4];
    out[2 * i + 1] = k[d[i] & 15];
  }
  out[2 * n] = 0;
}

// ---------------------------------------------------------------- sha ----
void mode_sha(int n) {
  std::mt19937_64 rng(1);
  for (int len = 0; len < n; ++len) {
    std::vector<uint8_t> buf(len);
    for (int i = 0; i < len; ++i) buf[i] = (uint8_t)(i * 131 + 7);
    uint8_t a[32], b[32];
    gh::Sha256 s;
    s.update(buf.data(), buf.size());
    s.final(a);
    gh::Sha256 t;
    for (size_t off = 0; off < buf.size();) {
      size_t step = std::min<size_t>(buf.size() - off, 1 + rng() % 97);
      t.update(buf.data() + off, step);
      off += step;
    }
    t.final(b);
    CHECK(memcmp(a, b, 32) == 0);
    char h[65];
    hex(a, 32, h);
    printf("%s\n", h);
  }
}

// ---------------------------------------------------------------- f16 ----
void mode_f16(const char *path) {
  std::vector<uint32_t> out;
  for (uint32_t h = 0; h < 65536; ++h) {
    float f = gh::f16_to_f32((uint16_t)h);
    uint32_t bits;
    memcpy(&bits, &f, 4);
    out.push_back(bits);
    if (f == f) CHECK(gh::f32_to_f16(f) == h);  // every non-NaN half round-trips
  }
  std::mt19937 rng(7);
  for (int i = 0; i < 65536; ++i) {
    uint32_t bits = rng();
    if (i < 4096) bits = (bits & 0x807FFFFFu) | ((uint32_t)(101 + (i % 40)) << 23);  // near f16 range
    float f;
    memcpy(&f, &bits, 4);
    out.push_back(bits);
    out.push_back(gh::f32_to_f16(f));
  }
  FILE *fp = fopen(path, "wb");
  CHECK(fp != nullptr);
  CHECK(fwrite(out.data(), 4, out.size(), fp) == out.size());
  fclose(fp);
}

// ---------------------------------------------------------- laneweave ----
glacier_hip_limits_t limits(uint32_t capacity) {
  glacier_hip_limits_t l;
  memset(&l, 0, sizeof l);
  l.host_bytes = 1 << 20;
  l.kv_bytes = 1 << 20;
  l.queue_slots = capacity;
  return l;
}

glacier_hip_request_spec_t spec(uint64_t key, uint64_t gen, uint64_t weight, uint64_t work,
                                uint64_t deadline) {
  glacier_hip_request_spec_t s;
  memset(&s, 0, sizeof s);
  s.tenant_key = key;
  s.request_key = key * 10;
  s.request_generation = gen;
  s.resource_owner_key = key * 100;
  s.weight = weight;
  s.work_quanta = work;
  s.deadline_tick = deadline;
  s.claim.kv_bytes = 64;
  s.claim.queue_slots = 1;
  return s;
}

glacier_hip_lane_weave *make_weave(uint32_t capacity, uint32_t max_weight) {
  uint8_t challenge[32] = {0xA5};
  glacier_hip_limits_t l = limits(capacity);
  return glacier_hip_lane_weave_create(capacity, &l, 0x42414E4B, 0x51534553, challenge, max_weight,
                                       10000, 1000000);
}

// `concurrent`: another thread drives the same scheduler, so the checks that
// compare two separate calls (plan vs serve, state before vs after a wave)
// are skipped; every call must still be memory- and race-safe.
void weave_trace(glacier_hip_lane_weave *lw, uint32_t capacity, std::mt19937_64 &rng, int ops,
                 uint64_t key_base, bool concurrent) {
  uint64_t next_key = key_base;
  std::vector<glacier_hip_lane_handle_t> handles;
  for (int op = 0; op < ops; ++op) {
    glacier_hip_lane_event_t ev;
    uint8_t before[32], after[32];
    switch (rng() % 8) {
      case 0:
      case 1: {  // admit (sometimes malformed or infeasible)
        uint64_t w = rng() % 6;  // 0 and 5 are out of range for max_weight 4
        glacier_hip_request_spec_t s = spec(next_key++, 1 + rng() % 3, w, rng() % 9,
                                            (rng() % 4 == 0) ? rng() % 40 : 0);
        int admitted = 0;
        glacier_hip_lane_handle_t h;
        int rc = glacier_hip_lane_weave_admit(lw, &s, &admitted, &h, &ev);
        CHECK(rc == GLACIER_HIP_OK || rc == GLACIER_HIP_INVALID_ARGUMENT ||
              rc == GLACIER_HIP_SCHEDULER_CLOSED);
        if (rc == GLACIER_HIP_OK && admitted) {
          handles.push_back(h);
          ++g_n.admitted;
        }
        break;
      }
      case 2: {  // plan, then serve: the plan names the slots serve_one picks
        uint32_t plan[64], n = 0;
        uint32_t maxc = 1 + rng() % capacity;
        int rc = glacier_hip_lane_weave_plan_wave(lw, maxc, plan, &n);
        if (rc) break;
        CHECK(n <= maxc);
        for (uint32_t i = 0; i < n; ++i) {
          rc = glacier_hip_lane_weave_serve_one(lw, &ev);
          if (concurrent) continue;
          CHECK(rc == GLACIER_HIP_OK && ev.kind == GLACIER_HIP_EVENT_SERVICE);
          CHECK(ev.handle.slot_index == plan[i]);
          ++g_n.served;
        }
        break;
      }
      case 3: {  // a wave whose device step fails or whose sink rejects changes nothing
        glacier_hip_lane_weave_state_sha256(lw, before);
        uint32_t slots[64], n = 0, ran = 0, published = 0, aborted_from = ~0u;
        glacier_hip_lane_event_t evs[64];
        const bool fail = rng() % 3 == 0, reject = rng() % 4 == 0;
        gh::WaveOps ops;
        ops.run = [&](const uint32_t *s, uint32_t k) {
          for (uint32_t i = 0; i < k; ++i)
            if (s[i] >= capacity) return (int)GLACIER_HIP_INVALID_ARGUMENT;
          ran = k;
          return fail ? (int)GLACIER_HIP_DEVICE_ERROR : (int)GLACIER_HIP_OK;
        };
        if (reject) ops.sink = [&]() { return (int)GLACIER_HIP_SINK_REJECTED; };
        ops.publish = [&](uint32_t i) {
          if (i != published || i >= ran) {  // quanta publish once each, in plan order
            ++g_fail;
            return (int)GLACIER_HIP_INVALID_ARGUMENT;
          }
          ++published;
          return (int)GLACIER_HIP_OK;
        };
        ops.abort = [&](uint32_t from) { aborted_from = from; };
        int rc = gh::lane_weave_run_wave(lw, 1 + rng() % capacity, ops, slots, evs, &n);
        glacier_hip_lane_weave_state_sha256(lw, after);
        if (rc != GLACIER_HIP_OK) {
          g_n.failed_waves += rc == GLACIER_HIP_DEVICE_ERROR || rc == GLACIER_HIP_SINK_REJECTED;
          CHECK(n == 0 && published == 0);
          if (rc == GLACIER_HIP_SINK_REJECTED) CHECK(aborted_from == 0);
          if (!concurrent) CHECK(memcmp(before, after, 32) == 0);
        } else {
          CHECK(published == n && n == ran && aborted_from == ~0u);
          for (uint32_t i = 0; i < n; ++i) CHECK(evs[i].handle.slot_index == slots[i]);
          ++g_n.waves;
          g_n.served += n;
        }
        break;
      }
      case 7: {  // a caller's prepared service, committed or aborted
        glacier_hip_service_permit_v1_t p;
        glacier_hip_lane_weave_state_sha256(lw, before);
        int rc = glacier_hip_lane_weave_prepare_service(lw, &p);
        if (rc) break;
        glacier_hip_lane_weave_state_sha256(lw, after);
        if (!concurrent) CHECK(memcmp(before, after, 32) == 0);
        glacier_hip_service_permit_v1_t bad = p;
        bad.remaining_before += 1;
        CHECK(glacier_hip_lane_weave_commit_service(lw, &bad, &ev) == GLACIER_HIP_STALE_SERVICE_PERMIT);
        if (rng() & 1) {
          rc = glacier_hip_lane_weave_commit_service(lw, &p, &ev);
          CHECK(rc == GLACIER_HIP_OK && ev.handle.slot_index == p.handle.slot_index);
          ++g_n.served;
        } else {
          CHECK(glacier_hip_lane_weave_abort_service(lw, &p) == GLACIER_HIP_OK);
        }
        CHECK(glacier_hip_lane_weave_abort_service(lw, &p) == GLACIER_HIP_STALE_SERVICE_PERMIT);
        break;
      }
      case 4: {  // cancel or retire a known (maybe stale) handle
        if (handles.empty()) break;
        size_t i = rng() % handles.size();
        glacier_hip_lane_handle_t h = handles[i];
        if (rng() % 5 == 0) h.slot_generation += 1;  // stale on purpose
        int rc = (rng() & 1) ? glacier_hip_lane_weave_cancel(lw, &h, &ev)
                             : glacier_hip_lane_weave_retire(lw, &h, &ev);
        if (rc == GLACIER_HIP_OK) handles.erase(handles.begin() + i);
        break;
      }
      case 5: {  // read every slot
        for (uint32_t s = 0; s < capacity + 2; ++s) {
          glacier_hip_lane_handle_t h;
          uint32_t st = 9;
          uint64_t rem = 0;
          int rc = glacier_hip_lane_weave_slot(lw, s, &h, &st, &rem);
          if (s >= capacity) CHECK(rc != GLACIER_HIP_OK);
          else CHECK(rc == GLACIER_HIP_OK && st <= 2);
        }
        break;
      }
      default: {
        uint8_t head[32];
        CHECK(glacier_hip_lane_weave_chain_head(lw, head) == GLACIER_HIP_OK);
        break;
      }
    }
  }
}

void drain_and_close(glacier_hip_lane_weave *lw, uint32_t capacity) {
  glacier_hip_lane_event_t ev;
  for (int guard = 0; guard < 100000; ++guard)
    if (glacier_hip_lane_weave_serve_one(lw, &ev) != GLACIER_HIP_OK) break;
  for (uint32_t s = 0; s < capacity; ++s) {
    glacier_hip_lane_handle_t h;
    uint32_t st;
    uint64_t rem;
    if (glacier_hip_lane_weave_slot(lw, s, &h, &st, &rem) == GLACIER_HIP_OK && st != 0)
      glacier_hip_lane_weave_retire(lw, &h, &ev);
  }
  int rc = glacier_hip_lane_weave_close(lw, &ev);
  CHECK(rc == GLACIER_HIP_OK && ev.kind == GLACIER_HIP_EVENT_CLOSE);
  // a closed scheduler admits nothing
  glacier_hip_request_spec_t s = spec(999999, 1, 1, 1, 0);
  int admitted = 1;
  glacier_hip_lane_handle_t h;
  rc = glacier_hip_lane_weave_admit(lw, &s, &admitted, &h, &ev);
  CHECK(rc != GLACIER_HIP_OK || admitted == 0);
}

void mode_laneweave(uint64_t seed, int ops) {
  std::mt19937_64 rng(seed);
  for (uint32_t capacity : {1u, 3u, 8u, 32u}) {
    glacier_hip_lane_weave *lw = make_weave(capacity, 4);
    CHECK(lw != nullptr);
    weave_trace(lw, capacity, rng, ops, 1, false);
    drain_and_close(lw, capacity);
    glacier_hip_lane_weave_destroy(lw);
  }
  // invalid configurations create nothing
  uint8_t zero[32] = {0};
  glacier_hip_limits_t l = limits(4);
  CHECK(glacier_hip_lane_weave_create(0, &l, 1, 1, zero, 4, 10, 10) == nullptr);
  uint8_t ch[32] = {1};
  CHECK(glacier_hip_lane_weave_create(4, &l, 1, 1, zero, 4, 10, 10) == nullptr);
  CHECK(glacier_hip_lane_weave_create(4, nullptr, 1, 1, ch, 4, 10, 10) == nullptr);
}

void mode_threads(uint64_t seed, int ops) {
  const uint32_t capacity = 16;
  glacier_hip_lane_weave *lw = make_weave(capacity, 4);
  CHECK(lw != nullptr);
  std::thread waves([&] {
    std::mt19937_64 rng(seed + 1);
    for (int i = 0; i < ops; ++i) {
      uint32_t slots[16], n = 0;
      glacier_hip_lane_event_t evs[16];
      gh::WaveOps ops;
      ops.run = [](const uint32_t *, uint32_t) { return (int)GLACIER_HIP_OK; };
      ops.publish = [](uint32_t) { return (int)GLACIER_HIP_OK; };
      ops.abort = [](uint32_t) {};
      gh::lane_weave_run_wave(lw, 1 + rng() % capacity, ops, slots, evs, &n);
      uint8_t head[32];
      glacier_hip_lane_weave_chain_head(lw, head);
    }
  });
  std::mt19937_64 rng(seed);
  weave_trace(lw, capacity, rng, ops, 1000, true);
  waves.join();
  drain_and_close(lw, capacity);
  glacier_hip_lane_weave_destroy(lw);
}

// ------------------------------------------------------------ pagedkv ----
void image_fuzz(const std::vector<uint8_t> &img, const uint8_t challenge[32], std::mt19937_64 &rng) {
  glacier_hip_page_image_v1_t info;
  CHECK(glacier_hip_page_image_decode(img.data(), img.size(), challenge, &info) == GLACIER_HIP_OK);
  for (int k = 0; k < 24; ++k) {
    std::vector<uint8_t> m = img;
    switch (k % 3) {
      case 0: m[rng() % m.size()] ^= (uint8_t)(1 + rng() % 255); break;
      case 1: m.resize(rng() % m.size()); break;
      default: {  // a header field replaced (small, large or random), or a payload byte
        size_t off = (k % 2) ? 8 * (rng() % 26) : 208 + rng() % (m.size() - 240);
        uint64_t v = rng() % 3 == 0 ? rng() % 64 : rng() % 3 == 0 ? ~0ull - rng() % 64 : rng();
        if (off + 8 <= m.size() - 32) memcpy(m.data() + off, &v, 8);
        // re-signed, so the checks behind the image digest run too
        static const char domain[] = "glacier-continuation-paged-kv-page-image-v1";
        gh::Sha256 h;
        h.update(domain, sizeof domain);  // the trailing NUL is part of the domain
        h.update(m.data(), m.size() - 32);
        h.final(m.data() + m.size() - 32);
      }
    }
    // decode reads only `len` bytes: copy into an exactly-sized heap buffer
    std::vector<uint8_t> exact(m.begin(), m.end());
    int rc = glacier_hip_page_image_decode(exact.empty() ? nullptr : exact.data(), exact.size(),
                                           challenge, &info);
    CHECK(rc == GLACIER_HIP_OK || info.error != GLACIER_HIP_PAGE_IMAGE_OK);
    ++(rc == GLACIER_HIP_OK ? g_n.decoded : g_n.refused);
  }
}

void mode_pagedkv(uint64_t seed, int ops) {
  std::mt19937_64 rng(seed);
  const uint32_t layers = 2, kvd = 8, max_seq = 80, pool = 6;
  glacier_hip_kv_pages *p = glacier_hip_kv_pages_create(layers, kvd, max_seq, pool);
  CHECK(p != nullptr);
  uint64_t last_root_gen = 1;
  uint8_t challenge[32];
  for (int i = 0; i < 32; ++i) challenge[i] = (uint8_t)(i + 1);
  for (int op = 0; op < ops; ++op) {
    glacier_hip_page_map_root_t root;
    glacier_hip_kv_pages_root(p, &root);
    const int what = (int)(rng() % 10);
    if (what < 7) {  // one row: begin, then commit or abort
      glacier_hip_row_txn_mark_t mark;
      int rc = glacier_hip_kv_pages_begin_row(p, &mark);
      if (rc == GLACIER_HIP_CACHE_FULL) {
        CHECK(root.committed_len == max_seq || root.committed_pages >= pool);
        CHECK(glacier_hip_kv_pages_reset(p) == GLACIER_HIP_OK);
        ++g_n.resets;
        continue;
      }
      CHECK(rc == GLACIER_HIP_OK);
      CHECK(mark.root_after_generation > last_root_gen);
      // a second begin while staged is refused
      glacier_hip_row_txn_mark_t m2;
      CHECK(glacier_hip_kv_pages_begin_row(p, &m2) == GLACIER_HIP_TRANSACTION_ACTIVE);
      glacier_hip_page_map_root_t b, a;
      CHECK(glacier_hip_kv_pages_staged_root(p, &mark, &b, &a) == GLACIER_HIP_OK);
      CHECK(memcmp(&b, &root, sizeof b) == 0);
      glacier_hip_row_txn_mark_t wrong = mark;
      wrong.generation += 1;
      CHECK(glacier_hip_kv_pages_commit_row(p, &wrong) == GLACIER_HIP_INVALID_TRANSACTION);
      last_root_gen = mark.root_after_generation;
      if (rng() % 4 == 0) {
        CHECK(glacier_hip_kv_pages_abort_row(p, &mark) == GLACIER_HIP_OK);
        glacier_hip_page_map_root_t r2;
        glacier_hip_kv_pages_root(p, &r2);
        CHECK(memcmp(&r2, &root, sizeof r2) == 0);  // nothing published
        ++g_n.aborts;
      } else {
        CHECK(glacier_hip_kv_pages_commit_row(p, &mark) == GLACIER_HIP_OK);
        glacier_hip_page_map_root_t r2;
        glacier_hip_kv_pages_root(p, &r2);
        CHECK(memcmp(&r2, &a, sizeof r2) == 0 && r2.committed_len == root.committed_len + 1);
        CHECK(glacier_hip_kv_pages_validate_page_ref(p, &mark.page_ref) == GLACIER_HIP_OK);
        ++g_n.commits;
      }
    } else if (what == 7) {
      CHECK(glacier_hip_kv_pages_reset(p) == GLACIER_HIP_OK);
      ++g_n.resets;
    } else {  // page images of every committed page, then a fuzzed decode
      if (root.committed_len == 0) continue;
      for (uint64_t lp = 0; lp < root.committed_pages; ++lp) {
        int32_t phys;
        uint64_t gen;
        CHECK(glacier_hip_kv_pages_page(p, (uint32_t)lp, &phys, &gen) == GLACIER_HIP_OK);
        const uint64_t rows = gpi::expected_rows(root, lp);
        const uint64_t nbytes = glacier_hip_page_image_bytes(layers, kvd, rows);
        CHECK(nbytes > 0);
        std::vector<uint8_t> payload((size_t)(nbytes - 240));
        for (auto &x : payload) x = (uint8_t)rng();
        glacier_hip_page_ref_t ref = {0x4750524600000001ull, root.cache_instance, lp, gen};
        std::vector<uint8_t> img((size_t)nbytes);
        uint64_t len = 0;
        glacier_hip_page_image_v1_t info;
        // a too-small destination is refused before anything is written
        int rc = glacier_hip_page_image_encode_canonical(&root, layers, kvd, max_seq, &ref, rows,
                                                         payload.data(), payload.size(), challenge,
                                                         img.data(), nbytes - 1, &len, &info);
        CHECK(rc != GLACIER_HIP_OK);
        rc = glacier_hip_page_image_encode_canonical(&root, layers, kvd, max_seq, &ref, rows,
                                                     payload.data(), payload.size(), challenge,
                                                     img.data(), nbytes, &len, &info);
        CHECK(rc == GLACIER_HIP_OK && len == nbytes);
        ++g_n.images;
        image_fuzz(img, challenge, rng);
      }
    }
    glacier_hip_kv_resident_ledger_t led;
    CHECK(glacier_hip_kv_pages_ledger(p, &led) == GLACIER_HIP_OK);
    CHECK(led.allocated_pages <= pool);
    int32_t phys;
    CHECK(glacier_hip_kv_pages_page(p, 1000, &phys, nullptr) == GLACIER_HIP_SHAPE_MISMATCH);
  }
  glacier_hip_kv_pages_destroy(p);
  // geometry limits of the codec
  CHECK(glacier_hip_page_image_bytes(0, 8, 1) == 0);
  CHECK(glacier_hip_page_image_bytes(2, 8, 17) == 0);
  CHECK(glacier_hip_page_image_bytes(~0ull, ~0ull, 16) == 0);
  // publication digests over arbitrary records
  glacier_hip_token_proposal_v1_t prop;
  uint8_t *raw = (uint8_t *)&prop;
  for (size_t i = 0; i < sizeof prop; ++i) raw[i] = (uint8_t)rng();
  uint8_t d1[32], d2[32];
  CHECK(glacier_hip_token_proposal_sha256(&prop, d1) == GLACIER_HIP_OK);
  glacier_hip_prepare_ack_v1_t ack;
  memset(&ack, 0, sizeof ack);
  memcpy(ack.proposal_sha256, d1, 32);
  ack.sink_epoch = 1;
  ack.reservation_id = 2;
  CHECK(glacier_hip_token_commit_sha256(d1, &ack, d2) == GLACIER_HIP_OK);
  CHECK(glacier_hip_token_proposal_sha256(nullptr, d1) == GLACIER_HIP_INVALID_ARGUMENT);
}

// --------------------------------------------------------------- glrt ----
uint64_t walk(glacier_hip_glrt_image *img) {
  uint64_t sum = 0;
  for (uint64_t i = 0;; ++i) {
    glacier_hip_glrt_record_t r;
    if (glacier_hip_glrt_record_at(img, i, &r) != GLACIER_HIP_OK) break;
    for (uint32_t s = 0; s < 5; ++s) {
      const void *data = nullptr;
      uint64_t len = 0;
      if (glacier_hip_glrt_stream(img, &r, s, &data, &len) != GLACIER_HIP_OK) continue;
      const uint8_t *b = (const uint8_t *)data;
      for (uint64_t k = 0; k < len; ++k) sum += b[k];  // every byte of every view
    }
    glacier_hip_glrt_record_t f;
    glacier_hip_glrt_find(img, r.layer_idx, r.kind, r.role, &f);
  }
  glacier_hip_glrt_record_t r;
  memset(&r, 0, sizeof r);
  const void *data = nullptr;
  uint64_t len = 0;
  if (glacier_hip_glrt_stream(img, &r, 99, &data, &len) == GLACIER_HIP_OK) ++g_fail;
  uint8_t id[32];
  uint64_t bytes = 0;
  glacier_hip_glrt_identity(img, id, &bytes);
  return sum + bytes;
}

std::vector<uint8_t> slurp(const char *path) {
  std::vector<uint8_t> v;
  FILE *fp = fopen(path, "rb");
  if (!fp) return v;
  fseek(fp, 0, SEEK_END);
  long n = ftell(fp);
  fseek(fp, 0, SEEK_SET);
  v.resize((size_t)n);
  if (n > 0 && fread(v.data(), 1, (size_t)n, fp) != (size_t)n) v.clear();
  fclose(fp);
  return v;
}

// The first `nvalid` paths are valid images: each is opened and walked, then
// mutated copies of it (bytes flipped, truncated, fields replaced; CRCs not
// repaired) are opened. The remaining paths are arbitrary images (edited
// with repaired CRCs by the caller): each is opened and walked if it opens.
void mode_glrt(uint64_t seed, const char *tmp, int nvalid, int nimg, char **paths) {
  std::mt19937_64 rng(seed);
  const std::string mut = std::string(tmp) + "/mutated.glrt";
  int opened = 0, rejected = 0;
  for (int i = nvalid; i < nimg; ++i) {
    for (int check = 0; check < 2; ++check) {
      glacier_hip_glrt_open_options_t opts;
      memset(&opts, 0, sizeof opts);
      opts.verify_payload_crc = check;
      opts.verify_payload_digest = check;
      opts.allow_v1 = 1;
      glacier_hip_glrt_image *img = nullptr;
      glacier_hip_glrt_info_t info;
      if (glacier_hip_glrt_open(paths[i], &opts, &img, &info) == GLACIER_HIP_OK) {
        ++opened;
        walk(img);
        glacier_hip_glrt_close(img);
      } else {
        ++rejected;
        CHECK(img == nullptr && info.error != 0);
      }
    }
  }
  for (int i = 0; i < nvalid; ++i) {
    glacier_hip_glrt_image *img = nullptr;
    glacier_hip_glrt_info_t info;
    CHECK(glacier_hip_glrt_open(paths[i], nullptr, &img, &info) == GLACIER_HIP_OK);
    walk(img);
    glacier_hip_glrt_close(img);
    std::vector<uint8_t> orig = slurp(paths[i]);
    CHECK(!orig.empty());
    for (int k = 0; k < 60; ++k) {
      std::vector<uint8_t> m = orig;
      switch (k % 4) {
        case 0: m[rng() % 512] ^= (uint8_t)(1 + rng() % 255); break;       // header
        case 1: m[rng() % m.size()] ^= (uint8_t)(1 + rng() % 255); break;  // anywhere
        case 2: m.resize(rng() % m.size()); break;                          // truncated
        default: {  // an 8-byte field of the header or the index set to a random value
          size_t off = 8 * (rng() % std::min<size_t>(m.size() / 8, 256));
          uint64_t v = rng() % 3 == 0 ? ~0ull - rng() % 4096 : rng();
          memcpy(m.data() + off, &v, 8);
        }
      }
      FILE *fp = fopen(mut.c_str(), "wb");
      CHECK(fp != nullptr);
      if (!m.empty()) CHECK(fwrite(m.data(), 1, m.size(), fp) == m.size());
      fclose(fp);
      glacier_hip_glrt_open_options_t opts;
      memset(&opts, 0, sizeof opts);
      opts.verify_payload_crc = (int32_t)(rng() & 1);  // unchecked payloads still stay in bounds
      opts.verify_payload_digest = opts.verify_payload_crc;
      opts.allow_v1 = 1;
      img = nullptr;
      int rc = glacier_hip_glrt_open(mut.c_str(), &opts, &img, &info);
      if (rc == GLACIER_HIP_OK) {
        ++opened;
        walk(img);
        glacier_hip_glrt_close(img);
      } else {
        ++rejected;
        CHECK(img == nullptr && info.error != 0);
      }
    }
  }
  glacier_hip_glrt_image *img = nullptr;
  glacier_hip_glrt_info_t info;
  CHECK(glacier_hip_glrt_open((std::string(tmp) + "/absent.glrt").c_str(), nullptr, &img, &info) !=
        GLACIER_HIP_OK);
  printf("glrt opened=%d rejected=%d\n", opened, rejected);
}

}  // namespace

// Leased page maps: random rows, aborts, pool limits, seals, reclaims and
// renewals of two coordinators per tree; `threads` trees on one bank from
// their own threads (the bank's lock). Invariant after every step: the
// tree's kv charge equals the live bindings' bytes and the pages the maps hold.
std::atomic<long> g_lease_ops{0};

void lease_worker(glacier_hip_lease_bank *bank, uint64_t seed, int ops, int slot) {
  std::mt19937_64 rng(seed);
  glacier_hip_claim_t one{};
  one.queue_slots = 1;
  glacier_hip_bank_receipt_t res, parent;
  if (glacier_hip_lease_bank_reserve(bank, 100 + slot, &one, &res) ||
      glacier_hip_lease_bank_commit(bank, &res, &parent)) {
    ++g_fail;
    return;
  }
  glacier_hip_claim_t ceil{};
  ceil.kv_bytes = 16 * 128;
  glacier_hip_lease_tree_t tree;
  glacier_hip_lease_node_t scope[2];
  if (glacier_hip_lease_tree_open(bank, &parent, 7, 8, &ceil, &tree)) {
    ++g_fail;
    return;
  }
  ceil.kv_bytes = 8 * 128;
  for (int i = 0; i < 2; ++i)
    if (glacier_hip_lease_scope_open(bank, &tree, 20 + i, 30 + i, &ceil, &scope[i])) ++g_fail;
  const uint64_t epoch = 5, sid = 0x5000 + slot;
  uint64_t seq = 0;
  if (glacier_hip_lease_session_bind(bank, &tree, epoch, sid)) ++g_fail;
  glacier_hip_kv_pages *pages[2] = {};
  glacier_hip_leased_kv *lk[2] = {};
  std::vector<glacier_hip_page_lease_binding_t> bind[2];
  glacier_hip_leased_row_txn_t txn[2];
  bool staged[2] = {false, false}, sealed[2] = {false, false};
  glacier_hip_terminal_seal_t seal[2];
  auto renew = [&](int l) {
    if (lk[l]) glacier_hip_leased_kv_destroy(lk[l]);
    if (pages[l]) glacier_hip_kv_pages_destroy(pages[l]);
    pages[l] = glacier_hip_kv_pages_create(1, 1, 64, 5);
    bind[l].assign(4, glacier_hip_page_lease_binding_t{});
    if (glacier_hip_leased_kv_create(bank, &tree, &scope[l], pages[l], bind[l].data(), 4, epoch,
                                     sid, &seq, &lk[l]))
      ++g_fail;
    staged[l] = sealed[l] = false;
  };
  renew(0);
  renew(1);
  long done = 0;
  for (int i = 0; i < ops; ++i) {
    const int l = (int)(rng() % 2), r = (int)(rng() % 100);
    if (r < 60) {
      if (!staged[l]) {
        glacier_hip_leased_row_plan_t plan;
        if (!glacier_hip_leased_kv_plan_next_row(lk[l], &plan) &&
            !glacier_hip_leased_kv_begin_row(lk[l], &plan, &txn[l])) {
          const float k = (float)(rng() % 1000), v = -k;
          if (glacier_hip_kv_pages_append_row(pages[l], &txn[l].mark, 0, &k, &v)) ++g_fail;
          staged[l] = true;
        }
      } else {
        if (glacier_hip_leased_kv_commit_row(lk[l], &txn[l], nullptr)) ++g_fail;
        staged[l] = false;
      }
    } else if (r < 70 && staged[l]) {
      if (glacier_hip_leased_kv_abort_row(lk[l], &txn[l])) ++g_fail;
      staged[l] = false;
    } else if (r < 78) {
      glacier_hip_kv_pages_set_pool_capacity(pages[l], (uint32_t)(rng() % 6));
    } else if (r < 84 && !staged[l] && !sealed[l]) {
      glacier_hip_page_map_root_t root;
      uint8_t kv[32];
      if (!glacier_hip_leased_kv_root(lk[l], &root) && !glacier_hip_leased_kv_kv_sha256(lk[l], kv) &&
          !glacier_hip_leased_kv_seal_terminal(lk[l], &root, kv, seq, 0, 1, &seal[l]))
        sealed[l] = true;
    } else if (r < 90 && sealed[l]) {
      glacier_hip_freed_payload_t f;
      if (!glacier_hip_leased_kv_begin_reclaim(lk[l], &seal[l], seq, &f) &&
          glacier_hip_leased_kv_commit_reclaim(lk[l], &f, nullptr))
        ++g_fail;
    } else if (r < 94) {
      if (glacier_hip_leased_kv_reclaim_for_teardown(lk[l], seq) == GLACIER_HIP_LEASE_OK) staged[l] = false;
    } else {
      uint32_t life;
      glacier_hip_leased_kv_lifecycle(lk[l], &life);
      if (life == GLACIER_HIP_LEASE_RECLAIMED) renew(l);
    }
    // invariant: charge == live bindings == pages held
    uint64_t held = 0, bound = 0;
    for (int j = 0; j < 2; ++j) {
      glacier_hip_kv_resident_ledger_t led;
      glacier_hip_kv_pages_ledger(pages[j], &led);
      uint32_t life;
      glacier_hip_leased_kv_lifecycle(lk[j], &life);
      if (life != GLACIER_HIP_LEASE_FREED_PENDING_UNCHARGE) held += led.resident_tensor_payload_bytes;
      for (const auto &b : bind[j])
        if (b.state != GLACIER_HIP_BINDING_FREE) bound += b.payload_bytes;
    }
    if (tree.current.kv_bytes != held || bound != held) {
      fprintf(stderr, "lease invariant: tree %llu held %llu bound %llu at op %d\n",
              (unsigned long long)tree.current.kv_bytes, (unsigned long long)held,
              (unsigned long long)bound, i);
      ++g_fail;
      break;
    }
    ++done;
  }
  g_lease_ops += done;
  for (int l = 0; l < 2; ++l) {
    if (glacier_hip_leased_kv_reclaim_for_teardown(lk[l], seq) != GLACIER_HIP_LEASE_OK) {
      // a sealed lane is reclaimed through its seal
      glacier_hip_freed_payload_t f;
      if (!sealed[l] || glacier_hip_leased_kv_begin_reclaim(lk[l], &seal[l], seq, &f) ||
          glacier_hip_leased_kv_commit_reclaim(lk[l], &f, nullptr))
        ++g_fail;
    }
    glacier_hip_leased_kv_destroy(lk[l]);
    glacier_hip_kv_pages_destroy(pages[l]);
  }
  if (tree.current.kv_bytes != 0 || glacier_hip_lease_session_close(bank, &parent, epoch, sid, seq) ||
      glacier_hip_lease_tree_close(bank, &tree) || glacier_hip_lease_bank_release(bank, &parent))
    ++g_fail;
}

void mode_lease(uint64_t seed, int ops, int threads) {
  glacier_hip_limits_t lim;
  memset(&lim, 0xff, sizeof lim);
  glacier_hip_lease_bank *bank = glacier_hip_lease_bank_create(threads, 8 * threads, &lim, 77);
  std::vector<std::thread> ts;
  for (int t = 0; t < threads; ++t) ts.emplace_back(lease_worker, bank, seed + t, ops, t);
  for (auto &t : ts) t.join();
  glacier_hip_lease_bank_snapshot_t snap;
  glacier_hip_lease_bank_snapshot(bank, &snap);
  if (snap.used.kv_bytes || snap.used.queue_slots || snap.active_lease_nodes) ++g_fail;
  glacier_hip_lease_bank_destroy(bank);
}

int main(int argc, char **argv) {
  if (argc < 2) {
    fprintf(stderr, "usage: %s mode args...\n", argv[0]);
    return 2;
  }
  const std::string mode = argv[1];
  if (mode == "sha" && argc == 3) mode_sha(atoi(argv[2]));
  else if (mode == "f16" && argc == 3) mode_f16(argv[2]);
  else if (mode == "laneweave" && argc == 4) mode_laneweave(strtoull(argv[2], 0, 0), atoi(argv[3]));
  else if (mode == "threads" && argc == 4) mode_threads(strtoull(argv[2], 0, 0), atoi(argv[3]));
  else if (mode == "pagedkv" && argc == 4) mode_pagedkv(strtoull(argv[2], 0, 0), atoi(argv[3]));
  else if (mode == "lease" && argc == 5)
    mode_lease(strtoull(argv[2], 0, 0), atoi(argv[3]), atoi(argv[4]));
  else if (mode == "glrt" && argc >= 6)
    mode_glrt(strtoull(argv[2], 0, 0), argv[3], atoi(argv[4]), argc - 5, argv + 5);
  else {
    fprintf(stderr, "bad arguments\n");
    return 2;
  }
  if (mode == "laneweave" || mode == "threads")
    printf("admitted=%ld served=%ld waves=%ld failed_waves=%ld\n", g_n.admitted, g_n.served,
           g_n.waves, g_n.failed_waves);
  if (mode == "lease") printf("lease_ops=%ld\n", g_lease_ops.load());
  if (mode == "pagedkv")
    printf("commits=%ld aborts=%ld resets=%ld images=%ld decoded=%ld refused=%ld\n", g_n.commits,
           g_n.aborts, g_n.resets, g_n.images, g_n.decoded, g_n.refused);
  if (g_fail) fprintf(stderr, "%d check(s) failed\n", g_fail);
  return g_fail ? 1 : 0;
}
