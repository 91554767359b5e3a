// paged_kv.h — host-side page map of one request's paged KV cache.
//
// The device holds the page payloads in a pool shared by the lanes of a
// session; this module owns everything the reference's PagedKVCache keeps on
// the host (paged_kv_cache.zig:511-1520): logical page -> payload, the
// ownership generation of every page, the committed PageMapRootV1 and its
// SHA-256 ownership chain, and the row transaction
//   beginRow        paged_kv_cache.zig:1006-1072 (consumes the page and root
//                   generations whether or not the row later commits)
//   prepareCommit   :1105-1118
//   commit          :1122-1135
//   abortRow        :1146-1158 (only clears the page's ownership generation;
//                   the payload stays with the logical page and is reused
//                   by the retry under a fresh generation)
//   reset           :1162-1182
// A payload once taken from the pool stays with its logical page until the
// request ends (release), as the reference keeps `entries[i].payload`.
//
// Several rows of one lane may be staged together (a prompt chunk): row i
// starts from row i-1's staged root, exactly as i sequential single-row
// transactions would; for one row it is the reference's transaction.
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <vector>

#include "../../include/glacier_hip.h"

namespace gpk {

constexpr uint64_t kPagedKvAbi = 0x47504b5600000001ull;      // paged_kv_cache.zig:18
constexpr uint64_t kPageRefAbi = 0x4750524600000001ull;      // :19
constexpr uint64_t kPageMapRootAbi = 0x47504d5200000001ull;  // :20
constexpr uint64_t kRowTxnAbi = 0x4750525400000001ull;       // :21
constexpr uint32_t kPagePositions = 16;

using Root = glacier_hip_page_map_root_t;
using Mark = glacier_hip_row_txn_mark_t;

void empty_ownership_digest(uint64_t inst, uint64_t layers, uint64_t dim, uint64_t max_seq,
                            uint8_t out[32]);
void append_ownership_digest(const uint8_t before[32], uint64_t inst, uint64_t page,
                             uint64_t gen, uint8_t out[32]);
uint64_t next_cache_instance();  // reserveCacheInstance: process-wide, nonzero

// Free physical pages of a device pool (lowest id handed out first).
struct PagePool {
  std::vector<int32_t> free;  // stack: back() is the next page
  void init(uint32_t pages) {
    free.clear();
    for (uint32_t p = pages; p-- > 0;) free.push_back((int32_t)p);
  }
};

// One staged row.
struct RowTxn {
  uint32_t lane = 0;
  uint64_t pos = 0;
  bool installs = false;   // row 0 of a page: the page gets a new generation
  bool fresh_payload = false;  // the payload was taken from the pool by this row
  int32_t page = -1;       // physical page
  Mark mark{};
  Root before{}, after{};
};

// RetirementReclaimPlanV1 (paged_kv_cache.zig:135-146)
struct RetirePlan {
  uint64_t cache_id = 0, cache_instance = 0;
  Root root{};
  uint64_t committed_len = 0, allocated_pages = 0, page_payload_bytes = 0;
  uint64_t payload_bytes_to_free = 0, next_root_generation = 0;
};

class Cache {
 public:
  void init(uint64_t layers, uint64_t dim, uint64_t max_seq);
  // A new request: returns every payload to `pool`, new cache instance,
  // generations restart (PagedKVCache.init).
  void start(PagePool &pool);
  // Return every payload to the pool and deactivate.
  void release(PagePool &pool);

  // Payloads `n` more rows would take from the pool (0 if they fit pages the
  // cache already holds).
  uint32_t pages_needed(uint32_t n) const;
  // Stage `n` consecutive rows. Validation happens before anything changes:
  // TRANSACTION_ACTIVE, CACHE_FULL (max_seq or an empty pool), INVALID_TRANSACTION.
  int begin(uint32_t lane, uint32_t n, PagePool &pool, std::vector<RowTxn> &out);
  // Commit / abort the staged rows (all of them, in order).
  int commit(const RowTxn *txns, size_t n);
  int abort(const RowTxn *txns, size_t n);
  int reset();

  int validate_page_ref(const glacier_hip_page_ref_t &ref) const;
  void ledger(glacier_hip_kv_resident_ledger_t *out) const;
  uint64_t allocated_pages() const;

  // planNextRowAllocation (paged_kv_cache.zig:962-990): the next row's page
  // and the payload bytes it would take from the pool; lease status codes.
  int plan_next_row(glacier_hip_row_allocation_plan_t *out) const;
  // planRetirementReclaim (:1187-1214) / reclaimRetiredAfterCommit
  // (:1216-1250): every payload goes back to the pool, the root becomes an
  // empty one under a fresh generation and the map is retired for good.
  int plan_retirement(RetirePlan *out) const;
  int reclaim_retired(const RetirePlan &plan, PagePool &pool, uint64_t *freed_bytes);
  // claimLeasedCoordinator / isLeasedCoordinator (:910-932)
  bool claim_leased(uint64_t instance, uintptr_t owner);
  bool is_leased(uint64_t instance, uintptr_t owner) const {
    return instance && owner && leased_instance == instance && leased_owner == owner;
  }

  bool active = false;
  uint64_t instance = 0, len = 0, layers = 0, dim = 0, max_seq = 0;
  uint64_t next_page_generation = 1, next_root_generation = 2, next_row_txn_generation = 1;
  std::vector<int32_t> page_of;    // logical page -> physical page (-1 = no payload)
  std::vector<uint64_t> page_gen;  // ownership generation (0 = not owned)
  Root root{};
  uint32_t staged = 0;             // rows begun and not yet committed / aborted
  uint64_t page_payload_bytes = 0; // one page's K and V rows over every layer
  bool retired = false;
  uint64_t leased_instance = 0;    // the lease coordinator that owns the map
  uintptr_t leased_owner = 0;
};

bool same_mark(const Mark &a, const Mark &b);

}  // namespace gpk

// A host page map with its own pool (no device), behind glacier_hip_kv_pages_*.
struct glacier_hip_kv_pages {
  gpk::PagePool pool;
  gpk::Cache cache;
  std::vector<gpk::RowTxn> staged;
  std::vector<float> rows;  // [pool page][layer][K, V][16][kv_dim], written by append_row
};

namespace gpk {
// logicalKvSha256 of a host page map's committed rows; lease status codes.
int host_kv_sha256(const glacier_hip_kv_pages *p, uint8_t out[32]);
}  // namespace gpk
