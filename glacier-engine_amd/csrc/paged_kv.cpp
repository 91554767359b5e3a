// paged_kv.cpp — host page map and row transaction of a paged KV cache
// (paged_kv_cache.zig:511-1520), plus the device-free C ABI over it.
#include "paged_kv.h"

#include <string.h>

#include <atomic>
#include <new>

#include "host_util.h"

namespace gpk {

void empty_ownership_digest(uint64_t inst, uint64_t layers, uint64_t dim, uint64_t max_seq,
                            uint8_t out[32]) {
  // emptyOwnershipDigest, paged_kv_cache.zig:323-338
  gh::Sha256 h;
  h.update("glacier-paged-kv-ownership-v1\0", 30);
  h.u64(inst);
  h.u64(layers);
  h.u64(dim);
  h.u64(max_seq);
  h.u64(kPagePositions);
  h.final(out);
}

void append_ownership_digest(const uint8_t before[32], uint64_t inst, uint64_t page,
                             uint64_t gen, uint8_t out[32]) {
  // appendOwnershipDigest over the PageRefV1 fields, paged_kv_cache.zig:341-353
  gh::Sha256 h;
  h.update("glacier-paged-kv-root-append-v1\0", 32);
  h.update(before, 32);
  h.u64(kPageRefAbi);
  h.u64(inst);
  h.u64(page);
  h.u64(gen);
  h.final(out);
}

uint64_t next_cache_instance() {
  static std::atomic<uint64_t> next{1};
  return next.fetch_add(1);
}

void Cache::init(uint64_t L, uint64_t d, uint64_t seq) {
  layers = L;
  dim = d;
  max_seq = seq;
  const size_t pages = (seq + kPagePositions - 1) / kPagePositions;
  page_of.assign(pages, -1);
  page_gen.assign(pages, 0);
  page_payload_bytes = L * 2 * kPagePositions * d * 4;  // f32 rows unless the owner says otherwise
  active = false;
}

void Cache::release(PagePool &pool) {
  for (auto &p : page_of)
    if (p >= 0) {
      pool.free.push_back(p);
      p = -1;
    }
  for (auto &g : page_gen) g = 0;
  staged = 0;
  active = false;
}

void Cache::start(PagePool &pool) {
  release(pool);
  active = true;
  retired = false;
  instance = next_cache_instance();
  len = 0;
  next_page_generation = 1;
  next_root_generation = 2;
  next_row_txn_generation = 1;
  root = Root{};
  root.abi_version = kPageMapRootAbi;
  root.cache_instance = instance;
  root.generation = 1;
  empty_ownership_digest(instance, layers, dim, max_seq, root.ownership_sha256);
}

uint32_t Cache::pages_needed(uint32_t n) const {
  uint32_t need = 0;
  for (uint64_t pos = len; pos < len + n && pos < max_seq; ++pos)
    if (pos % kPagePositions == 0 && page_of[pos / kPagePositions] < 0) ++need;
  return need;
}

int Cache::begin(uint32_t lane, uint32_t n, PagePool &pool, std::vector<RowTxn> &out) {
  // validateNextRowState (paged_kv_cache.zig:1386-1419), for every row
  // before any state changes
  if (!active || retired || n == 0) return GLACIER_HIP_INVALID_TRANSACTION;
  if (staged) return GLACIER_HIP_TRANSACTION_ACTIVE;
  if (len + n > max_seq) return GLACIER_HIP_CACHE_FULL;
  if (root.committed_len != len || root.cache_instance != instance) return GLACIER_HIP_INVALID_TRANSACTION;
  const uint64_t expect_pages = len / kPagePositions + (len % kPagePositions != 0);
  if (root.committed_pages != expect_pages) return GLACIER_HIP_INVALID_TRANSACTION;
  for (uint64_t pos = len; pos < len + n; ++pos) {
    const uint64_t p = pos / kPagePositions;
    if (pos % kPagePositions == 0) {
      if (page_gen[p] != 0) return GLACIER_HIP_INVALID_TRANSACTION;
    } else if (pos == len && (page_of[p] < 0 || page_gen[p] == 0)) {
      return GLACIER_HIP_INVALID_TRANSACTION;
    }
  }
  if (pages_needed(n) > pool.free.size()) return GLACIER_HIP_CACHE_FULL;

  // beginRowInternal (:1011-1072), row after row
  const size_t first = out.size();
  out.reserve(first + n);
  for (uint32_t i = 0; i < n; ++i) {
    RowTxn t;
    t.lane = lane;
    t.pos = len + i;
    const uint64_t p = t.pos / kPagePositions;
    t.installs = t.pos % kPagePositions == 0;
    if (t.installs) {
      if (page_of[p] < 0) {  // allocate the payload; kept by the page from now on
        page_of[p] = pool.free.back();
        pool.free.pop_back();
        t.fresh_payload = true;
      }
      page_gen[p] = next_page_generation++;
    }
    t.page = page_of[p];
    t.before = i == 0 ? root : out[first + i - 1].after;
    t.after.abi_version = kPageMapRootAbi;
    t.after.cache_instance = instance;
    t.after.generation = next_root_generation++;
    t.after.committed_len = t.pos + 1;
    t.after.committed_pages = t.before.committed_pages + (t.installs ? 1 : 0);
    if (t.installs)
      append_ownership_digest(t.before.ownership_sha256, instance, p, page_gen[p],
                              t.after.ownership_sha256);
    else
      memcpy(t.after.ownership_sha256, t.before.ownership_sha256, 32);
    t.mark.abi_version = kRowTxnAbi;
    t.mark.cache_id = (uint64_t)(uintptr_t)this;
    t.mark.cache_instance = instance;
    t.mark.generation = next_row_txn_generation++;
    t.mark.base_len = t.pos;
    t.mark.row_count = 1;
    t.mark.root_before_generation = t.before.generation;
    t.mark.root_after_generation = t.after.generation;
    t.mark.page_ref.abi_version = kPageRefAbi;
    t.mark.page_ref.cache_instance = instance;
    t.mark.page_ref.logical_page = p;
    t.mark.page_ref.ownership_generation = page_gen[p];
    out.push_back(t);
  }
  staged = n;
  return GLACIER_HIP_OK;
}

bool same_mark(const Mark &a, const Mark &b) { return memcmp(&a, &b, sizeof a) == 0; }

int Cache::commit(const RowTxn *txns, size_t n) {
  // commitPreparedAssumeValid (:1122-1135) after prepareCommit's checks
  if (n == 0 || n != staged) return GLACIER_HIP_INVALID_TRANSACTION;
  for (size_t i = 0; i < n; ++i) {
    const RowTxn &t = txns[i];
    if (t.mark.cache_id != (uint64_t)(uintptr_t)this || t.mark.cache_instance != instance ||
        t.pos != len + i || t.mark.base_len != t.pos ||
        page_gen[t.pos / kPagePositions] != t.mark.page_ref.ownership_generation ||
        t.mark.page_ref.ownership_generation == 0)
      return GLACIER_HIP_INVALID_TRANSACTION;
  }
  if (memcmp(&txns[0].before, &root, sizeof root) != 0) return GLACIER_HIP_INVALID_TRANSACTION;
  root = txns[n - 1].after;
  len += n;
  staged = 0;
  return GLACIER_HIP_OK;
}

int Cache::abort(const RowTxn *txns, size_t n) {
  // abortRow (:1146-1158): an installed page loses its ownership generation;
  // the payload, the consumed generations and the committed root stay.
  if (n == 0 || n != staged) return GLACIER_HIP_INVALID_TRANSACTION;
  for (size_t i = n; i-- > 0;) {
    const RowTxn &t = txns[i];
    if (t.mark.cache_id != (uint64_t)(uintptr_t)this || t.mark.cache_instance != instance ||
        t.pos != len + i)
      return GLACIER_HIP_INVALID_TRANSACTION;
    if (t.installs) {
      const uint64_t p = t.pos / kPagePositions;
      if (page_gen[p] != t.mark.page_ref.ownership_generation) return GLACIER_HIP_INVALID_TRANSACTION;
      page_gen[p] = 0;
    }
  }
  staged = 0;
  return GLACIER_HIP_OK;
}

int Cache::reset() {
  // reset (:1162-1182): every page ref and root becomes stale, payloads stay
  if (!active || retired) return GLACIER_HIP_INVALID_TRANSACTION;
  if (staged) return GLACIER_HIP_TRANSACTION_ACTIVE;
  for (auto &g : page_gen) g = 0;
  root = Root{};
  root.abi_version = kPageMapRootAbi;
  root.cache_instance = instance;
  root.generation = next_root_generation++;
  empty_ownership_digest(instance, layers, dim, max_seq, root.ownership_sha256);
  len = 0;
  return GLACIER_HIP_OK;
}

int Cache::validate_page_ref(const glacier_hip_page_ref_t &ref) const {
  // validateCommittedPageRef (:944-957)
  if (ref.abi_version != kPageRefAbi || ref.cache_instance != instance ||
      ref.logical_page >= root.committed_pages || ref.logical_page >= page_of.size())
    return GLACIER_HIP_INVALID_TRANSACTION;
  const size_t p = (size_t)ref.logical_page;
  if (page_of[p] < 0 || page_gen[p] == 0 || page_gen[p] != ref.ownership_generation)
    return GLACIER_HIP_INVALID_TRANSACTION;
  return GLACIER_HIP_OK;
}

void Cache::ledger(glacier_hip_kv_resident_ledger_t *o) const {
  // allocationCommitmentLedger (:840-892)
  memset(o, 0, sizeof *o);
  const uint64_t allocated = allocated_pages();
  uint64_t provisional = 0;
  // a staged row that installed a page holds it provisionally
  if (staged)
    for (uint64_t pos = len; pos < len + staged; ++pos)
      if (pos % kPagePositions == 0) ++provisional;
  const uint64_t page_payload = page_payload_bytes;
  o->page_count_capacity = page_of.size();
  o->allocated_pages = allocated;
  o->committed_pages = root.committed_pages;
  o->provisional_pages = provisional;
  o->reusable_pages = allocated - root.committed_pages - provisional;
  o->page_map_bytes = page_of.size() * 16;
  o->resident_tensor_payload_bytes = allocated * page_payload;
  o->resident_allocation_bytes = o->page_map_bytes + o->resident_tensor_payload_bytes;
  o->committed_tensor_payload_bytes = layers * 2 * len * dim * (page_payload / (layers * 2 * kPagePositions * dim));
}

uint64_t Cache::allocated_pages() const {
  uint64_t n = 0;
  for (int32_t p : page_of) n += p >= 0;
  return n;
}

int Cache::plan_next_row(glacier_hip_row_allocation_plan_t *o) const {
  // planNextRowAllocation (:962-990) after validateNextRowState (:1386-1419)
  if (retired) return GLACIER_HIP_LEASE_CACHE_RETIRED;
  if (!active) return GLACIER_HIP_LEASE_INVALID_TRANSACTION;
  if (staged) return GLACIER_HIP_LEASE_TRANSACTION_ACTIVE;
  if (len >= max_seq) return GLACIER_HIP_LEASE_CACHE_FULL;
  if (root.committed_len != len || root.cache_instance != instance) return GLACIER_HIP_LEASE_INVALID_ROOT;
  const uint64_t p = len / kPagePositions, row = len % kPagePositions;
  if (p >= page_of.size()) return GLACIER_HIP_LEASE_CACHE_FULL;
  if (root.committed_pages != p + (row != 0)) return GLACIER_HIP_LEASE_INVALID_ROOT;
  const bool installs = row == 0;
  if (installs ? page_gen[p] != 0 : (page_of[p] < 0 || page_gen[p] == 0))
    return GLACIER_HIP_LEASE_INVALID_ROOT;
  memset(o, 0, sizeof *o);
  o->abi_version = 0x4750415000000001ull;  // row_allocation_plan_abi
  o->cache_id = (uint64_t)(uintptr_t)this;
  o->cache_instance = instance;
  o->base_len = len;
  o->logical_page = p;
  o->row_in_page = row;
  o->root_generation = root.generation;
  o->row_txn_generation = next_row_txn_generation;
  o->root_after_generation = next_root_generation;
  o->page_ownership_generation = page_gen[p];
  o->next_page_ownership_generation = next_page_generation;
  o->allocated_pages = allocated_pages();
  o->page_payload_present = page_of[p] >= 0;
  o->allocation_bytes = installs && page_of[p] < 0 ? page_payload_bytes : 0;
  return GLACIER_HIP_LEASE_OK;
}

int Cache::plan_retirement(RetirePlan *o) const {
  // planRetirementReclaim (:1187-1214) with validateRetirementCommitment:
  // committed pages own payload and a generation, later pages own none
  if (retired) return GLACIER_HIP_LEASE_CACHE_RETIRED;
  if (!active) return GLACIER_HIP_LEASE_INVALID_TRANSACTION;
  if (staged) return GLACIER_HIP_LEASE_TRANSACTION_ACTIVE;
  if (root.cache_instance != instance || root.committed_len != len ||
      root.committed_pages != (len + kPagePositions - 1) / kPagePositions)
    return GLACIER_HIP_LEASE_INVALID_ROOT;
  for (size_t p = 0; p < page_of.size(); ++p) {
    const bool committed = p < root.committed_pages;
    if (committed ? (page_of[p] < 0 || page_gen[p] == 0) : page_gen[p] != 0)
      return GLACIER_HIP_LEASE_INVALID_ROOT;
  }
  *o = RetirePlan{};
  o->cache_id = (uint64_t)(uintptr_t)this;
  o->cache_instance = instance;
  o->root = root;
  o->committed_len = len;
  o->allocated_pages = allocated_pages();
  o->page_payload_bytes = page_payload_bytes;
  o->payload_bytes_to_free = o->allocated_pages * page_payload_bytes;
  o->next_root_generation = next_root_generation;
  return GLACIER_HIP_LEASE_OK;
}

int Cache::reclaim_retired(const RetirePlan &plan, PagePool &pool, uint64_t *freed_bytes) {
  // reclaimRetiredAfterCommit (:1216-1250)
  RetirePlan want;
  if (int rc = plan_retirement(&want)) return rc;
  if (memcmp(&want, &plan, sizeof plan) != 0) return GLACIER_HIP_LEASE_INVALID_TRANSACTION;
  for (auto &p : page_of)
    if (p >= 0) {
      pool.free.push_back(p);
      p = -1;
    }
  for (auto &g : page_gen) g = 0;
  root = Root{};
  root.abi_version = kPageMapRootAbi;
  root.cache_instance = instance;
  root.generation = next_root_generation++;
  empty_ownership_digest(instance, layers, dim, max_seq, root.ownership_sha256);
  len = 0;
  retired = true;
  *freed_bytes = plan.payload_bytes_to_free;
  return GLACIER_HIP_LEASE_OK;
}

bool Cache::claim_leased(uint64_t inst, uintptr_t owner) {
  if (!inst || !owner || retired || leased_instance || leased_owner) return false;
  leased_instance = inst;
  leased_owner = owner;
  return true;
}

}  // namespace gpk

// ---------------------------------------------------------------------------
// C ABI: a host page map with its own pool (no device). It carries the same
// row transaction the sessions run for their lanes, for hosts that stage rows
// themselves and for tests.
// ---------------------------------------------------------------------------
namespace gpk {
// logicalKvSha256 (paged_kv_cache.zig:1347-1350, hashLogicalPrefix :1532-1555)
// of a host page map's committed rows.
int host_kv_sha256(const glacier_hip_kv_pages *p, uint8_t out[32]) {
  const Cache &c = p->cache;
  if (c.retired) return GLACIER_HIP_LEASE_CACHE_RETIRED;
  const size_t L = c.layers, d = c.dim;
  gh::Sha256 h;
  h.update("glacier-logical-kv-state-v1\0", 28);
  h.u64(L);
  h.u64(d);
  h.u64(c.len);
  for (size_t l = 0; l < L; ++l)
    for (int v = 0; v < 2; ++v)
      for (uint64_t pos = 0; pos < c.len; ++pos) {
        const int32_t phys = c.page_of[pos / kPagePositions];
        if (phys < 0) return GLACIER_HIP_LEASE_INVALID_ROOT;
        const float *row = p->rows.data() +
                           ((((size_t)phys * L + l) * 2 + v) * kPagePositions + pos % kPagePositions) * d;
        for (size_t i = 0; i < d; ++i) {
          uint32_t b;
          memcpy(&b, row + i, 4);
          h.u32(b);
        }
      }
  h.final(out);
  return GLACIER_HIP_LEASE_OK;
}
}  // namespace gpk

extern "C" {

glacier_hip_kv_pages *glacier_hip_kv_pages_create(uint32_t num_layers, uint32_t kv_dim,
                                                  uint32_t max_seq, uint32_t pool_pages) {
  if (num_layers == 0 || kv_dim == 0 || max_seq == 0 || pool_pages == 0) return nullptr;
  auto *p = new (std::nothrow) glacier_hip_kv_pages();
  if (!p) return nullptr;
  p->pool.init(pool_pages);
  p->cache.init(num_layers, kv_dim, max_seq);
  p->cache.start(p->pool);
  p->rows.assign((size_t)pool_pages * num_layers * 2 * gpk::kPagePositions * kv_dim, 0.f);
  return p;
}

int glacier_hip_kv_pages_append_row(glacier_hip_kv_pages *p, const glacier_hip_row_txn_mark_t *mark,
                                    uint32_t layer, const float *k, const float *v) {
  // appendRowTxn (paged_kv_cache.zig:1074-1103): the staged row's K and V at one layer
  if (!p || !mark || !k || !v) return GLACIER_HIP_INVALID_ARGUMENT;
  if (p->staged.size() != 1 || !gpk::same_mark(p->staged[0].mark, *mark))
    return GLACIER_HIP_INVALID_TRANSACTION;
  if (layer >= p->cache.layers) return GLACIER_HIP_SHAPE_MISMATCH;
  const gpk::RowTxn &t = p->staged[0];
  const size_t L = p->cache.layers, d = p->cache.dim, r = t.pos % gpk::kPagePositions;
  float *base = p->rows.data() + (((size_t)t.page * L + layer) * 2) * gpk::kPagePositions * d;
  memcpy(base + r * d, k, d * 4);
  memcpy(base + (gpk::kPagePositions + r) * d, v, d * 4);
  return GLACIER_HIP_OK;
}

int glacier_hip_kv_pages_kv_sha256(glacier_hip_kv_pages *p, uint8_t out[32]) {
  if (!p || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  return gpk::host_kv_sha256(p, out) ? GLACIER_HIP_INVALID_TRANSACTION : GLACIER_HIP_OK;
}

int glacier_hip_kv_pages_is_retired(glacier_hip_kv_pages *p, int32_t *out) {
  if (!p || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  *out = p->cache.retired;
  return GLACIER_HIP_OK;
}

void glacier_hip_kv_pages_destroy(glacier_hip_kv_pages *p) { delete p; }

int glacier_hip_kv_pages_begin_row(glacier_hip_kv_pages *p, glacier_hip_row_txn_mark_t *mark_out) {
  if (!p || !mark_out) return GLACIER_HIP_INVALID_ARGUMENT;
  std::vector<gpk::RowTxn> t;
  int rc = p->cache.begin(0, 1, p->pool, t);
  if (rc) return rc;
  p->staged = t;
  *mark_out = t[0].mark;
  return GLACIER_HIP_OK;
}

int glacier_hip_kv_pages_commit_row(glacier_hip_kv_pages *p, const glacier_hip_row_txn_mark_t *mark) {
  if (!p || !mark) return GLACIER_HIP_INVALID_ARGUMENT;
  if (p->staged.size() != 1 || !gpk::same_mark(p->staged[0].mark, *mark))
    return GLACIER_HIP_INVALID_TRANSACTION;
  int rc = p->cache.commit(p->staged.data(), 1);
  if (!rc) p->staged.clear();
  return rc;
}

int glacier_hip_kv_pages_abort_row(glacier_hip_kv_pages *p, const glacier_hip_row_txn_mark_t *mark) {
  if (!p || !mark) return GLACIER_HIP_INVALID_ARGUMENT;
  if (p->staged.size() != 1 || !gpk::same_mark(p->staged[0].mark, *mark))
    return GLACIER_HIP_INVALID_TRANSACTION;
  int rc = p->cache.abort(p->staged.data(), 1);
  if (!rc) p->staged.clear();
  return rc;
}

int glacier_hip_kv_pages_staged_root(glacier_hip_kv_pages *p, const glacier_hip_row_txn_mark_t *mark,
                                     glacier_hip_page_map_root_t *before,
                                     glacier_hip_page_map_root_t *after) {
  // prepareCommit (:1105-1118): the roots the staged row moves between
  if (!p || !mark) return GLACIER_HIP_INVALID_ARGUMENT;
  if (p->staged.size() != 1 || !gpk::same_mark(p->staged[0].mark, *mark))
    return GLACIER_HIP_INVALID_TRANSACTION;
  if (before) *before = p->staged[0].before;
  if (after) *after = p->staged[0].after;
  return GLACIER_HIP_OK;
}

int glacier_hip_kv_pages_reset(glacier_hip_kv_pages *p) {
  if (!p) return GLACIER_HIP_INVALID_ARGUMENT;
  return p->cache.reset();
}

int glacier_hip_kv_pages_root(glacier_hip_kv_pages *p, glacier_hip_page_map_root_t *out) {
  if (!p || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  *out = p->cache.root;
  return GLACIER_HIP_OK;
}

int glacier_hip_kv_pages_page(glacier_hip_kv_pages *p, uint32_t logical_page,
                              int32_t *physical_out, uint64_t *ownership_generation_out) {
  if (!p) return GLACIER_HIP_INVALID_ARGUMENT;
  if (logical_page >= p->cache.page_of.size()) return GLACIER_HIP_SHAPE_MISMATCH;
  if (physical_out) *physical_out = p->cache.page_of[logical_page];
  if (ownership_generation_out) *ownership_generation_out = p->cache.page_gen[logical_page];
  return GLACIER_HIP_OK;
}

int glacier_hip_kv_pages_validate_page_ref(glacier_hip_kv_pages *p, const glacier_hip_page_ref_t *ref) {
  if (!p || !ref) return GLACIER_HIP_INVALID_ARGUMENT;
  return p->cache.validate_page_ref(*ref);
}

int glacier_hip_kv_pages_ledger(glacier_hip_kv_pages *p, glacier_hip_kv_resident_ledger_t *out) {
  if (!p || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  p->cache.ledger(out);
  return GLACIER_HIP_OK;
}

}  // extern "C"
