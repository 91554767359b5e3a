// leased_kv.cpp — LeasedPagedKVCache over host page maps and session lanes
// (leased_paged_kv_cache.zig; line references per function).
#include "leased_kv.h"

#include <string.h>

#include <atomic>
#include <new>

#include "host_util.h"

namespace glb {

namespace {
std::atomic<uint64_t> g_next_instance{1};

int map_begin_error(int rc, bool allocates) {
  // the page map's begin errors in the lease domain; an empty pool while
  // taking a payload is the allocator's OutOfMemory
  switch (rc) {
    case GLACIER_HIP_CACHE_FULL: return allocates ? GLACIER_HIP_LEASE_OUT_OF_MEMORY : GLACIER_HIP_LEASE_CACHE_FULL;
    case GLACIER_HIP_TRANSACTION_ACTIVE: return GLACIER_HIP_LEASE_TRANSACTION_ACTIVE;
    default: return GLACIER_HIP_LEASE_INVALID_TRANSACTION;
  }
}

Claim kv_claim(uint64_t bytes) {
  Claim c{};
  c.kv_bytes = bytes;
  return c;
}

bool claim_is_exact_kv(const Claim &c, uint64_t bytes) {
  Claim want = kv_claim(bytes);
  return claim_eq(c, want);
}

uint64_t mix_root(uint64_t h, const Root &r) {
  h = mix64(h ^ r.abi_version);
  h = mix64(h ^ r.cache_instance);
  h = mix64(h ^ r.generation);
  h = mix64(h ^ r.committed_len);
  h = mix64(h ^ r.committed_pages);
  for (int i = 0; i < 32; i += 8) {
    uint64_t w;
    memcpy(&w, r.ownership_sha256 + i, 8);
    h = mix64(h ^ w);
  }
  return h;
}

uint64_t mix_bytes(uint64_t h, const uint8_t *b, size_t n) {
  for (size_t i = 0; i < n; i += 8) {
    uint64_t w = 0;
    memcpy(&w, b + i, n - i < 8 ? n - i : 8);
    h = mix64(h ^ w);
  }
  return h;
}

uint64_t mix_tree(uint64_t h, const Tree &t) {
  for (uint64_t v : {t.tree_key, t.identity_generation, t.generation, t.structural_revision,
                     (uint64_t)t.active_nodes, t.state_digest, t.integrity})
    h = mix64(h ^ v);
  h = mix_claim(h, t.current);
  return h;
}

uint64_t mix_summary(uint64_t h, const Summary &s) {
  h = mix64(h ^ s.count);
  h = mix64(h ^ s.payload_bytes);
  return mix_bytes(h, s.digest, 32);
}

uint64_t plan_integrity(const glacier_hip_leased_row_plan_t &p) {
  uint64_t h = mix64(kRowPlanAbi ^ p.coordinator_instance);
  h = mix_tree(h, p.tree);
  h = mix64(h ^ p.publication_sequence);
  h = mix_bytes(h, (const uint8_t *)&p.cache_plan, sizeof p.cache_plan);
  h = mix_summary(h, p.bindings);
  return h ? h : 1;
}

uint64_t txn_integrity(const glacier_hip_leased_row_txn_t &t) {
  uint64_t h = mix64(kRowTxnAbi ^ t.coordinator_instance);
  h = mix64(h ^ t.generation);
  h = mix_bytes(h, (const uint8_t *)&t.mark, sizeof t.mark);
  h = mix64(h ^ t.installed_new_binding);
  h = mix_bytes(h, t.bindings_digest, 32);
  return h ? h : 1;
}

uint64_t freed_integrity(const glacier_hip_freed_payload_t &f) {
  uint64_t h = mix64(kFreedPayloadAbi ^ f.coordinator_instance);
  h = mix64(h ^ f.generation);
  h = mix_bytes(h, f.terminal_seal_digest, 32);
  h = mix64(h ^ f.permit_generation);
  h = mix_root(h, f.root_before);
  h = mix_root(h, f.root_after);
  h = mix64(h ^ f.binding_count);
  h = mix64(h ^ f.payload_bytes);
  h = mix_bytes(h, f.bindings_digest, 32);
  return h ? h : 1;
}

void seal_digest(const glacier_hip_terminal_seal_t &s, uint8_t out[32]) {
  // terminalSealDigest: every field of the seal but the digest itself
  gh::Sha256 h;
  h.update("glacier-hip-terminal-seal-v1\0", 29);
  h.u64(s.abi_version);
  h.u64(s.coordinator_instance);
  h.u64(s.cache_id);
  h.u64(s.cache_instance);
  h.u32(s.scope_index);
  h.u64(s.scope_generation);
  h.u64(s.tree_identity_generation);
  h.u64(s.tree_generation);
  h.u64(s.tree_structural_revision);
  h.u64(s.tree_state_digest);
  h.update(&s.root, sizeof s.root);
  h.update(s.logical_kv_sha256, 32);
  h.u32(s.bindings.count);
  h.u64(s.bindings.payload_bytes);
  h.update(s.bindings.digest, 32);
  h.u64(s.transaction_sequence);
  h.u32(s.terminal_reason);
  h.u32(s.terminal_token);
  h.u64(s.generation);
  h.final(out);
}

void seal_digest_v3(const glacier_hip_terminal_seal_t &s, const uint8_t proposal[32],
                    const uint8_t commit[32], uint8_t out[32]) {
  // terminalSealV3Digest: the seal's fields and the wave's proposal and commit digests
  uint8_t base[32];
  seal_digest(s, base);
  gh::Sha256 h;
  h.update("glacier-hip-terminal-seal-v3\0", 29);
  h.update(base, 32);
  h.update(proposal, 32);
  h.update(commit, 32);
  h.final(out);
}

void teardown_digest(uint64_t instance, uint64_t sequence, const Root &root, const uint8_t kv[32],
                     const Summary &b, uint8_t out[32]) {
  gh::Sha256 h;
  h.update("glacier-hip-teardown-seal-v1\0", 29);
  h.u64(instance);
  h.u64(sequence);
  h.update(&root, sizeof root);
  h.update(kv, 32);
  h.u32(b.count);
  h.u64(b.payload_bytes);
  h.update(b.digest, 32);
  h.final(out);
}

bool same(const void *a, const void *b, size_t n) { return memcmp(a, b, n) == 0; }
}  // namespace

uint64_t page_binding_key(uint64_t cache_instance, uint64_t logical_page) {
  // pageBindingKey (:1353-1357)
  const uint64_t v = mix64(0x706167656c656166ull ^ cache_instance ^ mix64(logical_page + 1));
  return v ? v : 1;
}

uint64_t page_binding_integrity(const Binding &b) {
  // pageBindingIntegrity (:1369-1382)
  uint64_t r = mix64(kBindingAbi ^ b.state);
  r = mix64(r ^ b.cache_instance);
  r = mix64(r ^ b.logical_page);
  r = mix64(r ^ b.payload_bytes);
  r = mix64(r ^ (uint64_t)b.scope_index);
  r = mix64(r ^ b.scope_generation);
  if (b.has_leaf) {
    r = mix64(r ^ b.leaf.integrity);
    r = mix64(r ^ b.leaf.generation);
    r = mix64(r ^ (uint64_t)b.leaf.node_index);
  }
  return r;
}

Binding Leased::free_binding() const {
  Binding b;
  memset(&b, 0, sizeof b);
  b.abi_version = kBindingAbi;
  b.state = GLACIER_HIP_BINDING_FREE;
  b.scope_index = kNoNode;
  return b;
}

Binding Leased::live_binding(uint64_t logical_page, uint64_t payload_bytes, const Node &leaf) const {
  Binding b = free_binding();
  b.state = GLACIER_HIP_BINDING_LIVE;
  b.cache_instance = target.cache->instance;
  b.logical_page = logical_page;
  b.payload_bytes = payload_bytes;
  b.scope_index = scope.node_index;
  b.scope_generation = scope.generation;
  b.has_leaf = 1;
  b.leaf = leaf;
  b.integrity = page_binding_integrity(b);
  return b;
}

int Leased::init(Bank *b, Tree *t, const Node &sc, const Target &tg, Binding *bs, uint32_t count,
                 uint64_t epoch, uint64_t session, uint64_t *seq) {
  // init (:311-357)
  if (epoch == 0 || session == 0 || sc.kind != GLACIER_HIP_LEASE_NODE_SCOPE || sc.binding_key != 0)
    return GLACIER_HIP_LEASE_INVALID_COORDINATOR;
  if (count != tg.cache->page_of.size()) return GLACIER_HIP_LEASE_INVALID_BINDING_STORAGE;
  if (tg.cache->retired || tg.cache->allocated_pages() != 0 || tg.cache->root.committed_len != 0 ||
      tg.cache->root.committed_pages != 0 || tg.cache->staged)
    return GLACIER_HIP_LEASE_INVALID_COORDINATOR;
  if (int rc = b->validate_node(*t, sc)) return rc;
  const uint64_t inst = g_next_instance.fetch_add(1);
  if (!tg.cache->claim_leased(inst, (uintptr_t)this)) return GLACIER_HIP_LEASE_INVALID_COORDINATOR;
  bank = b;
  tree = t;
  scope = sc;
  target = tg;
  bindings = bs;
  binding_count = count;
  request_epoch = epoch;
  session_id = session;
  sequence = seq;
  instance = inst;
  const Binding fb = free_binding();
  for (uint32_t i = 0; i < count; ++i) bindings[i] = fb;
  return GLACIER_HIP_LEASE_OK;
}

int Leased::validate_mutable() {
  // validateMutable (:1090-1098)
  if (!leased_ok()) return GLACIER_HIP_LEASE_INVALID_COORDINATOR;
  if (reclaimed) return GLACIER_HIP_LEASE_RECLAIM_COMPLETE;
  if (has_pending) return GLACIER_HIP_LEASE_RECLAIM_PENDING;
  if (has_seal) return GLACIER_HIP_LEASE_ALREADY_TERMINAL;
  return bank->validate_node(*tree, scope);
}

int Leased::binding_summary(uint32_t state, Summary *out) {
  // bindingSummaryForState (:1178-1250)
  if (!leased_ok()) return GLACIER_HIP_LEASE_INVALID_COORDINATOR;
  if (int rc = bank->validate_node(*tree, scope)) return rc;
  const gpk::Cache &c = *target.cache;
  uint32_t count = 0;
  uint64_t bytes = 0;
  gh::Sha256 h;
  h.update("glacier-paged-lease-bindings-v1\0", 32);
  h.u64(instance);
  h.u64(c.root.cache_instance);
  h.u32(scope.node_index);
  h.u64(scope.generation);
  const Binding fb = free_binding();
  for (uint32_t i = 0; i < binding_count; ++i) {
    const Binding &b = bindings[i];
    if (b.state == GLACIER_HIP_BINDING_FREE) {
      if (!same(&b, &fb, sizeof b)) return GLACIER_HIP_LEASE_INVALID_BINDING;
      continue;
    }
    if (b.state != state || b.abi_version != kBindingAbi || b.cache_instance != c.root.cache_instance ||
        b.logical_page != i || b.payload_bytes == 0 || b.scope_index != scope.node_index ||
        b.scope_generation != scope.generation || b.integrity != page_binding_integrity(b) ||
        !b.has_leaf)
      return GLACIER_HIP_LEASE_INVALID_BINDING;
    const Node &leaf = b.leaf;
    if (leaf.kind != GLACIER_HIP_LEASE_NODE_ALLOCATION || leaf.parent_index != scope.node_index ||
        leaf.parent_generation != scope.generation || leaf.tenant_key != scope.tenant_key ||
        leaf.node_key != b.logical_page + 1 ||
        leaf.binding_key != page_binding_key(b.cache_instance, b.logical_page) ||
        !claim_is_exact_kv(leaf.claim, b.payload_bytes))
      return GLACIER_HIP_LEASE_INVALID_BINDING;
    if (int rc = bank->validate_node(*tree, leaf)) return rc;
    ++count;
    bytes += b.payload_bytes;
    h.u64(i);
    h.u64(b.integrity);
    h.u64(leaf.integrity);
    h.u64(leaf.generation);
    h.u32(leaf.node_index);
  }
  if (state == GLACIER_HIP_BINDING_LIVE &&
      (c.allocated_pages() != count || c.allocated_pages() * c.page_payload_bytes != bytes))
    return GLACIER_HIP_LEASE_INVALID_BINDING;
  memset(out, 0, sizeof *out);
  out->count = count;
  out->payload_bytes = bytes;
  h.final(out->digest);
  return GLACIER_HIP_LEASE_OK;
}

static void hash_claim_fields(gh::Sha256 &h, const glacier_hip_claim_t &c) {
  const uint64_t *f = &c.capsule_bytes;
  for (int i = 0; i < 10; ++i) h.u64(f[i]);
}

// hashLeaseNode (:1597-1616)
static void hash_lease_node(gh::Sha256 &h, const Node &n) {
  h.u64(n.abi_version);
  h.u64(n.parent.bank_epoch);
  h.u32((uint32_t)n.parent.slot_index);
  h.u64(n.parent.generation);
  h.u64(n.parent.owner_key);
  hash_claim_fields(h, n.parent.claim);
  h.u64(n.parent.integrity);
  h.u64(n.tree_key);
  h.u64(n.tree_identity_generation);
  h.u32(n.node_index);
  h.u64(n.generation);
  h.u32(n.parent_index);
  h.u64(n.parent_generation);
  h.u64(n.node_key);
  h.u64(n.tenant_key);
  h.u64(n.binding_key);
  const uint8_t kind = (uint8_t)n.kind;
  h.update(&kind, 1);
  hash_claim_fields(h, n.ceiling);
  hash_claim_fields(h, n.claim);
  h.u64(n.integrity);
}

int Leased::allocation_set(uint32_t state, glacier_hip_allocation_set_v2_t *out) {
  // allocationSetCommitmentForState (:1253-1291): the raw bindings with
  // their LeaseNode leaves, after the binding summary's checks
  Summary sum;
  if (int rc = binding_summary(state, &sum)) return rc;
  gh::Sha256 h;
  static const char dom[] = "glacier-paged-lease-allocation-set-v2";
  h.update(dom, sizeof dom);
  h.u64(0x47504C4100000002ull);  // allocation_set_abi (:29)
  h.u64(instance);
  h.u64(target.cache->root.cache_instance);
  h.u64(binding_count);
  hash_lease_node(h, scope);
  for (uint32_t i = 0; i < binding_count; ++i) {
    const Binding &b = bindings[i];
    if (b.state == GLACIER_HIP_BINDING_FREE) continue;
    h.u64(i);
    h.u64(b.abi_version);
    const uint8_t st = (uint8_t)b.state;
    h.update(&st, 1);
    h.u64(b.cache_instance);
    h.u64(b.logical_page);
    h.u64(b.payload_bytes);
    h.u32(b.scope_index);
    h.u64(b.scope_generation);
    h.u64(b.integrity);
    hash_lease_node(h, b.leaf);
  }
  memset(out, 0, sizeof *out);
  out->abi_version = 0x47504C4100000002ull;
  out->count = sum.count;
  out->payload_bytes = sum.payload_bytes;
  h.final(out->sha256);
  return GLACIER_HIP_LEASE_OK;
}

int Leased::lifecycle(uint32_t *out) const {
  // lifecycle (:423-430)
  *out = reclaimed     ? GLACIER_HIP_LEASE_RECLAIMED
         : has_pending ? GLACIER_HIP_LEASE_FREED_PENDING_UNCHARGE
         : has_seal    ? GLACIER_HIP_LEASE_TERMINAL_RETAINED
                       : GLACIER_HIP_LEASE_LIVE;
  return GLACIER_HIP_LEASE_OK;
}

int Leased::root(Root *out) const {
  if (!leased_ok()) return GLACIER_HIP_LEASE_INVALID_COORDINATOR;
  if (has_row || lane_active) return GLACIER_HIP_LEASE_INVALID_LEASED_TRANSACTION;
  *out = target.cache->root;
  return GLACIER_HIP_LEASE_OK;
}

int Leased::plan_next_row(glacier_hip_leased_row_plan_t *out) {
  // planNextRow (:453-480)
  if (lane_target()) return GLACIER_HIP_LEASE_INVALID_COORDINATOR;
  if (int rc = validate_mutable()) return rc;
  if (has_row) return GLACIER_HIP_LEASE_INVALID_LEASED_TRANSACTION;
  Summary bs;
  if (int rc = binding_summary(GLACIER_HIP_BINDING_LIVE, &bs)) return rc;
  glacier_hip_row_allocation_plan_t cp;
  if (int rc = target.cache->plan_next_row(&cp)) return rc;
  if (cp.logical_page >= binding_count) return GLACIER_HIP_LEASE_INVALID_BINDING_STORAGE;
  const Binding &b = bindings[cp.logical_page];
  if ((cp.allocation_bytes == 0 && cp.page_payload_present && b.state != GLACIER_HIP_BINDING_LIVE) ||
      (cp.allocation_bytes != 0 && (cp.page_payload_present || b.state != GLACIER_HIP_BINDING_FREE)))
    return GLACIER_HIP_LEASE_INVALID_BINDING;
  memset(out, 0, sizeof *out);
  out->abi_version = kRowPlanAbi;
  out->coordinator_instance = instance;
  out->tree = *tree;
  out->publication_sequence = *sequence;
  out->cache_plan = cp;
  out->bindings = bs;
  out->integrity = plan_integrity(*out);
  return GLACIER_HIP_LEASE_OK;
}

int Leased::begin_row(const glacier_hip_leased_row_plan_t &plan, glacier_hip_leased_row_txn_t *out) {
  // beginRowPlanned (:482-565)
  glacier_hip_leased_row_plan_t expected;
  if (int rc = plan_next_row(&expected)) return rc;
  if (plan.abi_version != kRowPlanAbi || plan.integrity != plan_integrity(plan) ||
      !same(&plan, &expected, sizeof plan))
    return GLACIER_HIP_LEASE_INVALID_LEASED_PLAN;
  if (next_generation == 0 || next_generation == UINT64_MAX) return GLACIER_HIP_LEASE_INVALID_COORDINATOR;
  glacier_hip_kv_pages *host = target.host;
  std::vector<gpk::RowTxn> t;
  bool installed = false;
  const uint64_t page = plan.cache_plan.logical_page;
  if (plan.cache_plan.allocation_bytes != 0) {
    Spec spec{scope, page + 1, page_binding_key(plan.cache_plan.cache_instance, page),
              kv_claim(plan.cache_plan.allocation_bytes)};
    Node leaf;
    Batch b;
    Tree tr;
    if (int rc = bank->reserve_allocations(*tree, request_epoch, session_id,
                                           plan.publication_sequence, &spec, 1, &leaf, &tr, &b))
      return rc;
    *tree = tr;
    if (int rc = host->cache.begin(0, 1, host->pool, t)) {
      // the map took nothing: uncharge before reporting
      if (bank->abort_allocations(b, &tr) == GLACIER_HIP_LEASE_OK) *tree = tr;
      return map_begin_error(rc, true);
    }
    if (bank->commit_allocations(b, &tr) == GLACIER_HIP_LEASE_OK) *tree = tr;
    bindings[page] = live_binding(page, plan.cache_plan.allocation_bytes, leaf);
    installed = true;
  } else if (int rc = host->cache.begin(0, 1, host->pool, t)) {
    return map_begin_error(rc, false);
  }
  host->staged = t;
  // from here the row is active and any new page is charged; nothing fails
  Summary after;
  if (binding_summary(GLACIER_HIP_BINDING_LIVE, &after)) memset(&after, 0, sizeof after);
  memset(&row, 0, sizeof row);
  row.abi_version = kRowTxnAbi;
  row.coordinator_instance = instance;
  row.generation = next_generation++;
  row.mark = t[0].mark;
  row.installed_new_binding = installed;
  memcpy(row.bindings_digest, after.digest, 32);
  row.integrity = txn_integrity(row);
  has_row = true;
  *out = row;
  return GLACIER_HIP_LEASE_OK;
}

int Leased::validate_active(const glacier_hip_leased_row_txn_t &txn) const {
  // validateActiveRow (:1099-1110)
  if (!leased_ok()) return GLACIER_HIP_LEASE_INVALID_COORDINATOR;
  if (!has_row || txn.abi_version != kRowTxnAbi || txn.integrity != txn_integrity(txn) ||
      !same(&txn, &row, sizeof txn))
    return GLACIER_HIP_LEASE_INVALID_LEASED_TRANSACTION;
  return GLACIER_HIP_LEASE_OK;
}

int Leased::commit_row(const glacier_hip_leased_row_txn_t &txn, Root *root_out) {
  // commitRowTxn (:666-676)
  if (int rc = validate_active(txn)) return rc;
  glacier_hip_kv_pages *host = target.host;
  if (host->cache.commit(host->staged.data(), host->staged.size())) return GLACIER_HIP_LEASE_INVALID_TRANSACTION;
  host->staged.clear();
  has_row = false;
  if (root_out) *root_out = host->cache.root;
  return GLACIER_HIP_LEASE_OK;
}

int Leased::abort_row(const glacier_hip_leased_row_txn_t &txn) {
  // abortRowTxn (:678-689): the payload stays with its page and charged
  if (int rc = validate_active(txn)) return rc;
  glacier_hip_kv_pages *host = target.host;
  if (host->cache.abort(host->staged.data(), host->staged.size())) return GLACIER_HIP_LEASE_INVALID_TRANSACTION;
  host->staged.clear();
  has_row = false;
  return GLACIER_HIP_LEASE_OK;
}

int Leased::reserve_rows(uint32_t rows) {
  // beginRowPlanned's reservation for the rows of one session step: every
  // page a row installs without a payload gets its leaf charged first
  if (int rc = validate_mutable()) return rc;
  if (lane_active || has_batch) return GLACIER_HIP_LEASE_INVALID_LEASED_TRANSACTION;
  const gpk::Cache &c = *target.cache;
  std::vector<Spec> specs;
  batch_pages.clear();
  for (uint64_t pos = c.len; pos < c.len + rows && pos < c.max_seq; ++pos) {
    if (pos % gpk::kPagePositions) continue;
    const uint64_t p = pos / gpk::kPagePositions;
    if (p >= binding_count) return GLACIER_HIP_LEASE_INVALID_BINDING_STORAGE;
    const bool present = c.page_of[p] >= 0;
    if (present != (bindings[p].state == GLACIER_HIP_BINDING_LIVE)) return GLACIER_HIP_LEASE_INVALID_BINDING;
    if (present) continue;
    specs.push_back(Spec{scope, p + 1, page_binding_key(c.instance, p), kv_claim(c.page_payload_bytes)});
    batch_pages.push_back(p);
  }
  // rows that take no new page keep the lane's binding set as it is (their
  // pages' bindings were checked above); the full membership check
  // (bindingSummaryForState) runs before any new page is charged, and again
  // at seal and reclaim
  if (!specs.empty()) {
    Summary bs;
    if (int rc = binding_summary(GLACIER_HIP_BINDING_LIVE, &bs)) return rc;
  }
  lane_active = true;
  if (specs.empty()) return GLACIER_HIP_LEASE_OK;
  batch_leaves.resize(specs.size());
  Tree tr;
  if (int rc = bank->reserve_allocations(*tree, request_epoch, session_id, *sequence, specs.data(),
                                         specs.size(), batch_leaves.data(), &tr, &batch)) {
    lane_active = false;
    return rc;
  }
  *tree = tr;
  has_batch = true;
  return GLACIER_HIP_LEASE_OK;
}

void Leased::settle_rows(bool taken) {
  // commitAllocationsAfterAllocate once the map holds the payloads, or
  // abortAllocationsAfterFree when it took none
  if (!taken) lane_active = false;
  if (!has_batch) return;
  has_batch = false;
  Tree tr;
  if (taken) {
    if (bank->commit_allocations(batch, &tr) == GLACIER_HIP_LEASE_OK) *tree = tr;
    for (size_t i = 0; i < batch_pages.size(); ++i)
      bindings[batch_pages[i]] = live_binding(batch_pages[i], target.cache->page_payload_bytes,
                                              batch_leaves[i]);
  } else if (bank->abort_allocations(batch, &tr) == GLACIER_HIP_LEASE_OK) {
    *tree = tr;
  }
}

int Leased::seal_terminal(const Root &expected_root, const uint8_t kv[32], uint64_t seq,
                          uint32_t reason, uint32_t token, glacier_hip_terminal_seal_t *out) {
  // sealTerminalForPublication (:691-757)
  if (int rc = validate_mutable()) return rc;
  if (has_row || lane_active) return GLACIER_HIP_LEASE_INVALID_LEASED_TRANSACTION;
  if (seq == UINT64_MAX || seq != *sequence) return GLACIER_HIP_LEASE_INVALID_TERMINAL_SEAL;
  if (!same(&expected_root, &target.cache->root, sizeof expected_root)) return GLACIER_HIP_LEASE_INVALID_ROOT;
  uint8_t digest[32];
  if (int rc = target.kv_sha256(digest)) return rc;
  if (!same(digest, kv, 32)) return GLACIER_HIP_LEASE_INVALID_TERMINAL_SEAL;
  Summary bs;
  if (int rc = binding_summary(GLACIER_HIP_BINDING_LIVE, &bs)) return rc;
  if (next_generation == 0 || next_generation == UINT64_MAX) return GLACIER_HIP_LEASE_INVALID_COORDINATOR;
  glacier_hip_terminal_seal_t s;
  memset(&s, 0, sizeof s);
  s.abi_version = kTerminalSealAbi;
  s.coordinator_instance = instance;
  s.cache_id = (uint64_t)(uintptr_t)target.cache;
  s.cache_instance = expected_root.cache_instance;
  s.scope_index = scope.node_index;
  s.scope_generation = scope.generation;
  s.tree_identity_generation = tree->identity_generation;
  s.tree_generation = tree->generation;
  s.tree_structural_revision = tree->structural_revision;
  s.tree_state_digest = tree->state_digest;
  s.root = expected_root;
  memcpy(s.logical_kv_sha256, digest, 32);
  s.bindings = bs;
  s.transaction_sequence = seq;
  s.terminal_reason = reason;
  s.terminal_token = token;
  s.generation = next_generation;
  seal_digest(s, s.digest);
  PubPermit permit;
  if (int rc = bank->begin_publication(*tree, request_epoch, session_id, seq, &permit)) return rc;
  if (int rc = bank->commit_publication(permit)) return rc;
  *sequence = seq + 1;
  ++next_generation;
  seal = s;
  has_seal = true;
  *out = s;
  return GLACIER_HIP_LEASE_OK;
}

int Leased::finalize_wave_terminal(uint64_t sequence, uint32_t reason, uint32_t token,
                                   const uint8_t proposal[32], const uint8_t commit[32]) {
  if (int rc = validate_mutable()) return rc;
  if (has_row || lane_active) return GLACIER_HIP_LEASE_INVALID_LEASED_TRANSACTION;
  if (*this->sequence != sequence + 1) return GLACIER_HIP_LEASE_INVALID_TERMINAL_SEAL;
  uint8_t digest[32];
  if (int rc = target.kv_sha256(digest)) return rc;
  Summary bs;
  if (int rc = binding_summary(GLACIER_HIP_BINDING_LIVE, &bs)) return rc;
  glacier_hip_terminal_seal_t s;
  memset(&s, 0, sizeof s);
  s.abi_version = kTerminalSealAbi;
  s.coordinator_instance = instance;
  s.cache_id = (uint64_t)(uintptr_t)target.cache;
  s.cache_instance = target.cache->root.cache_instance;
  s.scope_index = scope.node_index;
  s.scope_generation = scope.generation;
  s.tree_identity_generation = tree->identity_generation;
  s.tree_generation = tree->generation;
  s.tree_structural_revision = tree->structural_revision;
  s.tree_state_digest = tree->state_digest;
  s.root = target.cache->root;
  memcpy(s.logical_kv_sha256, digest, 32);
  s.bindings = bs;
  s.transaction_sequence = sequence;
  s.terminal_reason = reason;
  s.terminal_token = token;
  s.generation = next_generation++;
  memcpy(seal_proposal, proposal, 32);
  memcpy(seal_commit, commit, 32);
  seal_digest_v3(s, proposal, commit, s.digest);
  seal = s;
  seal_v3 = true;
  has_seal = true;
  return GLACIER_HIP_LEASE_OK;
}

int Leased::terminal_seal(glacier_hip_terminal_seal_t *out, uint8_t proposal[32],
                          uint8_t commit[32]) const {
  if (!leased_ok()) return GLACIER_HIP_LEASE_INVALID_COORDINATOR;
  if (!has_seal) return GLACIER_HIP_LEASE_TERMINAL_REQUIRED;
  *out = seal;
  if (proposal) memcpy(proposal, seal_proposal, 32);
  if (commit) memcpy(commit, seal_commit, 32);
  return GLACIER_HIP_LEASE_OK;
}

int Leased::begin_reclaim(const glacier_hip_terminal_seal_t &sl, uint64_t expected_sequence,
                          glacier_hip_freed_payload_t *out) {
  // beginTerminalReclaim (:852-867) after validateTerminalSeal (:1112-1127)
  if (!leased_ok()) return GLACIER_HIP_LEASE_INVALID_COORDINATOR;
  if (!has_seal) return GLACIER_HIP_LEASE_TERMINAL_REQUIRED;
  uint8_t d[32];
  if (seal_v3) seal_digest_v3(sl, seal_proposal, seal_commit, d);
  else seal_digest(sl, d);
  if (sl.abi_version != kTerminalSealAbi || !same(d, sl.digest, 32) || !same(&sl, &seal, sizeof sl) ||
      sl.coordinator_instance != instance || sl.cache_id != (uint64_t)(uintptr_t)target.cache ||
      sl.scope_index != scope.node_index || sl.scope_generation != scope.generation)
    return GLACIER_HIP_LEASE_INVALID_TERMINAL_SEAL;
  return begin_reclaim_exact(sl.digest, sl.root, sl.logical_kv_sha256, sl.bindings,
                             &sl.transaction_sequence, expected_sequence, out);
}

int Leased::begin_reclaim_exact(const uint8_t seal_dig[32], const Root &expected_root,
                                const uint8_t kv[32], const Summary &expected_bindings,
                                const uint64_t *terminal_sequence, uint64_t expected_sequence,
                                glacier_hip_freed_payload_t *out) {
  // beginReclaimExact (:918-1036)
  if (has_pending) return GLACIER_HIP_LEASE_RECLAIM_PENDING;
  if (reclaimed) return GLACIER_HIP_LEASE_RECLAIM_COMPLETE;
  if (next_generation == 0 || next_generation == UINT64_MAX) return GLACIER_HIP_LEASE_INVALID_COORDINATOR;
  if (expected_sequence != *sequence || (terminal_sequence && expected_sequence <= *terminal_sequence))
    return GLACIER_HIP_LEASE_INVALID_TERMINAL_SEAL;
  gpk::Cache &c = *target.cache;
  const Root root_before = c.root;
  if (c.retired) return GLACIER_HIP_LEASE_CACHE_RETIRED;
  if (!same(&expected_root, &c.root, sizeof expected_root)) return GLACIER_HIP_LEASE_INVALID_ROOT;
  uint8_t digest[32];
  if (int rc = target.kv_sha256(digest)) return rc;
  if (!same(digest, kv, 32)) return GLACIER_HIP_LEASE_INVALID_TERMINAL_SEAL;
  Summary bs;
  if (int rc = binding_summary(GLACIER_HIP_BINDING_LIVE, &bs)) return rc;
  if (!same(&bs, &expected_bindings, sizeof bs)) return GLACIER_HIP_LEASE_INVALID_BINDING;
  gpk::RetirePlan plan;
  if (int rc = c.plan_retirement(&plan)) return rc;
  if (!same(&plan.root, &expected_root, sizeof expected_root) || plan.allocated_pages != bs.count ||
      plan.payload_bytes_to_free != bs.payload_bytes)
    return GLACIER_HIP_LEASE_INVALID_BINDING;
  Tree tr;
  Ticket ticket;
  if (int rc = bank->begin_retire(*tree, scope, request_epoch, session_id, expected_sequence, &tr,
                                  &ticket))
    return rc;
  *tree = tr;
  Summary quiesced;
  int rc = binding_summary(GLACIER_HIP_BINDING_LIVE, &quiesced);
  if (rc || !same(&quiesced, &bs, sizeof bs) || ticket.node_count != bs.count ||
      !claim_is_exact_kv(ticket.claim, bs.payload_bytes)) {
    if (bank->cancel_retire(ticket, &tr) == GLACIER_HIP_LEASE_OK) *tree = tr;
    return rc ? rc : GLACIER_HIP_LEASE_INVALID_BINDING;
  }
  FreePermit permit;
  if (int r2 = bank->authorize_free(ticket, &tr, &permit)) return r2;
  *tree = tr;
  uint64_t freed_bytes = 0;
  c.reclaim_retired(plan, *target.pool, &freed_bytes);  // prevalidated: cannot fail
  for (uint32_t i = 0; i < binding_count; ++i) {
    Binding &b = bindings[i];
    if (b.state != GLACIER_HIP_BINDING_LIVE) continue;
    b.state = GLACIER_HIP_BINDING_FREED_PENDING_UNCHARGE;
    b.integrity = page_binding_integrity(b);
  }
  Summary pend;
  binding_summary(GLACIER_HIP_BINDING_FREED_PENDING_UNCHARGE, &pend);
  glacier_hip_freed_payload_t f;
  memset(&f, 0, sizeof f);
  f.abi_version = kFreedPayloadAbi;
  f.coordinator_instance = instance;
  f.generation = next_generation;
  memcpy(f.terminal_seal_digest, seal_dig, 32);
  f.permit_generation = permit.generation;
  f.root_before = root_before;
  f.root_after = c.root;
  f.binding_count = bs.count;
  f.payload_bytes = bs.payload_bytes;
  memcpy(f.bindings_digest, pend.digest, 32);
  f.integrity = freed_integrity(f);
  ++next_generation;
  pending_freed = f;
  pending_permit = permit;
  has_pending = true;
  *out = f;
  return GLACIER_HIP_LEASE_OK;
}

int Leased::commit_reclaim(const glacier_hip_freed_payload_t &freed, glacier_hip_reclaim_receipt_t *out) {
  // commitReclaimAfterFree (:1040-1080)
  if (!leased_ok()) return GLACIER_HIP_LEASE_INVALID_COORDINATOR;
  if (!has_pending) return reclaimed ? GLACIER_HIP_LEASE_RECLAIM_COMPLETE : GLACIER_HIP_LEASE_INVALID_FREED_PAYLOAD;
  if (freed.abi_version != kFreedPayloadAbi || freed.integrity != freed_integrity(freed) ||
      !same(&freed, &pending_freed, sizeof freed))
    return GLACIER_HIP_LEASE_INVALID_FREED_PAYLOAD;
  Summary s;
  if (int rc = binding_summary(GLACIER_HIP_BINDING_FREED_PENDING_UNCHARGE, &s)) return rc;
  if (s.count != freed.binding_count || s.payload_bytes != freed.payload_bytes ||
      !same(s.digest, freed.bindings_digest, 32))
    return GLACIER_HIP_LEASE_INVALID_BINDING;
  Tree after;
  if (int rc = bank->commit_free(pending_permit, &after)) return rc;
  *tree = after;
  const Binding fb = free_binding();
  for (uint32_t i = 0; i < binding_count; ++i) bindings[i] = fb;
  has_pending = false;
  reclaimed = true;
  if (out) {
    memset(out, 0, sizeof *out);
    out->abi_version = kReclaimReceiptAbi;
    out->coordinator_instance = instance;
    out->generation = freed.generation;
    out->freed = freed;
    out->tree_after = after;
    uint64_t h = mix64(kReclaimReceiptAbi ^ instance);
    h = mix64(h ^ freed.generation ^ freed.integrity);
    h = mix_tree(h, after);
    out->integrity = h ? h : 1;
  }
  return GLACIER_HIP_LEASE_OK;
}

int Leased::reclaim_for_teardown(uint64_t expected_sequence) {
  // reclaimForTeardown (:894-916)
  if (!leased_ok()) return GLACIER_HIP_LEASE_INVALID_COORDINATOR;
  if (reclaimed) return GLACIER_HIP_LEASE_OK;
  if (has_pending) return commit_reclaim(pending_freed, nullptr);
  if (has_row)
    if (int rc = abort_row(row)) return rc;
  if (lane_active) return GLACIER_HIP_LEASE_INVALID_LEASED_TRANSACTION;  // a session step is running
  if (expected_sequence != *sequence) return GLACIER_HIP_LEASE_INVALID_TERMINAL_SEAL;
  gpk::Cache &c = *target.cache;
  const Root r = c.root;
  uint8_t digest[32];
  if (int rc = target.kv_sha256(digest)) return rc;
  Summary bs;
  if (int rc = binding_summary(GLACIER_HIP_BINDING_LIVE, &bs)) return rc;
  if (bs.count == 0) {
    gpk::RetirePlan plan;
    if (int rc = c.plan_retirement(&plan)) return rc;
    if (!same(&plan.root, &r, sizeof r) || plan.allocated_pages != 0 || plan.payload_bytes_to_free != 0)
      return GLACIER_HIP_LEASE_INVALID_BINDING;
    uint64_t freed = 0;
    if (int rc = c.reclaim_retired(plan, *target.pool, &freed)) return rc;
    const Binding fb = free_binding();
    for (uint32_t i = 0; i < binding_count; ++i) bindings[i] = fb;
    reclaimed = true;
    return GLACIER_HIP_LEASE_OK;
  }
  uint8_t sd[32];
  teardown_digest(instance, expected_sequence, r, digest, bs, sd);
  glacier_hip_freed_payload_t freed;
  if (int rc = begin_reclaim_exact(sd, r, digest, bs, nullptr, expected_sequence, &freed)) return rc;
  return commit_reclaim(freed, nullptr);
}

}  // namespace glb

// ---------------------------------------------------------------------------
// C ABI (host page maps; session lanes in session.hip)
// ---------------------------------------------------------------------------
extern "C" {

int glacier_hip_leased_kv_create(glacier_hip_lease_bank *b, glacier_hip_lease_tree_t *tree,
                                 const glacier_hip_lease_node_t *scope, glacier_hip_kv_pages *pages,
                                 glacier_hip_page_lease_binding_t *bindings, uint32_t binding_count,
                                 uint64_t request_epoch, uint64_t session_id, uint64_t *sequence,
                                 glacier_hip_leased_kv **out) {
  if (!b || !tree || !scope || !pages || !bindings || !sequence || !out)
    return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  auto *c = new (std::nothrow) glacier_hip_leased_kv();
  if (!c) return GLACIER_HIP_LEASE_INVALID_CONFIGURATION;
  glb::Target t;
  t.cache = &pages->cache;
  t.pool = &pages->pool;
  t.host = pages;
  t.kv_sha256 = [pages](uint8_t o[32]) { return gpk::host_kv_sha256(pages, o); };
  if (pages->staged.size()) {
    delete c;
    return GLACIER_HIP_LEASE_INVALID_COORDINATOR;
  }
  const int rc = c->lease.init(&b->bank, tree, *scope, t, bindings, binding_count, request_epoch,
                               session_id, sequence);
  if (rc) {
    delete c;
    return rc;
  }
  *out = c;
  return GLACIER_HIP_LEASE_OK;
}

void glacier_hip_leased_kv_destroy(glacier_hip_leased_kv *c) {
  if (!c) return;
  if (c->detach) c->detach(c);
  delete c;
}

int glacier_hip_leased_kv_plan_next_row(glacier_hip_leased_kv *c, glacier_hip_leased_row_plan_t *out) {
  if (!c || !out) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return c->lease.plan_next_row(out);
}

int glacier_hip_leased_kv_begin_row(glacier_hip_leased_kv *c, const glacier_hip_leased_row_plan_t *plan,
                                    glacier_hip_leased_row_txn_t *out) {
  if (!c || !plan || !out) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return c->lease.begin_row(*plan, out);
}

int glacier_hip_leased_kv_commit_row(glacier_hip_leased_kv *c, const glacier_hip_leased_row_txn_t *txn,
                                     glacier_hip_page_map_root_t *root_out) {
  if (!c || !txn) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return c->lease.commit_row(*txn, root_out);
}

int glacier_hip_leased_kv_abort_row(glacier_hip_leased_kv *c, const glacier_hip_leased_row_txn_t *txn) {
  if (!c || !txn) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return c->lease.abort_row(*txn);
}

int glacier_hip_leased_kv_binding_summary(glacier_hip_leased_kv *c, glacier_hip_binding_summary_t *out) {
  if (!c || !out) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return c->lease.binding_summary(GLACIER_HIP_BINDING_LIVE, out);
}

int glacier_hip_leased_kv_allocation_set(glacier_hip_leased_kv *c,
                                         glacier_hip_allocation_set_v2_t *out) {
  if (!c || !out) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return c->lease.allocation_set(GLACIER_HIP_BINDING_LIVE, out);
}

int glacier_hip_leased_kv_lifecycle(glacier_hip_leased_kv *c, uint32_t *out) {
  if (!c || !out) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return c->lease.lifecycle(out);
}

int glacier_hip_leased_kv_root(glacier_hip_leased_kv *c, glacier_hip_page_map_root_t *out) {
  if (!c || !out) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return c->lease.root(out);
}

int glacier_hip_leased_kv_kv_sha256(glacier_hip_leased_kv *c, uint8_t out[32]) {
  if (!c || !out) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  if (!c->lease.leased_ok()) return GLACIER_HIP_LEASE_INVALID_COORDINATOR;
  return c->lease.kv_sha256(out);
}

int glacier_hip_leased_kv_seal_terminal(glacier_hip_leased_kv *c, const glacier_hip_page_map_root_t *root,
                                        const uint8_t kv[32], uint64_t transaction_sequence,
                                        uint32_t reason, uint32_t terminal_token,
                                        glacier_hip_terminal_seal_t *out) {
  if (!c || !root || !kv || !out || reason > GLACIER_HIP_TERMINAL_CANCELLED)
    return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return c->lease.seal_terminal(*root, kv, transaction_sequence, reason, terminal_token, out);
}

int glacier_hip_leased_kv_begin_reclaim(glacier_hip_leased_kv *c, const glacier_hip_terminal_seal_t *seal,
                                        uint64_t expected_sequence, glacier_hip_freed_payload_t *out) {
  if (!c || !seal || !out) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return c->lease.begin_reclaim(*seal, expected_sequence, out);
}

int glacier_hip_leased_kv_commit_reclaim(glacier_hip_leased_kv *c, const glacier_hip_freed_payload_t *freed,
                                         glacier_hip_reclaim_receipt_t *out) {
  if (!c || !freed) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return c->lease.commit_reclaim(*freed, out);
}

int glacier_hip_leased_kv_terminal_seal(glacier_hip_leased_kv *c, glacier_hip_terminal_seal_t *out,
                                        uint8_t proposal_sha256[32], uint8_t commit_sha256[32]) {
  if (!c || !out) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return c->lease.terminal_seal(out, proposal_sha256, commit_sha256);
}

int glacier_hip_leased_kv_reclaim_for_teardown(glacier_hip_leased_kv *c, uint64_t expected_sequence) {
  if (!c) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return c->lease.reclaim_for_teardown(expected_sequence);
}

int glacier_hip_kv_pages_set_pool_capacity(glacier_hip_kv_pages *p, uint32_t pages) {
  // the payload pool stands for an allocator with a limit: at most `pages`
  // payloads held by the map and free together
  if (!p) return GLACIER_HIP_INVALID_ARGUMENT;
  const uint64_t held = p->cache.allocated_pages();
  const uint64_t total = p->rows.size() / (p->cache.layers * 2 * gpk::kPagePositions * p->cache.dim);
  if (pages < held || pages > total) return GLACIER_HIP_SHAPE_MISMATCH;
  std::vector<bool> used(total, false);
  for (int32_t q : p->cache.page_of)
    if (q >= 0) used[q] = true;
  p->pool.free.clear();
  for (uint64_t q = total; q-- > 0 && held + p->pool.free.size() < pages;)
    if (!used[q]) p->pool.free.push_back((int32_t)q);
  return GLACIER_HIP_OK;
}

}  // extern "C"
