// lease_bank.cpp — ResourceBank receipts, LeaseTree and publication sessions
// for leased paged KV (core/resource_bank.zig; line references per function).
#include "lease_bank.h"

#include <string.h>

#include <new>

namespace glb {

namespace {
constexpr uint64_t kReservationDomain = 0x7265736572766174ull;
constexpr uint64_t kReceiptDomain = 0x7265636569707430ull;
constexpr uint64_t kTreeDomain = 0x6c74726565763031ull;
constexpr uint64_t kNodeDomain = 0x6c6e6f6465763031ull;
constexpr uint64_t kBatchDomain = 0x6c62617463683031ull;
constexpr uint64_t kTicketDomain = 0x6c7469636b657431ull;
constexpr uint64_t kPermitDomain = 0x6c7065726d697431ull;
constexpr uint64_t kPubDomain = 0x7075626c69636131ull;
constexpr uint64_t kStateDomain = 0x6c73746174653031ull;

const uint64_t *fields(const Claim &c) { return &c.capsule_bytes; }
uint64_t *fields(Claim &c) { return &c.capsule_bytes; }
constexpr int kClassCount = 10;

bool host_bytes(const Claim &c, uint64_t *out) {
  // Claim.hostBytes (:73-88): every class but device_bytes, io_bytes, queue_slots
  uint64_t t = 0;
  const uint64_t *f = fields(c);
  for (int i = 0; i < 7; ++i) {
    if (f[i] > UINT64_MAX - t) return false;
    t += f[i];
  }
  *out = t;
  return true;
}

Claim max_claims(const Claim &a, const Claim &b) {
  Claim o;
  for (int i = 0; i < kClassCount; ++i) fields(o)[i] = fields(a)[i] > fields(b)[i] ? fields(a)[i] : fields(b)[i];
  return o;
}

uint64_t mix_receipt(uint64_t h, const Receipt &r) {
  h = mix64(h ^ r.bank_epoch);
  h = mix64(h ^ r.slot_index);
  h = mix64(h ^ r.generation);
  h = mix64(h ^ r.owner_key);
  h = mix_claim(h, r.claim);
  return mix64(h ^ r.integrity);
}

bool receipt_eq(const Receipt &a, const Receipt &b) { return memcmp(&a, &b, sizeof a) == 0; }

void clear_pending(RootSlot &root) {
  // clearLeasePending (:4177-4198)
  root.pending = Pending::None;
  root.pending_generation = root.pending_completion = 0;
  root.pending_free_permit = root.pending_free_completion = 0;
  root.pending_scope = kNoNode;
  root.pending_count = 0;
  root.pending_claim = Claim{};
  root.pending_digest = 0;
}
}  // namespace

uint64_t mix64(uint64_t v) {
  v ^= v >> 30;
  v *= 0xbf58476d1ce4e5b9ull;
  v ^= v >> 27;
  v *= 0x94d049bb133111ebull;
  v ^= v >> 31;
  return v;
}

bool claim_zero(const Claim &c) {
  for (int i = 0; i < kClassCount; ++i)
    if (fields(c)[i]) return false;
  return true;
}
bool claim_eq(const Claim &a, const Claim &b) { return memcmp(&a, &b, sizeof a) == 0; }
bool claim_within(const Claim &v, const Claim &ceiling) {
  for (int i = 0; i < kClassCount; ++i)
    if (fields(v)[i] > fields(ceiling)[i]) return false;
  return true;
}
bool add_claims(const Claim &a, const Claim &b, Claim *out) {
  Claim o;
  for (int i = 0; i < kClassCount; ++i) {
    if (fields(a)[i] > UINT64_MAX - fields(b)[i]) return false;
    fields(o)[i] = fields(a)[i] + fields(b)[i];
  }
  *out = o;
  return true;
}
bool sub_claims(const Claim &a, const Claim &b, Claim *out) {
  Claim o;
  for (int i = 0; i < kClassCount; ++i) {
    if (fields(a)[i] < fields(b)[i]) return false;
    fields(o)[i] = fields(a)[i] - fields(b)[i];
  }
  *out = o;
  return true;
}
uint64_t mix_claim(uint64_t h, const Claim &c) {
  for (int i = 0; i < kClassCount; ++i) h = mix64(h ^ fields(c)[i] ^ ((uint64_t)i << 56));
  return h;
}

Bank::Bank(uint32_t slot_count, uint32_t node_count, const Limits &l, uint64_t e)
    : epoch(e), limits(l), slots(slot_count), roots(slot_count), nodes(node_count) {}

bool Bank::fits(const Claim &c) const {
  // Limits.fitsWithHost (:117-131)
  uint64_t hb;
  if (!host_bytes(c, &hb) || hb > limits.host_bytes) return false;
  const uint64_t *lf = &limits.capsule_bytes;
  for (int i = 0; i < kClassCount; ++i)
    if (fields(c)[i] > lf[i]) return false;
  return true;
}

uint64_t Bank::token_integrity(uint64_t ep, uint64_t slot, uint64_t gen, uint64_t owner,
                               const Claim &claim, uint64_t domain) {
  uint64_t h = mix64(domain ^ ep);
  h = mix64(h ^ slot);
  h = mix64(h ^ gen);
  h = mix64(h ^ owner);
  h = mix_claim(h, claim);
  return h ? h : 1;
}

int Bank::validate_receipt(const Receipt &r, Slot **out) {
  // validateReceipt (:4084-4108)
  if (r.bank_epoch != epoch || r.slot_index >= slots.size()) return GLACIER_HIP_LEASE_STALE_RESERVATION;
  Slot &s = slots[r.slot_index];
  if (s.state == SlotState::Free || s.generation != r.generation || s.owner_key != r.owner_key ||
      !claim_eq(s.claim, r.claim) || s.integrity != r.integrity ||
      r.integrity != token_integrity(epoch, r.slot_index, r.generation, r.owner_key, r.claim,
                                     s.state == SlotState::Committed ? kReceiptDomain
                                                                     : kReservationDomain))
    return GLACIER_HIP_LEASE_STALE_RESERVATION;
  *out = &s;
  return GLACIER_HIP_LEASE_OK;
}

int Bank::reserve(uint64_t owner_key, const Claim &claim, Receipt *out) {
  // reserve (:976-1044)
  if (owner_key == 0 || claim_zero(claim)) return GLACIER_HIP_LEASE_INVALID_CLAIM;
  std::lock_guard<std::mutex> g(mu);
  Claim next;
  uint64_t hb;
  if (!add_claims(used, claim, &next) || !host_bytes(next, &hb)) {
    ++counters.rejected_capacity;
    return GLACIER_HIP_LEASE_CLAIM_OVERFLOW;
  }
  if (!fits(next)) {
    ++counters.rejected_capacity;
    return GLACIER_HIP_LEASE_CAPACITY_EXCEEDED;
  }
  size_t index = slots.size();
  for (size_t i = 0; i < slots.size(); ++i)
    if (slots[i].state == SlotState::Free) {
      index = i;
      break;
    }
  if (index == slots.size()) {
    ++counters.rejected_slots;
    return GLACIER_HIP_LEASE_SLOTS_EXHAUSTED;
  }
  if (next_generation == 0 || next_generation == UINT64_MAX) return GLACIER_HIP_LEASE_INVALID_CONFIGURATION;
  const uint64_t gen = next_generation++;
  Slot s;
  s.state = SlotState::Reserved;
  s.generation = gen;
  s.owner_key = owner_key;
  s.claim = claim;
  s.integrity = token_integrity(epoch, index, gen, owner_key, claim, kReservationDomain);
  slots[index] = s;
  used = next;
  peak = max_claims(peak, next);
  if (hb > peak_host_bytes) peak_host_bytes = hb;
  ++counters.successful_reservations;
  *out = Receipt{epoch, index, gen, owner_key, claim, s.integrity};
  return GLACIER_HIP_LEASE_OK;
}

int Bank::commit(const Receipt &res, Receipt *out) {
  // commit (:1046-1076)
  std::lock_guard<std::mutex> g(mu);
  Slot *s;
  if (int rc = validate_receipt(res, &s)) return rc;
  if (s->state != SlotState::Reserved) return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  s->state = SlotState::Committed;
  s->integrity = token_integrity(epoch, res.slot_index, res.generation, res.owner_key, res.claim,
                                 kReceiptDomain);
  ++counters.successful_commits;
  *out = res;
  out->integrity = s->integrity;
  return GLACIER_HIP_LEASE_OK;
}

int Bank::cancel(const Receipt &res) {
  // cancel (:1078-1095)
  std::lock_guard<std::mutex> g(mu);
  Slot *s;
  if (int rc = validate_receipt(res, &s)) return rc;
  if (s->state != SlotState::Reserved) return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  Claim next;
  if (!sub_claims(used, res.claim, &next)) return GLACIER_HIP_LEASE_CLAIM_OVERFLOW;
  used = next;
  *s = Slot{};
  ++counters.cancellations;
  return GLACIER_HIP_LEASE_OK;
}

int Bank::release(const Receipt &r) {
  // release (:3166-3184)
  std::lock_guard<std::mutex> g(mu);
  Slot *s;
  if (int rc = validate_receipt(r, &s)) return rc;
  if (s->state != SlotState::Committed || s->pub_session != 0 || s->pub_active ||
      roots[r.slot_index].active)
    return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  Claim next;
  if (!sub_claims(used, r.claim, &next)) return GLACIER_HIP_LEASE_CLAIM_OVERFLOW;
  used = next;
  *s = Slot{};
  ++counters.releases;
  return GLACIER_HIP_LEASE_OK;
}

int Bank::reserve_generations(uint64_t count, uint64_t *first) {
  // reserveLeaseGenerations (:3625-3638)
  if (count == 0 || next_lease_generation == 0 || next_lease_generation == UINT64_MAX ||
      count >= UINT64_MAX - next_lease_generation)
    return GLACIER_HIP_LEASE_INVALID_CONFIGURATION;
  *first = next_lease_generation;
  next_lease_generation += count;
  return GLACIER_HIP_LEASE_OK;
}

uint64_t Bank::state_digest(uint32_t slot, const RootSlot &root) const {
  // leaseTreeStateDigest: the tree's pending decision and every node of it
  uint64_t h = mix64(kStateDomain ^ slot);
  h = mix64(h ^ root.identity_generation);
  h = mix64(h ^ (uint64_t)root.pending);
  h = mix64(h ^ root.pending_generation);
  h = mix64(h ^ root.pending_completion);
  h = mix64(h ^ root.pending_free_permit);
  h = mix64(h ^ root.pending_free_completion);
  h = mix64(h ^ root.pending_scope);
  h = mix64(h ^ root.pending_count);
  h = mix_claim(h, root.pending_claim);
  h = mix64(h ^ root.pending_digest);
  for (size_t i = 0; i < nodes.size(); ++i) {
    const NodeSlot &n = nodes[i];
    if (!n.active || n.receipt_slot != slot || n.tree_identity_generation != root.identity_generation)
      continue;
    h = mix64(h ^ i);
    h = mix64(h ^ n.generation);
    h = mix64(h ^ (uint64_t)n.state);
    h = mix64(h ^ n.pending_generation);
    h = mix_claim(h, n.subtree);
    h = mix64(h ^ n.integrity);
  }
  return h;
}

uint64_t Bank::tree_integrity(const Receipt &r, const RootSlot &root) {
  uint64_t h = mix_receipt(kTreeDomain, r);
  h = mix64(h ^ root.tree_key);
  h = mix64(h ^ root.authority_key);
  h = mix64(h ^ root.identity_generation);
  h = mix64(h ^ root.generation);
  h = mix64(h ^ root.structural_revision);
  h = mix_claim(h, root.ceiling);
  h = mix_claim(h, root.current);
  h = mix64(h ^ root.active_nodes);
  h = mix64(h ^ root.state_digest);
  return h ? h : 1;
}

uint64_t Bank::node_integrity(const Receipt &r, uint64_t tree_key, uint32_t index,
                              const NodeSlot &n) {
  // the stable identity of a node: never its state, pending decision or
  // subtree sum, so a leaf token stays valid from reservation to free
  uint64_t h = mix_receipt(kNodeDomain, r);
  h = mix64(h ^ tree_key);
  h = mix64(h ^ index);
  h = mix64(h ^ n.tree_identity_generation);
  h = mix64(h ^ n.generation);
  h = mix64(h ^ n.parent_index);
  h = mix64(h ^ n.parent_generation);
  h = mix64(h ^ n.node_key);
  h = mix64(h ^ n.tenant_key);
  h = mix64(h ^ n.binding_key);
  h = mix64(h ^ n.kind);
  h = mix_claim(h, n.ceiling);
  h = mix_claim(h, n.claim);
  return h ? h : 1;
}

void Bank::refresh(const Receipt &r, RootSlot &root) {
  // refreshLeaseTreeRootLocked (:3723-3737)
  root.state_digest = state_digest((uint32_t)r.slot_index, root);
  root.integrity = tree_integrity(r, root);
}

Tree Bank::make_tree(const Receipt &r, const RootSlot &root) const {
  // makeLeaseTree (:4200-4214)
  Tree t{};
  t.abi_version = kTreeAbi;
  t.parent = r;
  t.tree_key = root.tree_key;
  t.authority_key = root.authority_key;
  t.identity_generation = root.identity_generation;
  t.generation = root.generation;
  t.structural_revision = root.structural_revision;
  t.ceiling = root.ceiling;
  t.current = root.current;
  t.active_nodes = root.active_nodes;
  t.state_digest = root.state_digest;
  t.integrity = root.integrity;
  return t;
}

Node Bank::make_node(const Receipt &r, uint64_t tree_key, uint32_t index, const NodeSlot &n) const {
  // makeLeaseNode (:4216-4236)
  Node o{};
  o.abi_version = kNodeAbi;
  o.parent = r;
  o.tree_key = tree_key;
  o.tree_identity_generation = n.tree_identity_generation;
  o.node_index = index;
  o.generation = n.generation;
  o.parent_index = n.parent_index;
  o.parent_generation = n.parent_generation;
  o.node_key = n.node_key;
  o.tenant_key = n.tenant_key;
  o.binding_key = n.binding_key;
  o.kind = n.kind;
  o.ceiling = n.ceiling;
  o.claim = n.claim;
  o.integrity = n.integrity;
  return o;
}

int Bank::validate_tree_locked(const Tree &t, RootSlot **out) {
  // validateLeaseTreeLocked (:3739-3776) with validateLeaseTreeAccounting
  if (t.abi_version != kTreeAbi) return GLACIER_HIP_LEASE_STALE_RESERVATION;
  Slot *s;
  if (int rc = validate_receipt(t.parent, &s)) return rc;
  if (s->state != SlotState::Committed) return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  RootSlot &root = roots[t.parent.slot_index];
  const uint32_t slot = (uint32_t)t.parent.slot_index;
  if (!root.active || root.tree_key != t.tree_key || root.authority_key != t.authority_key ||
      root.identity_generation != t.identity_generation || root.generation != t.generation ||
      root.structural_revision != t.structural_revision || !claim_eq(root.ceiling, t.ceiling) ||
      !claim_eq(root.current, t.current) || root.active_nodes != t.active_nodes ||
      root.state_digest != t.state_digest || root.integrity != t.integrity ||
      root.state_digest != state_digest(slot, root) ||
      root.integrity != tree_integrity(t.parent, root))
    return GLACIER_HIP_LEASE_STALE_RESERVATION;
  Claim sum{};
  uint32_t count = 0;
  for (const NodeSlot &n : nodes) {
    if (!n.active || n.receipt_slot != slot || n.tree_identity_generation != root.identity_generation)
      continue;
    ++count;
    if (n.kind == GLACIER_HIP_LEASE_NODE_ALLOCATION && !add_claims(sum, n.claim, &sum))
      return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  }
  if (count != root.active_nodes || !claim_eq(sum, root.current) ||
      !claim_within(root.current, root.ceiling))
    return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  *out = &root;
  return GLACIER_HIP_LEASE_OK;
}

int Bank::validate_node_locked(const Tree &t, const Node &n, NodeSlot **out) {
  // validateLeaseNodeLocked (:3778-3814)
  RootSlot *root;
  if (int rc = validate_tree_locked(t, &root)) return rc;
  if (n.abi_version != kNodeAbi || !receipt_eq(n.parent, t.parent) || n.tree_key != t.tree_key ||
      n.tree_identity_generation != t.identity_generation || n.node_index >= nodes.size())
    return GLACIER_HIP_LEASE_STALE_RESERVATION;
  NodeSlot &s = nodes[n.node_index];
  if (!s.active || s.receipt_slot != t.parent.slot_index ||
      s.tree_identity_generation != t.identity_generation || s.generation != n.generation ||
      s.parent_index != n.parent_index || s.parent_generation != n.parent_generation ||
      s.node_key != n.node_key || s.tenant_key != n.tenant_key || s.binding_key != n.binding_key ||
      s.kind != n.kind || !claim_eq(s.ceiling, n.ceiling) || !claim_eq(s.claim, n.claim) ||
      s.integrity != n.integrity ||
      n.integrity != node_integrity(t.parent, t.tree_key, n.node_index, s))
    return GLACIER_HIP_LEASE_STALE_RESERVATION;
  *out = &s;
  return GLACIER_HIP_LEASE_OK;
}

int Bank::open_tree(const Receipt &r, uint64_t tree_key, uint64_t authority_key,
                    const Claim &ceiling, Tree *out) {
  // openLeaseTreeWithFundingMode (:1404-1446), additive funding
  if (tree_key == 0 || authority_key == 0 || claim_zero(ceiling)) return GLACIER_HIP_LEASE_INVALID_CLAIM;
  std::lock_guard<std::mutex> g(mu);
  Slot *s;
  if (int rc = validate_receipt(r, &s)) return rc;
  RootSlot &root = roots[r.slot_index];
  if (s->state != SlotState::Committed || root.active || s->pub_epoch != 0 || s->pub_session != 0 ||
      s->pub_active)
    return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  uint64_t gen;
  if (int rc = reserve_generations(2, &gen)) return rc;
  root = RootSlot{};
  root.active = true;
  root.tree_key = tree_key;
  root.authority_key = authority_key;
  root.identity_generation = gen;
  root.generation = gen + 1;
  root.structural_revision = 1;
  root.ceiling = ceiling;
  refresh(r, root);
  ++counters.lease_tree_opens;
  *out = make_tree(r, root);
  return GLACIER_HIP_LEASE_OK;
}

int Bank::open_scope(const Tree &t, uint64_t scope_key, uint64_t tenant_key, const Claim &ceiling,
                     Tree *tree_out, Node *scope_out) {
  // openLeaseScope (:1448-1514)
  if (scope_key == 0 || tenant_key == 0 || claim_zero(ceiling)) return GLACIER_HIP_LEASE_INVALID_CLAIM;
  std::lock_guard<std::mutex> g(mu);
  RootSlot *root;
  if (int rc = validate_tree_locked(t, &root)) return rc;
  Slot &ps = slots[t.parent.slot_index];
  if (root->pending != Pending::None || ps.pub_active || ps.pub_epoch != 0 || ps.pub_session != 0 ||
      !claim_within(ceiling, root->ceiling))
    return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  size_t free_index = nodes.size();
  for (size_t i = 0; i < nodes.size(); ++i) {
    const NodeSlot &n = nodes[i];
    if (n.active && n.receipt_slot == t.parent.slot_index &&
        n.tree_identity_generation == t.identity_generation &&
        n.kind == GLACIER_HIP_LEASE_NODE_SCOPE && n.node_key == scope_key)
      return GLACIER_HIP_LEASE_INVALID_TRANSITION;
    if (!n.active && free_index == nodes.size()) free_index = i;
  }
  if (free_index == nodes.size()) {
    ++counters.rejected_lease_nodes;
    return GLACIER_HIP_LEASE_NODES_EXHAUSTED;
  }
  uint64_t gen;
  if (int rc = reserve_generations(2, &gen)) return rc;
  NodeSlot n;
  n.active = true;
  n.receipt_slot = (uint32_t)t.parent.slot_index;
  n.tree_identity_generation = t.identity_generation;
  n.generation = gen;
  n.parent_index = kNoNode;
  n.parent_generation = t.identity_generation;
  n.node_key = scope_key;
  n.tenant_key = tenant_key;
  n.kind = GLACIER_HIP_LEASE_NODE_SCOPE;
  n.state = NState::Live;
  n.ceiling = ceiling;
  n.integrity = node_integrity(t.parent, t.tree_key, (uint32_t)free_index, n);
  nodes[free_index] = n;
  root->active_nodes += 1;
  root->generation = gen + 1;
  root->structural_revision += 1;
  refresh(t.parent, *root);
  ++counters.lease_scope_opens;
  *tree_out = make_tree(t.parent, *root);
  *scope_out = make_node(t.parent, t.tree_key, (uint32_t)free_index, n);
  return GLACIER_HIP_LEASE_OK;
}

int Bank::validate_tree(const Tree &t) {
  std::lock_guard<std::mutex> g(mu);
  RootSlot *root;
  return validate_tree_locked(t, &root);
}

int Bank::validate_node(const Tree &t, const Node &n) {
  std::lock_guard<std::mutex> g(mu);
  NodeSlot *s;
  return validate_node_locked(t, n, &s);
}

int Bank::close_tree(const Tree &t) {
  // closeLeaseTree (:2582-2622)
  std::lock_guard<std::mutex> g(mu);
  RootSlot *root;
  if (int rc = validate_tree_locked(t, &root)) return rc;
  const Slot &ps = slots[t.parent.slot_index];
  if (root->pending != Pending::None || !claim_zero(root->current) || ps.pub_active ||
      ps.pub_session != 0)
    return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  uint32_t count = 0;
  for (const NodeSlot &n : nodes) {
    if (!n.active || n.receipt_slot != t.parent.slot_index ||
        n.tree_identity_generation != t.identity_generation)
      continue;
    if (n.kind != GLACIER_HIP_LEASE_NODE_SCOPE || !claim_zero(n.claim) || !claim_zero(n.subtree))
      return GLACIER_HIP_LEASE_INVALID_TRANSITION;
    ++count;
  }
  if (count != root->active_nodes) return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  for (NodeSlot &n : nodes)
    if (n.active && n.receipt_slot == t.parent.slot_index &&
        n.tree_identity_generation == t.identity_generation)
      n = NodeSlot{};
  *root = RootSlot{};
  ++counters.lease_tree_closes;
  return GLACIER_HIP_LEASE_OK;
}

int Bank::bind_session(const Tree &t, uint64_t request_epoch, uint64_t session_id) {
  // bindPublicationSessionWithLeaseTree (:2731-2750) + bindPublicationSessionLocked (:2873-2890)
  if (request_epoch == 0 || session_id == 0) return GLACIER_HIP_LEASE_INVALID_CONFIGURATION;
  std::lock_guard<std::mutex> g(mu);
  RootSlot *root;
  if (int rc = validate_tree_locked(t, &root)) return rc;
  if (root->pending != Pending::None) return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  Slot &s = slots[t.parent.slot_index];
  if (s.state != SlotState::Committed || s.pub_session != 0 || s.pub_epoch != 0)
    return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  s.pub_epoch = request_epoch;
  s.pub_session = session_id;
  s.pub_next = 0;
  s.pub_active = false;
  s.pub_permit_integrity = 0;
  return GLACIER_HIP_LEASE_OK;
}

int Bank::close_session(const Receipt &r, uint64_t request_epoch, uint64_t session_id,
                        uint64_t expected_next) {
  // closePublicationSession (:3104-3124); a tree still holding charges,
  // or with a decision pending, keeps the session open
  std::lock_guard<std::mutex> g(mu);
  Slot *s;
  if (int rc = validate_receipt(r, &s)) return rc;
  const RootSlot &root = roots[r.slot_index];
  if (root.active && (root.pending != Pending::None || !claim_zero(root.current)))
    return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  if (s->state != SlotState::Committed || s->pub_epoch != request_epoch ||
      s->pub_session != session_id || s->pub_active || s->pub_next != expected_next)
    return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  s->pub_session = 0;  // the epoch and sequence stay as a tombstone until release
  s->pub_permit_integrity = 0;
  return GLACIER_HIP_LEASE_OK;
}

uint64_t Bank::pub_permit_integrity(const Receipt &r, uint64_t ep, uint64_t session, uint64_t seq,
                                    uint64_t gen) {
  uint64_t h = mix_receipt(kPubDomain, r);
  h = mix64(h ^ ep);
  h = mix64(h ^ session);
  h = mix64(h ^ seq);
  h = mix64(h ^ gen);
  return h ? h : 1;
}

int Bank::begin_publication_locked(const Receipt &r, uint64_t request_epoch, uint64_t session_id,
                                   uint64_t expected_sequence, PubPermit *out) {
  // beginPublicationLocked (:2982-3015)
  Slot *s;
  if (int rc = validate_receipt(r, &s)) return rc;
  if (roots[r.slot_index].active && roots[r.slot_index].pending != Pending::None)
    return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  if (s->state != SlotState::Committed || s->pub_epoch != request_epoch ||
      s->pub_session != session_id || s->pub_active || s->pub_next != expected_sequence)
    return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  if (s->pub_permit_gen == UINT64_MAX) return GLACIER_HIP_LEASE_INVALID_CONFIGURATION;
  s->pub_permit_gen += 1;
  PubPermit p{r, request_epoch, session_id, expected_sequence, s->pub_permit_gen, 0};
  p.integrity = pub_permit_integrity(r, request_epoch, session_id, expected_sequence, p.generation);
  s->pub_active = true;
  s->pub_permit_integrity = p.integrity;
  *out = p;
  return GLACIER_HIP_LEASE_OK;
}

int Bank::begin_publication(const Tree &t, uint64_t request_epoch, uint64_t session_id,
                            uint64_t expected_sequence, PubPermit *out) {
  // beginPublicationWithLeaseTree (:2938-2960)
  std::lock_guard<std::mutex> g(mu);
  RootSlot *root;
  if (int rc = validate_tree_locked(t, &root)) return rc;
  if (root->pending != Pending::None) return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  return begin_publication_locked(t.parent, request_epoch, session_id, expected_sequence, out);
}

int Bank::validate_pub_permit_locked(const PubPermit &p, Slot **out) {
  // validatePublicationPermit (:4133-4155): the permit is the committed
  // slot's live one for this request epoch, session and sequence, and its
  // integrity recomputes
  Slot *s;
  if (int rc = validate_receipt(p.receipt, &s)) return rc;
  if (s->state != SlotState::Committed || !s->pub_active || s->pub_permit_integrity != p.integrity ||
      s->pub_epoch != p.request_epoch || s->pub_session != p.session_id ||
      s->pub_next != p.sequence || s->pub_permit_gen != p.generation ||
      p.integrity != pub_permit_integrity(p.receipt, p.request_epoch, p.session_id, p.sequence,
                                          p.generation))
    return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  *out = s;
  return GLACIER_HIP_LEASE_OK;
}

int Bank::validate_publication(const PubPermit &p) {
  std::lock_guard<std::mutex> g(mu);
  Slot *s;
  return validate_pub_permit_locked(p, &s);
}

int Bank::commit_publication(const PubPermit &p) {
  // commitPublicationAssumeValid (:3076-3089): a permit that no longer
  // validates is reported instead of trapping
  std::lock_guard<std::mutex> g(mu);
  Slot *s;
  if (int rc = validate_pub_permit_locked(p, &s)) return rc;
  if (p.sequence == UINT64_MAX) return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  s->pub_active = false;
  s->pub_permit_integrity = 0;
  s->pub_next = p.sequence + 1;
  return GLACIER_HIP_LEASE_OK;
}

int Bank::abort_publication(const PubPermit &p) {
  // abortPublication (:3091-3102): the same permit validation as commit
  std::lock_guard<std::mutex> g(mu);
  Slot *s;
  if (int rc = validate_pub_permit_locked(p, &s)) return rc;
  s->pub_active = false;
  s->pub_permit_integrity = 0;
  return GLACIER_HIP_LEASE_OK;
}

uint64_t Bank::pending_digest(uint32_t slot, uint64_t tree_identity, uint64_t generation,
                              NState state) const {
  // leasePendingNodeDigest: the exact node set a decision covers
  uint64_t h = mix64(kStateDomain ^ generation ^ ((uint64_t)state << 60));
  for (size_t i = 0; i < nodes.size(); ++i) {
    const NodeSlot &n = nodes[i];
    if (!n.active || n.receipt_slot != slot || n.tree_identity_generation != tree_identity ||
        n.pending_generation != generation || n.state != state)
      continue;
    h = mix64(h ^ i);
    h = mix64(h ^ n.generation);
    h = mix64(h ^ n.integrity);
  }
  return h;
}

int Bank::validate_pending_locked(uint32_t slot, const RootSlot &root) {
  // validateLeasePendingState: the nodes of the pending decision are exactly
  // the ones it counted, in the state the decision put them in
  NState want = root.pending == Pending::Allocation ? NState::Reserved
                : root.pending == Pending::Retire   ? NState::Quiescing
                                                    : NState::FreeAuthorized;
  uint32_t count = 0;
  Claim sum{};
  for (const NodeSlot &n : nodes) {
    if (!n.active || n.receipt_slot != slot || n.tree_identity_generation != root.identity_generation ||
        n.pending_generation != root.pending_generation)
      continue;
    if (n.state != want) return GLACIER_HIP_LEASE_INVALID_TRANSITION;
    ++count;
    if (!add_claims(sum, n.claim, &sum)) return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  }
  if (count != root.pending_count || !claim_eq(sum, root.pending_claim) ||
      pending_digest(slot, root.identity_generation, root.pending_generation, want) !=
          root.pending_digest)
    return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  return GLACIER_HIP_LEASE_OK;
}

uint64_t Bank::batch_integrity(const Batch &b) {
  uint64_t h = mix_receipt(kBatchDomain, b.parent);
  for (uint64_t v : {b.tree_key, b.tree_identity_generation, b.tree_generation,
                     b.structural_revision, b.request_epoch, b.session_id, b.sequence, b.generation,
                     b.completion_tree_generation, (uint64_t)b.node_count, b.node_set_digest})
    h = mix64(h ^ v);
  h = mix_claim(h, b.claim);
  return h ? h : 1;
}

int Bank::reserve_allocations(const Tree &t, uint64_t request_epoch, uint64_t session_id,
                              uint64_t expected_sequence, const Spec *specs, size_t count,
                              Node *nodes_out, Tree *tree_out, Batch *batch_out) {
  // reserveAllocationsForSessionWithFundingMode (:1575-1783), additive
  if (request_epoch == 0 || session_id == 0 || count == 0 || count > UINT32_MAX)
    return GLACIER_HIP_LEASE_INVALID_CONFIGURATION;
  std::lock_guard<std::mutex> g(mu);
  RootSlot *root;
  if (int rc = validate_tree_locked(t, &root)) return rc;
  const Slot &ps = slots[t.parent.slot_index];
  if (root->pending != Pending::None || ps.pub_active || ps.pub_epoch != request_epoch ||
      ps.pub_session != session_id || ps.pub_next != expected_sequence ||
      root->structural_revision > UINT64_MAX - 2)
    return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  size_t free_nodes = 0;
  for (const NodeSlot &n : nodes) free_nodes += !n.active;
  if (free_nodes < count) {
    ++counters.rejected_lease_nodes;
    return GLACIER_HIP_LEASE_NODES_EXHAUSTED;
  }
  Claim aggregate{};
  for (size_t i = 0; i < count; ++i) {
    const Spec &sp = specs[i];
    if (sp.node_key == 0 || sp.binding_key == 0 || claim_zero(sp.claim))
      return GLACIER_HIP_LEASE_INVALID_CLAIM;
    NodeSlot *scope;
    if (int rc = validate_node_locked(t, sp.scope, &scope)) return rc;
    if (scope->kind != GLACIER_HIP_LEASE_NODE_SCOPE || scope->state != NState::Live)
      return GLACIER_HIP_LEASE_INVALID_TRANSITION;
    if (!add_claims(aggregate, sp.claim, &aggregate)) return GLACIER_HIP_LEASE_CLAIM_OVERFLOW;
    for (const NodeSlot &n : nodes) {
      if (!n.active || n.receipt_slot != t.parent.slot_index ||
          n.tree_identity_generation != t.identity_generation ||
          n.kind != GLACIER_HIP_LEASE_NODE_ALLOCATION)
        continue;
      if ((n.parent_index == sp.scope.node_index && n.node_key == sp.node_key) ||
          n.binding_key == sp.binding_key)
        return GLACIER_HIP_LEASE_INVALID_TRANSITION;
    }
    for (size_t j = 0; j < i; ++j)
      if ((specs[j].scope.node_index == sp.scope.node_index && specs[j].node_key == sp.node_key) ||
          specs[j].binding_key == sp.binding_key)
        return GLACIER_HIP_LEASE_INVALID_TRANSITION;
    Claim addition{};
    for (size_t j = 0; j < count; ++j)
      if (specs[j].scope.node_index == sp.scope.node_index &&
          !add_claims(addition, specs[j].claim, &addition))
        return GLACIER_HIP_LEASE_CLAIM_OVERFLOW;
    Claim scope_next;
    if (!add_claims(scope->subtree, addition, &scope_next)) return GLACIER_HIP_LEASE_CLAIM_OVERFLOW;
    if (!claim_within(scope_next, scope->ceiling)) return GLACIER_HIP_LEASE_INVALID_CLAIM;
  }
  Claim next_tree;
  if (!add_claims(root->current, aggregate, &next_tree)) return GLACIER_HIP_LEASE_CLAIM_OVERFLOW;
  if (!claim_within(next_tree, root->ceiling)) return GLACIER_HIP_LEASE_INVALID_CLAIM;
  Claim next_used;
  uint64_t hb;
  if (!add_claims(used, aggregate, &next_used) || !host_bytes(next_used, &hb)) {
    ++counters.rejected_lease_capacity;
    return GLACIER_HIP_LEASE_CLAIM_OVERFLOW;
  }
  if (!fits(next_used)) {
    ++counters.rejected_lease_capacity;
    return GLACIER_HIP_LEASE_CAPACITY_EXCEEDED;
  }
  // batch, each node, the reserve-tree and the settle/abort-tree generations
  uint64_t start;
  if (int rc = reserve_generations(count + 3, &start)) return rc;
  const uint64_t batch_gen = start;
  const uint64_t reserve_tree_gen = start + 1 + count;
  const uint64_t completion_gen = reserve_tree_gen + 1;
  size_t search = 0;
  for (size_t i = 0; i < count; ++i) {
    const Spec &sp = specs[i];
    while (nodes[search].active) ++search;
    const uint32_t index = (uint32_t)search++;
    NodeSlot n;
    n.active = true;
    n.receipt_slot = (uint32_t)t.parent.slot_index;
    n.tree_identity_generation = t.identity_generation;
    n.generation = start + 1 + i;
    n.parent_index = sp.scope.node_index;
    n.parent_generation = sp.scope.generation;
    n.node_key = sp.node_key;
    n.tenant_key = sp.scope.tenant_key;
    n.binding_key = sp.binding_key;
    n.kind = GLACIER_HIP_LEASE_NODE_ALLOCATION;
    n.state = NState::Reserved;
    n.ceiling = n.claim = n.subtree = sp.claim;
    n.pending_generation = batch_gen;
    n.integrity = node_integrity(t.parent, t.tree_key, index, n);
    nodes[index] = n;
    NodeSlot &scope = nodes[sp.scope.node_index];
    add_claims(scope.subtree, sp.claim, &scope.subtree);
    nodes_out[i] = make_node(t.parent, t.tree_key, index, n);
  }
  root->current = next_tree;
  root->active_nodes += (uint32_t)count;
  root->pending = Pending::Allocation;
  root->pending_generation = batch_gen;
  root->pending_completion = completion_gen;
  root->pending_count = (uint32_t)count;
  root->pending_claim = aggregate;
  root->pending_digest =
      pending_digest((uint32_t)t.parent.slot_index, t.identity_generation, batch_gen, NState::Reserved);
  root->generation = reserve_tree_gen;
  root->structural_revision += 1;
  used = next_used;
  peak = max_claims(peak, next_used);
  if (hb > peak_host_bytes) peak_host_bytes = hb;
  refresh(t.parent, *root);
  Batch b{t.parent, t.tree_key, t.identity_generation, root->generation, root->structural_revision,
          request_epoch, session_id, expected_sequence, batch_gen, completion_gen,
          (uint32_t)count, aggregate, root->pending_digest, 0};
  b.integrity = batch_integrity(b);
  ++counters.lease_allocation_reserves;
  *tree_out = make_tree(t.parent, *root);
  *batch_out = b;
  return GLACIER_HIP_LEASE_OK;
}

int Bank::validate_batch_locked(const Batch &b, RootSlot **out) {
  // validateLeaseAllocationBatchLocked (:3816-3857)
  if (b.node_count == 0 || claim_zero(b.claim) || b.integrity != batch_integrity(b))
    return GLACIER_HIP_LEASE_STALE_RESERVATION;
  Slot *s;
  if (int rc = validate_receipt(b.parent, &s)) return rc;
  RootSlot &root = roots[b.parent.slot_index];
  if (s->state != SlotState::Committed || s->pub_active || s->pub_epoch != b.request_epoch ||
      s->pub_session != b.session_id || s->pub_next != b.sequence || !root.active ||
      root.tree_key != b.tree_key || root.identity_generation != b.tree_identity_generation ||
      root.generation != b.tree_generation || root.structural_revision != b.structural_revision ||
      root.pending != Pending::Allocation || root.pending_generation != b.generation ||
      root.pending_completion != b.completion_tree_generation || root.pending_free_permit != 0 ||
      root.pending_free_completion != 0 || root.pending_count != b.node_count ||
      !claim_eq(root.pending_claim, b.claim) || root.pending_digest != b.node_set_digest ||
      root.pending_scope != kNoNode ||
      root.state_digest != state_digest((uint32_t)b.parent.slot_index, root) ||
      root.integrity != tree_integrity(b.parent, root))
    return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  if (int rc = validate_pending_locked((uint32_t)b.parent.slot_index, root)) return rc;
  *out = &root;
  return GLACIER_HIP_LEASE_OK;
}

int Bank::commit_allocations(const Batch &b, Tree *tree_out) {
  // commitAllocationsAfterAllocate (:1785-1823)
  std::lock_guard<std::mutex> g(mu);
  RootSlot *root;
  if (int rc = validate_batch_locked(b, &root)) return rc;
  for (NodeSlot &n : nodes)
    if (n.active && n.receipt_slot == b.parent.slot_index &&
        n.tree_identity_generation == b.tree_identity_generation && n.pending_generation == b.generation) {
      if (n.state != NState::Reserved) return GLACIER_HIP_LEASE_INVALID_TRANSITION;
      n.state = NState::Live;
      n.pending_generation = 0;
    }
  clear_pending(*root);
  root->generation = b.completion_tree_generation;
  root->structural_revision += 1;
  refresh(b.parent, *root);
  ++counters.lease_allocation_materializations;
  *tree_out = make_tree(b.parent, *root);
  return GLACIER_HIP_LEASE_OK;
}

int Bank::abort_allocations(const Batch &b, Tree *tree_out) {
  // abortAllocationsAfterFree (:1909-1956)
  std::lock_guard<std::mutex> g(mu);
  RootSlot *root;
  if (int rc = validate_batch_locked(b, &root)) return rc;
  Claim next_tree, next_used;
  if (!sub_claims(root->current, b.claim, &next_tree) || !sub_claims(used, b.claim, &next_used))
    return GLACIER_HIP_LEASE_CLAIM_OVERFLOW;
  for (NodeSlot &n : nodes) {
    if (!n.active || n.receipt_slot != b.parent.slot_index ||
        n.tree_identity_generation != b.tree_identity_generation || n.pending_generation != b.generation)
      continue;
    if (n.state != NState::Reserved) return GLACIER_HIP_LEASE_INVALID_TRANSITION;
    NodeSlot &scope = nodes[n.parent_index];
    sub_claims(scope.subtree, n.claim, &scope.subtree);
    n = NodeSlot{};
  }
  root->current = next_tree;
  root->active_nodes -= b.node_count;
  clear_pending(*root);
  root->generation = b.completion_tree_generation;
  root->structural_revision += 1;
  used = next_used;
  refresh(b.parent, *root);
  ++counters.lease_allocation_aborts;
  *tree_out = make_tree(b.parent, *root);
  return GLACIER_HIP_LEASE_OK;
}

uint64_t Bank::ticket_integrity(const Ticket &k) {
  uint64_t h = mix_receipt(kTicketDomain, k.parent);
  for (uint64_t v : {k.tree_key, k.tree_identity_generation, k.tree_generation, k.structural_revision,
                     k.request_epoch, k.session_id, k.sequence, k.generation,
                     k.decision_tree_generation, k.free_permit_generation,
                     k.free_completion_tree_generation, (uint64_t)k.scope_index, k.scope_generation,
                     (uint64_t)k.node_count, k.node_set_digest})
    h = mix64(h ^ v);
  h = mix_claim(h, k.claim);
  return h ? h : 1;
}

uint64_t Bank::free_permit_integrity(const FreePermit &p) {
  uint64_t h = mix_receipt(kPermitDomain, p.parent);
  for (uint64_t v : {p.tree_key, p.tree_identity_generation, p.tree_generation, p.structural_revision,
                     p.request_epoch, p.session_id, p.sequence, p.generation,
                     p.completion_tree_generation, (uint64_t)p.scope_index, p.scope_generation,
                     (uint64_t)p.node_count, p.node_set_digest})
    h = mix64(h ^ v);
  h = mix_claim(h, p.claim);
  return h ? h : 1;
}

int Bank::begin_retire(const Tree &t, const Node &scope, uint64_t request_epoch,
                       uint64_t session_id, uint64_t expected_sequence, Tree *tree_out,
                       Ticket *ticket_out) {
  // beginRetireSubtreeForSession (:2227-2343)
  if (request_epoch == 0 || session_id == 0) return GLACIER_HIP_LEASE_INVALID_CONFIGURATION;
  std::lock_guard<std::mutex> g(mu);
  RootSlot *root;
  if (int rc = validate_tree_locked(t, &root)) return rc;
  NodeSlot *ss;
  if (int rc = validate_node_locked(t, scope, &ss)) return rc;
  const Slot &ps = slots[t.parent.slot_index];
  if (ss->kind != GLACIER_HIP_LEASE_NODE_SCOPE || ss->state != NState::Live ||
      root->pending != Pending::None || ps.pub_active || ps.pub_epoch != request_epoch ||
      ps.pub_session != session_id || ps.pub_next != expected_sequence ||
      root->structural_revision > UINT64_MAX - 3)
    return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  uint32_t count = 0;
  Claim claim{};
  for (const NodeSlot &n : nodes) {
    if (!n.active || n.receipt_slot != t.parent.slot_index ||
        n.tree_identity_generation != t.identity_generation ||
        n.kind != GLACIER_HIP_LEASE_NODE_ALLOCATION || n.parent_index != scope.node_index)
      continue;
    if (n.state != NState::Live) return GLACIER_HIP_LEASE_INVALID_TRANSITION;
    ++count;
    if (!add_claims(claim, n.claim, &claim)) return GLACIER_HIP_LEASE_CLAIM_OVERFLOW;
  }
  if (count == 0 || claim_zero(claim) || !claim_eq(claim, ss->subtree))
    return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  // ticket, begin-tree, decision-tree, free permit and free-completion-tree
  uint64_t gen;
  if (int rc = reserve_generations(5, &gen)) return rc;
  for (NodeSlot &n : nodes)
    if (n.active && n.receipt_slot == t.parent.slot_index &&
        n.tree_identity_generation == t.identity_generation &&
        n.kind == GLACIER_HIP_LEASE_NODE_ALLOCATION && n.parent_index == scope.node_index) {
      n.state = NState::Quiescing;
      n.pending_generation = gen;
    }
  root->pending = Pending::Retire;
  root->pending_generation = gen;
  root->pending_completion = gen + 2;
  root->pending_free_permit = gen + 3;
  root->pending_free_completion = gen + 4;
  root->pending_scope = scope.node_index;
  root->pending_count = count;
  root->pending_claim = claim;
  root->pending_digest =
      pending_digest((uint32_t)t.parent.slot_index, t.identity_generation, gen, NState::Quiescing);
  root->generation = gen + 1;
  root->structural_revision += 1;
  refresh(t.parent, *root);
  Ticket k{t.parent, t.tree_key, t.identity_generation, root->generation, root->structural_revision,
           request_epoch, session_id, expected_sequence, gen, gen + 2, gen + 3, gen + 4,
           scope.node_index, scope.generation, count, claim, root->pending_digest, 0};
  k.integrity = ticket_integrity(k);
  ++counters.lease_reclaim_prepares;
  *tree_out = make_tree(t.parent, *root);
  *ticket_out = k;
  return GLACIER_HIP_LEASE_OK;
}

int Bank::validate_ticket_locked(const Ticket &k, RootSlot **out) {
  // validateLeaseRetireTicketLocked (:3859-3907)
  if (k.node_count == 0 || claim_zero(k.claim) || k.integrity != ticket_integrity(k))
    return GLACIER_HIP_LEASE_STALE_RESERVATION;
  Slot *s;
  if (int rc = validate_receipt(k.parent, &s)) return rc;
  if (k.scope_index >= nodes.size()) return GLACIER_HIP_LEASE_STALE_RESERVATION;
  RootSlot &root = roots[k.parent.slot_index];
  const NodeSlot &scope = nodes[k.scope_index];
  if (s->state != SlotState::Committed || s->pub_active || s->pub_epoch != k.request_epoch ||
      s->pub_session != k.session_id || s->pub_next != k.sequence || !root.active ||
      root.tree_key != k.tree_key || root.identity_generation != k.tree_identity_generation ||
      root.generation != k.tree_generation || root.structural_revision != k.structural_revision ||
      root.pending != Pending::Retire || root.pending_generation != k.generation ||
      root.pending_completion != k.decision_tree_generation ||
      root.pending_free_permit != k.free_permit_generation ||
      root.pending_free_completion != k.free_completion_tree_generation ||
      root.pending_scope != k.scope_index || root.pending_count != k.node_count ||
      !claim_eq(root.pending_claim, k.claim) || root.pending_digest != k.node_set_digest ||
      !scope.active || scope.kind != GLACIER_HIP_LEASE_NODE_SCOPE ||
      scope.generation != k.scope_generation || scope.receipt_slot != k.parent.slot_index ||
      scope.tree_identity_generation != k.tree_identity_generation ||
      root.state_digest != state_digest((uint32_t)k.parent.slot_index, root) ||
      root.integrity != tree_integrity(k.parent, root))
    return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  if (int rc = validate_pending_locked((uint32_t)k.parent.slot_index, root)) return rc;
  *out = &root;
  return GLACIER_HIP_LEASE_OK;
}

int Bank::cancel_retire(const Ticket &k, Tree *tree_out) {
  // cancelRetire (:2345-2381)
  std::lock_guard<std::mutex> g(mu);
  RootSlot *root;
  if (int rc = validate_ticket_locked(k, &root)) return rc;
  for (NodeSlot &n : nodes)
    if (n.active && n.receipt_slot == k.parent.slot_index &&
        n.tree_identity_generation == k.tree_identity_generation && n.pending_generation == k.generation) {
      if (n.state != NState::Quiescing) return GLACIER_HIP_LEASE_INVALID_TRANSITION;
      n.state = NState::Live;
      n.pending_generation = 0;
    }
  clear_pending(*root);
  root->generation = k.decision_tree_generation;
  root->structural_revision += 1;
  refresh(k.parent, *root);
  ++counters.lease_reclaim_cancels;
  *tree_out = make_tree(k.parent, *root);
  return GLACIER_HIP_LEASE_OK;
}

int Bank::authorize_free(const Ticket &k, Tree *tree_out, FreePermit *permit_out) {
  // authorizeFree (:2383-2452)
  std::lock_guard<std::mutex> g(mu);
  RootSlot *root;
  if (int rc = validate_ticket_locked(k, &root)) return rc;
  for (NodeSlot &n : nodes)
    if (n.active && n.receipt_slot == k.parent.slot_index &&
        n.tree_identity_generation == k.tree_identity_generation && n.pending_generation == k.generation) {
      if (n.state != NState::Quiescing) return GLACIER_HIP_LEASE_INVALID_TRANSITION;
      n.state = NState::FreeAuthorized;
      n.pending_generation = k.free_permit_generation;
    }
  root->pending = Pending::Free;
  root->pending_generation = k.free_permit_generation;
  root->pending_completion = k.free_completion_tree_generation;
  root->pending_free_permit = root->pending_free_completion = 0;
  root->pending_digest = pending_digest((uint32_t)k.parent.slot_index, k.tree_identity_generation,
                                        k.free_permit_generation, NState::FreeAuthorized);
  root->generation = k.decision_tree_generation;
  root->structural_revision += 1;
  refresh(k.parent, *root);
  FreePermit p{k.parent, k.tree_key, k.tree_identity_generation, root->generation,
               root->structural_revision, k.request_epoch, k.session_id, k.sequence,
               k.free_permit_generation, k.free_completion_tree_generation, k.scope_index,
               k.scope_generation, k.node_count, k.claim, root->pending_digest, 0};
  p.integrity = free_permit_integrity(p);
  ++counters.lease_reclaim_authorizations;
  *tree_out = make_tree(k.parent, *root);
  *permit_out = p;
  return GLACIER_HIP_LEASE_OK;
}

int Bank::validate_free_permit_locked(const FreePermit &p, RootSlot **out) {
  // validateLeaseFreePermitLocked (:3909-3957)
  if (p.node_count == 0 || claim_zero(p.claim) || p.integrity != free_permit_integrity(p))
    return GLACIER_HIP_LEASE_STALE_RESERVATION;
  Slot *s;
  if (int rc = validate_receipt(p.parent, &s)) return rc;
  if (p.scope_index >= nodes.size()) return GLACIER_HIP_LEASE_STALE_RESERVATION;
  RootSlot &root = roots[p.parent.slot_index];
  const NodeSlot &scope = nodes[p.scope_index];
  if (s->state != SlotState::Committed || s->pub_active || s->pub_epoch != p.request_epoch ||
      s->pub_session != p.session_id || s->pub_next != p.sequence || !root.active ||
      root.tree_key != p.tree_key || root.identity_generation != p.tree_identity_generation ||
      root.generation != p.tree_generation || root.structural_revision != p.structural_revision ||
      root.pending != Pending::Free || root.pending_generation != p.generation ||
      root.pending_completion != p.completion_tree_generation || root.pending_free_permit != 0 ||
      root.pending_free_completion != 0 || root.pending_scope != p.scope_index ||
      root.pending_count != p.node_count || !claim_eq(root.pending_claim, p.claim) ||
      root.pending_digest != p.node_set_digest || !scope.active ||
      scope.kind != GLACIER_HIP_LEASE_NODE_SCOPE || scope.generation != p.scope_generation ||
      scope.receipt_slot != p.parent.slot_index ||
      scope.tree_identity_generation != p.tree_identity_generation ||
      root.state_digest != state_digest((uint32_t)p.parent.slot_index, root) ||
      root.integrity != tree_integrity(p.parent, root))
    return GLACIER_HIP_LEASE_INVALID_TRANSITION;
  if (int rc = validate_pending_locked((uint32_t)p.parent.slot_index, root)) return rc;
  *out = &root;
  return GLACIER_HIP_LEASE_OK;
}

int Bank::commit_free(const FreePermit &p, Tree *tree_out) {
  // commitFreeAfterAllocatorFree (:2454-2502)
  std::lock_guard<std::mutex> g(mu);
  RootSlot *root;
  if (int rc = validate_free_permit_locked(p, &root)) return rc;
  NodeSlot &scope = nodes[p.scope_index];
  Claim next_tree, next_used, next_scope;
  if (!sub_claims(root->current, p.claim, &next_tree) || !sub_claims(used, p.claim, &next_used) ||
      !sub_claims(scope.subtree, p.claim, &next_scope))
    return GLACIER_HIP_LEASE_CLAIM_OVERFLOW;
  for (NodeSlot &n : nodes) {
    if (!n.active || n.receipt_slot != p.parent.slot_index ||
        n.tree_identity_generation != p.tree_identity_generation || n.pending_generation != p.generation)
      continue;
    if (n.state != NState::FreeAuthorized) return GLACIER_HIP_LEASE_INVALID_TRANSITION;
    n = NodeSlot{};
  }
  scope.subtree = next_scope;
  root->current = next_tree;
  root->active_nodes -= p.node_count;
  clear_pending(*root);
  root->generation = p.completion_tree_generation;
  root->structural_revision += 1;
  used = next_used;
  refresh(p.parent, *root);
  ++counters.lease_reclaim_commits;
  *tree_out = make_tree(p.parent, *root);
  return GLACIER_HIP_LEASE_OK;
}

void Bank::snapshot(glacier_hip_lease_bank_snapshot_t *out) {
  // snapshotV3 (:3218-3406): accounting and node-state counts
  std::lock_guard<std::mutex> g(mu);
  *out = counters;
  out->used = used;
  out->peak = peak;
  out->peak_host_bytes = peak_host_bytes;
  for (const Slot &s : slots) {
    out->active_reservations += s.state == SlotState::Reserved;
    out->committed_receipts += s.state == SlotState::Committed;
  }
  for (const RootSlot &r : roots) out->active_lease_trees += r.active;
  for (const NodeSlot &n : nodes) {
    if (!n.active) continue;
    ++out->active_lease_nodes;
    if (n.kind == GLACIER_HIP_LEASE_NODE_SCOPE) {
      ++out->active_lease_scopes;
      continue;
    }
    out->reserved_unmaterialized_allocations += n.state == NState::Reserved;
    out->live_allocations += n.state == NState::Live;
    out->quiescing_allocations += n.state == NState::Quiescing;
    out->free_authorized_allocations += n.state == NState::FreeAuthorized;
  }
}

}  // namespace glb

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

glacier_hip_lease_bank *glacier_hip_lease_bank_create(uint32_t slot_count, uint32_t node_count,
                                                      const glacier_hip_limits_t *limits,
                                                      uint64_t epoch) {
  // Bank.initWithLeaseTree (:929-974)
  if (slot_count == 0 || node_count == 0 || !limits || epoch == 0) return nullptr;
  return new (std::nothrow) glacier_hip_lease_bank(slot_count, node_count, *limits, epoch);
}

void glacier_hip_lease_bank_destroy(glacier_hip_lease_bank *b) { delete b; }

int glacier_hip_lease_bank_reserve(glacier_hip_lease_bank *b, uint64_t owner_key,
                                   const glacier_hip_claim_t *claim,
                                   glacier_hip_bank_receipt_t *out) {
  if (!b || !claim || !out) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return b->bank.reserve(owner_key, *claim, out);
}

int glacier_hip_lease_bank_commit(glacier_hip_lease_bank *b, const glacier_hip_bank_receipt_t *res,
                                  glacier_hip_bank_receipt_t *out) {
  if (!b || !res || !out) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return b->bank.commit(*res, out);
}

int glacier_hip_lease_bank_cancel(glacier_hip_lease_bank *b, const glacier_hip_bank_receipt_t *res) {
  if (!b || !res) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return b->bank.cancel(*res);
}

int glacier_hip_lease_bank_release(glacier_hip_lease_bank *b, const glacier_hip_bank_receipt_t *r) {
  if (!b || !r) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return b->bank.release(*r);
}

int glacier_hip_lease_tree_open(glacier_hip_lease_bank *b, const glacier_hip_bank_receipt_t *r,
                                uint64_t tree_key, uint64_t authority_key,
                                const glacier_hip_claim_t *ceiling, glacier_hip_lease_tree_t *out) {
  if (!b || !r || !ceiling || !out) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return b->bank.open_tree(*r, tree_key, authority_key, *ceiling, out);
}

int glacier_hip_lease_scope_open(glacier_hip_lease_bank *b, glacier_hip_lease_tree_t *tree,
                                 uint64_t scope_key, uint64_t tenant_key,
                                 const glacier_hip_claim_t *ceiling, glacier_hip_lease_node_t *out) {
  if (!b || !tree || !ceiling || !out) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  glacier_hip_lease_tree_t t;
  glacier_hip_lease_node_t n;
  int rc = b->bank.open_scope(*tree, scope_key, tenant_key, *ceiling, &t, &n);
  if (rc) return rc;
  *tree = t;
  *out = n;
  return GLACIER_HIP_LEASE_OK;
}

int glacier_hip_lease_tree_close(glacier_hip_lease_bank *b, const glacier_hip_lease_tree_t *tree) {
  if (!b || !tree) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return b->bank.close_tree(*tree);
}

int glacier_hip_lease_tree_validate(glacier_hip_lease_bank *b, const glacier_hip_lease_tree_t *tree) {
  if (!b || !tree) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return b->bank.validate_tree(*tree);
}

int glacier_hip_lease_node_validate(glacier_hip_lease_bank *b, const glacier_hip_lease_tree_t *tree,
                                    const glacier_hip_lease_node_t *node) {
  if (!b || !tree || !node) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return b->bank.validate_node(*tree, *node);
}

int glacier_hip_lease_session_bind(glacier_hip_lease_bank *b, const glacier_hip_lease_tree_t *tree,
                                   uint64_t request_epoch, uint64_t session_id) {
  if (!b || !tree) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return b->bank.bind_session(*tree, request_epoch, session_id);
}

int glacier_hip_lease_session_close(glacier_hip_lease_bank *b, const glacier_hip_bank_receipt_t *r,
                                    uint64_t request_epoch, uint64_t session_id,
                                    uint64_t expected_next_sequence) {
  if (!b || !r) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return b->bank.close_session(*r, request_epoch, session_id, expected_next_sequence);
}

int glacier_hip_lease_publication_begin(glacier_hip_lease_bank *b, const glacier_hip_lease_tree_t *tree,
                                        uint64_t request_epoch, uint64_t session_id,
                                        uint64_t expected_sequence,
                                        glacier_hip_publication_permit_t *out) {
  if (!b || !tree || !out) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return b->bank.begin_publication(*tree, request_epoch, session_id, expected_sequence, out);
}

int glacier_hip_lease_publication_commit(glacier_hip_lease_bank *b,
                                         const glacier_hip_publication_permit_t *p) {
  if (!b || !p) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return b->bank.commit_publication(*p);
}

int glacier_hip_lease_publication_abort(glacier_hip_lease_bank *b,
                                        const glacier_hip_publication_permit_t *p) {
  if (!b || !p) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  return b->bank.abort_publication(*p);
}

int glacier_hip_lease_bank_snapshot(glacier_hip_lease_bank *b, glacier_hip_lease_bank_snapshot_t *out) {
  if (!b || !out) return GLACIER_HIP_LEASE_INVALID_ARGUMENT;
  b->bank.snapshot(out);
  return GLACIER_HIP_LEASE_OK;
}

}  // extern "C"
