// lease_bank.h — ResourceBank receipts with LeaseTree page ownership.
//
// Host-side restatement of the parts of the reference's ResourceBank
// (core/resource_bank.zig) that leased paged KV uses:
//   receipts        reserve :976-1044, commit :1046-1076, cancel :1078-1095,
//                   release :3166-3184, validateReceipt :4084-4108
//   LeaseTree       openLeaseTree :1368-1446, openLeaseScope :1448-1514,
//                   reserveAllocationsForSession :1534-1783,
//                   commitAllocationsAfterAllocate :1785-1823,
//                   abortAllocationsAfterFree :1909-1956,
//                   beginRetireSubtreeForSession :2227-2343,
//                   cancelRetire :2345-2381, authorizeFree :2383-2452,
//                   commitFreeAfterAllocatorFree :2454-2502,
//                   closeLeaseTree :2582-2622, validate* :3739-3957
//   publication     bindPublicationSessionWithLeaseTree :2731-2750,
//                   beginPublicationWithLeaseTree :2938-2960 with
//                   beginPublicationLocked, commitPublicationAssumeValid
//                   :3076-3089, abortPublication :3091-3102,
//                   closePublicationSession :3104-3124
//   accounting      Claim/Limits :61-140, SnapshotV3 :703-754
// Generations come from one bank-wide counter in the reference's order
// (each operation reserves its block before it changes anything), so the
// generation fields of every token equal the reference's for the same call
// sequence. Integrity words and the tree state digest are this library's own
// mixes (SplitMix64's finaliser chained over the token fields): tokens are
// only ever compared with the bank's own state.
//
// Left out (no caller on the leased page path): child leases, pins,
// receipt-funded trees and restored publication sessions.
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <mutex>
#include <vector>

#include "../../include/glacier_hip.h"

namespace glb {

using Claim = glacier_hip_claim_t;
using Limits = glacier_hip_limits_t;
using Receipt = glacier_hip_bank_receipt_t;
using Tree = glacier_hip_lease_tree_t;
using Node = glacier_hip_lease_node_t;

constexpr uint32_t kNoNode = 0xffffffffu;
constexpr uint64_t kTreeAbi = 0x474c545200000001ull;
constexpr uint64_t kNodeAbi = 0x474c4e4400000001ull;

uint64_t mix64(uint64_t v);  // SplitMix64 finaliser
bool claim_zero(const Claim &c);
bool claim_eq(const Claim &a, const Claim &b);
bool claim_within(const Claim &v, const Claim &ceiling);
bool add_claims(const Claim &a, const Claim &b, Claim *out);
bool sub_claims(const Claim &a, const Claim &b, Claim *out);
uint64_t mix_claim(uint64_t h, const Claim &c);

enum class SlotState : uint8_t { Free, Reserved, Committed };
struct Slot {
  SlotState state = SlotState::Free;
  uint64_t generation = 0, owner_key = 0;
  Claim claim{};
  uint64_t integrity = 0;
  uint64_t pub_epoch = 0, pub_session = 0, pub_next = 0, pub_permit_gen = 0;
  bool pub_active = false;
  uint64_t pub_permit_integrity = 0;
};

enum class NState : uint8_t { Free, Live, Reserved, Quiescing, FreeAuthorized };
enum class Pending : uint8_t { None, Allocation, Retire, Free };

struct RootSlot {
  bool active = false;
  uint64_t tree_key = 0, authority_key = 0, identity_generation = 0, generation = 0;
  uint64_t structural_revision = 0;
  Claim ceiling{}, current{};
  uint32_t active_nodes = 0;
  uint64_t state_digest = 0, integrity = 0;
  Pending pending = Pending::None;
  uint64_t pending_generation = 0, pending_completion = 0;
  uint64_t pending_free_permit = 0, pending_free_completion = 0;
  uint32_t pending_scope = kNoNode, pending_count = 0;
  Claim pending_claim{};
  uint64_t pending_digest = 0;
};

struct NodeSlot {
  bool active = false;
  uint32_t receipt_slot = 0;
  uint64_t tree_identity_generation = 0, generation = 0;
  uint32_t parent_index = kNoNode;
  uint64_t parent_generation = 0, node_key = 0, tenant_key = 0, binding_key = 0;
  uint32_t kind = GLACIER_HIP_LEASE_NODE_SCOPE;
  NState state = NState::Free;
  Claim ceiling{}, claim{}, subtree{};
  uint64_t pending_generation = 0;
  uint64_t integrity = 0;
};

// LeaseAllocationSpecV1 (:337-342)
struct Spec {
  Node scope;
  uint64_t node_key, binding_key;
  Claim claim;
};

// LeaseAllocationBatchV1 (:344-360)
struct Batch {
  Receipt parent;
  uint64_t tree_key, tree_identity_generation, tree_generation, structural_revision;
  uint64_t request_epoch, session_id, sequence, generation, completion_tree_generation;
  uint32_t node_count;
  Claim claim;
  uint64_t node_set_digest, integrity;
};

// LeaseRetireTicketV1 (:392-412) and LeaseFreePermitV1 (:367-385)
struct Ticket {
  Receipt parent;
  uint64_t tree_key, tree_identity_generation, tree_generation, structural_revision;
  uint64_t request_epoch, session_id, sequence, generation;
  uint64_t decision_tree_generation, free_permit_generation, free_completion_tree_generation;
  uint32_t scope_index;
  uint64_t scope_generation;
  uint32_t node_count;
  Claim claim;
  uint64_t node_set_digest, integrity;
};
struct FreePermit {
  Receipt parent;
  uint64_t tree_key, tree_identity_generation, tree_generation, structural_revision;
  uint64_t request_epoch, session_id, sequence, generation, completion_tree_generation;
  uint32_t scope_index;
  uint64_t scope_generation;
  uint32_t node_count;
  Claim claim;
  uint64_t node_set_digest, integrity;
};

// PublicationPermit (:646-654)
using PubPermit = glacier_hip_publication_permit_t;

class Bank {
 public:
  Bank(uint32_t slot_count, uint32_t node_count, const Limits &limits, uint64_t epoch);

  int reserve(uint64_t owner_key, const Claim &claim, Receipt *out);
  int commit(const Receipt &reservation, Receipt *out);
  int cancel(const Receipt &reservation);
  int release(const Receipt &receipt);

  int open_tree(const Receipt &receipt, uint64_t tree_key, uint64_t authority_key,
                const Claim &ceiling, Tree *out);
  int open_scope(const Tree &tree, uint64_t scope_key, uint64_t tenant_key, const Claim &ceiling,
                 Tree *tree_out, Node *scope_out);
  int close_tree(const Tree &tree);
  int validate_tree(const Tree &tree);
  int validate_node(const Tree &tree, const Node &node);

  int bind_session(const Tree &tree, uint64_t request_epoch, uint64_t session_id);
  int close_session(const Receipt &receipt, uint64_t request_epoch, uint64_t session_id,
                    uint64_t expected_next_sequence);
  int begin_publication(const Tree &tree, uint64_t request_epoch, uint64_t session_id,
                        uint64_t expected_sequence, PubPermit *out);
  int validate_publication(const PubPermit &permit);
  int commit_publication(const PubPermit &permit);
  int abort_publication(const PubPermit &permit);

  int reserve_allocations(const Tree &tree, uint64_t request_epoch, uint64_t session_id,
                          uint64_t expected_sequence, const Spec *specs, size_t count,
                          Node *nodes_out, Tree *tree_out, Batch *batch_out);
  int commit_allocations(const Batch &batch, Tree *tree_out);
  int abort_allocations(const Batch &batch, Tree *tree_out);
  int begin_retire(const Tree &tree, const Node &scope, uint64_t request_epoch,
                   uint64_t session_id, uint64_t expected_sequence, Tree *tree_out,
                   Ticket *ticket_out);
  int cancel_retire(const Ticket &ticket, Tree *tree_out);
  int authorize_free(const Ticket &ticket, Tree *tree_out, FreePermit *permit_out);
  int commit_free(const FreePermit &permit, Tree *tree_out);

  void snapshot(glacier_hip_lease_bank_snapshot_t *out);

  // Integrity of a token as the bank would issue it (used by coordinators
  // to bind tokens into their own digests).
  static uint64_t node_integrity(const Receipt &parent, uint64_t tree_key, uint32_t index,
                                 const NodeSlot &n);

 private:
  int validate_receipt(const Receipt &r, Slot **out);
  int reserve_generations(uint64_t count, uint64_t *first);
  int validate_tree_locked(const Tree &t, RootSlot **out);
  int validate_node_locked(const Tree &t, const Node &n, NodeSlot **out);
  int validate_batch_locked(const Batch &b, RootSlot **out);
  int validate_ticket_locked(const Ticket &k, RootSlot **out);
  int validate_free_permit_locked(const FreePermit &p, RootSlot **out);
  int validate_pending_locked(uint32_t slot, const RootSlot &root);
  int validate_pub_permit_locked(const PubPermit &p, Slot **out);
  uint64_t state_digest(uint32_t slot, const RootSlot &root) const;
  uint64_t pending_digest(uint32_t slot, uint64_t tree_identity, uint64_t generation,
                          NState state) const;
  void refresh(const Receipt &r, RootSlot &root);
  Tree make_tree(const Receipt &r, const RootSlot &root) const;
  Node make_node(const Receipt &r, uint64_t tree_key, uint32_t index, const NodeSlot &n) const;
  static uint64_t token_integrity(uint64_t epoch, uint64_t slot, uint64_t gen, uint64_t owner,
                                  const Claim &claim, uint64_t domain);
  static uint64_t tree_integrity(const Receipt &r, const RootSlot &root);
  static uint64_t batch_integrity(const Batch &b);
  static uint64_t ticket_integrity(const Ticket &k);
  static uint64_t free_permit_integrity(const FreePermit &p);
  static uint64_t pub_permit_integrity(const Receipt &r, uint64_t epoch, uint64_t session,
                                       uint64_t seq, uint64_t gen);
  int begin_publication_locked(const Receipt &r, uint64_t request_epoch, uint64_t session_id,
                               uint64_t expected_sequence, PubPermit *out);
  bool fits(const Claim &c) const;

 public:
  std::mutex mu;
  uint64_t epoch;
  Limits limits;
  std::vector<Slot> slots;
  std::vector<RootSlot> roots;
  std::vector<NodeSlot> nodes;
  Claim used{}, peak{};
  uint64_t peak_host_bytes = 0;
  uint64_t next_generation = 1, next_lease_generation = 1;
  glacier_hip_lease_bank_snapshot_t counters{};  // the event counters only
};

}  // namespace glb

struct glacier_hip_lease_bank {
  glb::Bank bank;
  glacier_hip_lease_bank(uint32_t s, uint32_t n, const glacier_hip_limits_t &l, uint64_t e)
      : bank(s, n, l, e) {}
};
