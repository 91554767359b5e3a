// leased_kv.h — LeaseTree-backed page ownership of one lane's page map.
//
// Restates the reference's LeasedPagedKVCache (leased_paged_kv_cache.zig):
// one caller-owned PageLeaseBindingV1 per logical page; a page payload is
// charged as an exact allocation leaf of the lane's scope before the page
// map takes it from the pool, settled right after, uncharged if the map
// could not take it; terminal seal binds the committed root and logical KV
// digest to one publication sequence of the cohort; terminal reclaim
// retires the scope, returns every payload to the pool, then uncharges.
//   init                      :311-357
//   bindingSummaryForState    :1178-1250
//   planNextRow               :453-480
//   beginRowPlanned           :482-565
//   commitRowTxn / abortRowTxn :666-689
//   sealTerminalForPublication :691-757
//   beginTerminalReclaim       :852-867, beginReclaimExact :918-1036
//   commitReclaimAfterFree     :1040-1080
//   reclaimForTeardown         :894-916
//   pageBindingKey / pageBindingIntegrity :1353-1382
// The coordinator works on a host page map (rows staged through it, as the
// reference's caller does) or on a device session lane (the session's
// decode and prefill steps call reserve_rows / settle_rows / end_rows around
// the page map's row transaction, so a step's new pages are charged before
// it takes them). Address-bound identity (the reference fences copies of the
// coordinator object) is the opaque handle here: the ABI hands out no copies.
#pragma once
#include <stdint.h>

#include <functional>
#include <vector>

#include "lease_bank.h"
#include "paged_kv.h"

namespace glb {

using Binding = glacier_hip_page_lease_binding_t;
using Summary = glacier_hip_binding_summary_t;
using Root = glacier_hip_page_map_root_t;

constexpr uint64_t kLeasedAbi = 0x47504c4300000002ull;
constexpr uint64_t kBindingAbi = 0x47504c4200000001ull;
constexpr uint64_t kRowPlanAbi = 0x47504c5000000001ull;
constexpr uint64_t kRowTxnAbi = 0x47504c5200000001ull;
constexpr uint64_t kTerminalSealAbi = 0x47504c5300000001ull;
constexpr uint64_t kFreedPayloadAbi = 0x47504c4600000001ull;
constexpr uint64_t kReclaimReceiptAbi = 0x47504c4300000002ull;

uint64_t page_binding_key(uint64_t cache_instance, uint64_t logical_page);
uint64_t page_binding_integrity(const Binding &b);

struct Target {
  gpk::Cache *cache = nullptr;
  gpk::PagePool *pool = nullptr;
  glacier_hip_kv_pages *host = nullptr;       // host map: rows staged through the coordinator
  std::function<int(uint8_t out[32])> kv_sha256;  // logicalKvSha256, lease status codes
};

class Leased {
 public:
  int init(Bank *bank, Tree *tree, const Node &scope, const Target &target, Binding *bindings,
           uint32_t binding_count, uint64_t request_epoch, uint64_t session_id, uint64_t *sequence);

  // host page maps
  int plan_next_row(glacier_hip_leased_row_plan_t *out);
  int begin_row(const glacier_hip_leased_row_plan_t &plan, glacier_hip_leased_row_txn_t *out);
  int commit_row(const glacier_hip_leased_row_txn_t &txn, Root *root_out);
  int abort_row(const glacier_hip_leased_row_txn_t &txn);

  // device session lanes: around the page map's begin of `rows` rows
  int reserve_rows(uint32_t rows);   // charge the payloads the rows will take
  void settle_rows(bool taken);      // the map took them (settle) or did not (uncharge)
  void end_rows() { lane_active = false; }  // the step committed or aborted
  bool lane_target() const { return target.host == nullptr; }
  // the map still exists and this coordinator still owns it
  bool leased_ok() const { return target.cache && target.cache->is_leased(instance, (uintptr_t)this); }
  void orphan() { target.cache = nullptr; }  // the session that held the lane is gone

  int binding_summary(uint32_t state, Summary *out);
  // allocationSetCommitmentForState (:1253-1291)
  int allocation_set(uint32_t state, glacier_hip_allocation_set_v2_t *out);
  int lifecycle(uint32_t *out) const;
  int root(Root *out) const;
  int kv_sha256(uint8_t out[32]) { return target.kv_sha256(out); }
  int seal_terminal(const Root &expected_root, const uint8_t kv[32], uint64_t sequence,
                    uint32_t reason, uint32_t token, glacier_hip_terminal_seal_t *out);
  int begin_reclaim(const glacier_hip_terminal_seal_t &seal, uint64_t expected_sequence,
                    glacier_hip_freed_payload_t *out);
  int commit_reclaim(const glacier_hip_freed_payload_t &freed, glacier_hip_reclaim_receipt_t *out);
  int reclaim_for_teardown(uint64_t expected_sequence);
  // A staged publication wave's terminal lane (planTerminalForTokenTxn
  // :759-808 + finalizeTerminalAssumePublished :810-850): after the wave's
  // permit for `sequence` committed, the seal binds the lane's committed
  // root, logical KV digest and bindings to the wave's proposal and commit
  // digests, with the token's terminal reason.
  int finalize_wave_terminal(uint64_t sequence, uint32_t reason, uint32_t token,
                             const uint8_t proposal[32], const uint8_t commit[32]);
  int terminal_seal(glacier_hip_terminal_seal_t *out, uint8_t proposal[32], uint8_t commit[32]) const;

  Bank *bank = nullptr;
  Tree *tree = nullptr;
  Node scope{};
  Target target;
  Binding *bindings = nullptr;
  uint32_t binding_count = 0;
  uint64_t request_epoch = 0, session_id = 0;
  uint64_t *sequence = nullptr;
  uint64_t instance = 0, next_generation = 1;

 private:
  int validate_mutable();
  int validate_active(const glacier_hip_leased_row_txn_t &txn) const;
  int begin_reclaim_exact(const uint8_t seal_digest[32], const Root &expected_root,
                          const uint8_t kv[32], const Summary &expected_bindings,
                          const uint64_t *terminal_sequence, uint64_t expected_sequence,
                          glacier_hip_freed_payload_t *out);
  Binding free_binding() const;
  Binding live_binding(uint64_t logical_page, uint64_t payload_bytes, const Node &leaf) const;

  bool has_row = false, lane_active = false;
  glacier_hip_leased_row_txn_t row{};
  bool has_seal = false, seal_v3 = false;
  glacier_hip_terminal_seal_t seal{};
  uint8_t seal_proposal[32] = {}, seal_commit[32] = {};
  bool has_pending = false;
  glacier_hip_freed_payload_t pending_freed{};
  FreePermit pending_permit{};
  bool reclaimed = false;
  // a session step's reservation between reserve_rows and settle_rows
  bool has_batch = false;
  Batch batch{};
  std::vector<Node> batch_leaves;
  std::vector<uint64_t> batch_pages;
};

}  // namespace glb

struct glacier_hip_leased_kv {
  glb::Leased lease;
  void (*detach)(glacier_hip_leased_kv *) = nullptr;  // session lanes: unhook on destroy
  void *owner = nullptr;
  uint32_t lane = 0;
};
