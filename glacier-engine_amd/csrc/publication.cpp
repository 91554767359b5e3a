// publication.cpp — digests of the per-token publication transaction
// (src/paged_token_txn.zig): the KV state chain of a lane (initialStateChain
// :774-786, appendedStateChain :788-808 over hashRoot :762-772),
// proposalSha256 (:1064-1130) and commitSha256 (:1132-1148), all over the
// reference's field order with little-endian integers. Pure host code: the
// sessions fill the proposal, these functions seal it.
#include <string.h>

#include "host_util.h"
#include "publication.h"

namespace gpub {

static void hash_root(gh::Sha256 &h, const glacier_hip_page_map_root_t &r) {
  h.u64(r.abi_version);
  h.u64(r.cache_instance);
  h.u64(r.generation);
  h.u64(r.committed_len);
  h.u64(r.committed_pages);
  h.update(r.ownership_sha256, 32);
}

static void u8(gh::Sha256 &h, uint8_t v) { h.update(&v, 1); }

static void seed_chain(const char *domain, size_t n, const uint8_t logical_kv_sha256[32],
                       const glacier_hip_page_map_root_t &root, uint8_t out[32]) {
  gh::Sha256 h;
  h.update(domain, n);  // with its NUL
  h.update(logical_kv_sha256, 32);
  hash_root(h, root);
  h.final(out);
}

static void append_chain(const char *domain, size_t n, const uint8_t chain_before[32],
                         const glacier_hip_page_map_root_t &before,
                         const glacier_hip_page_map_root_t &after,
                         const glacier_hip_row_txn_mark_t &mark,
                         const uint8_t row_payload_sha256[32], uint8_t out[32]) {
  gh::Sha256 h;
  h.update(domain, n);  // with its NUL
  h.update(chain_before, 32);
  hash_root(h, before);
  hash_root(h, after);
  h.u64(mark.page_ref.abi_version);
  h.u64(mark.page_ref.cache_instance);
  h.u64(mark.page_ref.logical_page);
  h.u64(mark.page_ref.ownership_generation);
  h.u64(mark.generation);
  h.update(row_payload_sha256, 32);
  h.final(out);
}

void initial_state_chain(const uint8_t logical_kv_sha256[32], const glacier_hip_page_map_root_t &root,
                         uint8_t out[32]) {
  static const char d[] = "glacier-paged-token-kv-chain-seed-v1";
  seed_chain(d, sizeof d, logical_kv_sha256, root, out);
}

void appended_state_chain(const uint8_t chain_before[32], const glacier_hip_page_map_root_t &before,
                          const glacier_hip_page_map_root_t &after,
                          const glacier_hip_row_txn_mark_t &mark, const uint8_t row_payload_sha256[32],
                          uint8_t out[32]) {
  static const char d[] = "glacier-paged-token-kv-chain-append-v1";
  append_chain(d, sizeof d, chain_before, before, after, mark, row_payload_sha256, out);
}

void initial_state_chain_v3(const uint8_t logical_kv_sha256[32],
                            const glacier_hip_page_map_root_t &root, uint8_t out[32]) {
  static const char d[] = "glacier-paged-lease-token-kv-chain-seed-v3";
  seed_chain(d, sizeof d, logical_kv_sha256, root, out);
}

void appended_state_chain_v3(const uint8_t chain_before[32], const glacier_hip_page_map_root_t &before,
                             const glacier_hip_page_map_root_t &after,
                             const glacier_hip_row_txn_mark_t &mark,
                             const uint8_t row_payload_sha256[32], uint8_t out[32]) {
  static const char d[] = "glacier-paged-lease-token-kv-chain-append-v3";
  append_chain(d, sizeof d, chain_before, before, after, mark, row_payload_sha256, out);
}

void proposal_sha256(const glacier_hip_token_proposal_v1_t &p, uint8_t out[32]) {
  gh::Sha256 h;
  h.update("glacier-paged-token-txn-proposal-v1", sizeof("glacier-paged-token-txn-proposal-v1"));  // with its NUL
  h.u64(p.abi_version);
  h.u64(p.resource_bank_abi);
  h.u64(p.resource_publication_fence_abi);
  h.u64(p.paged_kv_abi);
  h.u64(p.page_map_root_abi);
  h.u64(p.page_ref_abi);
  h.u64(p.page_transition_abi);
  h.u64(p.kv_row_txn_abi);
  h.u64(p.execution_abi);
  h.u64(p.request_epoch);
  h.u64(p.transaction_sequence);
  h.u64(p.resource_permit_generation);
  u8(h, (uint8_t)p.live_mask);
  u8(h, (uint8_t)p.live_lane_count);
  h.u64(p.kv_capacity_bytes);
  h.u64(p.receipt.bank_epoch);
  h.u32((uint32_t)p.receipt.slot_index);
  h.u64(p.receipt.generation);
  h.u64(p.receipt.owner_key);
  const uint64_t *claim = &p.receipt.claim.capsule_bytes;
  for (int i = 0; i < 10; ++i) h.u64(claim[i]);
  h.u64(p.receipt.integrity);
  for (int l = 0; l < GLACIER_HIP_PUBLICATION_WIDTH; ++l) {
    const glacier_hip_lane_proposal_v1_t &lane = p.lanes[l];
    h.u32(lane.lane_index);
    h.u64(lane.step_index);
    h.u64(lane.prompt_len);
    h.u64(lane.kv_before);
    h.u64(lane.kv_after);
    h.u64(lane.kv_capacity_bytes);
    u8(h, lane.has_kv_transition ? 1 : 0);
    const glacier_hip_root_transition_v1_t &t = lane.kv_transition;
    h.u64(t.abi_version);
    h.u64(t.kv_row_txn_abi);
    h.u64(t.page_map_root_abi);
    h.u64(t.page_ref_abi);
    h.u64(t.cache_instance);
    h.u64(t.row_txn_generation);
    h.u64(t.root_before_generation);
    h.u64(t.root_after_generation);
    h.u64(t.root_before_len);
    h.u64(t.root_after_len);
    h.u64(t.root_before_pages);
    h.u64(t.root_after_pages);
    h.update(t.root_before_ownership_sha256, 32);
    h.update(t.root_after_ownership_sha256, 32);
    h.u64(t.logical_page);
    h.u64(t.page_ownership_generation);
    u8(h, t.installs_new_page ? 1 : 0);
    h.update(t.initial_logical_kv_sha256, 32);
    h.update(t.row_payload_sha256, 32);
    h.update(t.state_chain_before, 32);
    h.update(t.state_chain_after, 32);
    h.u64(lane.output_before);
    h.u64(lane.output_after);
    for (int i = 0; i < 4; ++i) h.u64(lane.rng_before[i]);
    for (int i = 0; i < 4; ++i) h.u64(lane.rng_after[i]);
    h.u64(lane.sampling_calls_before);
    h.u64(lane.sampling_calls_after);
    h.u32(lane.token_id);
    u8(h, lane.terminal ? 1 : 0);
  }
  h.final(out);
}

void commit_sha256(const uint8_t proposal_sha[32], const glacier_hip_prepare_ack_v1_t &ack,
                   uint8_t out[32]) {
  gh::Sha256 h;
  h.update("glacier-paged-token-txn-commit-v1", sizeof("glacier-paged-token-txn-commit-v1"));  // with its NUL
  h.u64(kCommitReceiptAbi);
  h.update(proposal_sha, 32);
  h.u64(ack.abi_version);
  h.update(ack.proposal_sha256, 32);
  h.u64(ack.sink_epoch);
  h.u64(ack.reservation_id);
  h.final(out);
}

void empty_transition(glacier_hip_root_transition_v1_t &t) {
  memset(&t, 0, sizeof t);
  t.abi_version = kPageTransitionAbi;
  t.kv_row_txn_abi = gpk::kRowTxnAbi;
  t.page_map_root_abi = gpk::kPageMapRootAbi;
  t.page_ref_abi = gpk::kPageRefAbi;
}

void empty_proposal(glacier_hip_token_proposal_v1_t &p) {
  memset(&p, 0, sizeof p);
  p.abi_version = kProposalAbi;
  p.resource_bank_abi = kResourceBankAbi;
  p.resource_publication_fence_abi = kPublicationFenceAbi;
  p.paged_kv_abi = gpk::kPagedKvAbi;
  p.page_map_root_abi = gpk::kPageMapRootAbi;
  p.page_ref_abi = gpk::kPageRefAbi;
  p.page_transition_abi = kPageTransitionAbi;
  p.kv_row_txn_abi = gpk::kRowTxnAbi;
  for (auto &l : p.lanes) empty_transition(l.kv_transition);
}

static void hash_claim(gh::Sha256 &h, const glacier_hip_claim_t &c) {
  const uint64_t *f = &c.capsule_bytes;
  for (int i = 0; i < 10; ++i) h.u64(f[i]);
}

static void hash_receipt(gh::Sha256 &h, const glacier_hip_bank_receipt_t &r) {
  h.u64(r.bank_epoch);
  h.u32((uint32_t)r.slot_index);
  h.u64(r.generation);
  h.u64(r.owner_key);
  hash_claim(h, r.claim);
  h.u64(r.integrity);
}

static void hash_transition(gh::Sha256 &h, const glacier_hip_root_transition_v1_t &t) {
  h.u64(t.abi_version);
  h.u64(t.kv_row_txn_abi);
  h.u64(t.page_map_root_abi);
  h.u64(t.page_ref_abi);
  h.u64(t.cache_instance);
  h.u64(t.row_txn_generation);
  h.u64(t.root_before_generation);
  h.u64(t.root_after_generation);
  h.u64(t.root_before_len);
  h.u64(t.root_after_len);
  h.u64(t.root_before_pages);
  h.u64(t.root_after_pages);
  h.update(t.root_before_ownership_sha256, 32);
  h.update(t.root_after_ownership_sha256, 32);
  h.u64(t.logical_page);
  h.u64(t.page_ownership_generation);
  u8(h, t.installs_new_page ? 1 : 0);
  h.update(t.initial_logical_kv_sha256, 32);
  h.update(t.row_payload_sha256, 32);
  h.update(t.state_chain_before, 32);
  h.update(t.state_chain_after, 32);
}

void proposal_v3_sha256(const glacier_hip_token_proposal_v3_t &p, uint8_t out[32]) {
  static const char d[] = "glacier-paged-lease-token-txn-proposal-v3";
  gh::Sha256 h;
  h.update(d, sizeof d);  // with its NUL
  h.u64(p.abi_version);
  h.u64(p.resource_bank_abi);
  h.u64(p.resource_lease_tree_abi);
  h.u64(p.resource_publication_fence_abi);
  h.u64(p.leased_paged_kv_abi);
  h.u64(p.paged_kv_abi);
  h.u64(p.page_transition_abi);
  h.u64(p.execution_abi);
  h.u64(p.request_epoch);
  h.u64(p.transaction_sequence);
  h.u64(p.resource_permit_generation);
  u8(h, (uint8_t)p.live_mask);
  u8(h, (uint8_t)p.live_lane_count);
  hash_receipt(h, p.parent_receipt);
  const glacier_hip_lease_tree_commitment_v3_t &t = p.tree;
  h.u64(t.abi_version);
  h.u64(t.tree_key);
  h.u64(t.identity_generation);
  h.u64(t.generation);
  h.u64(t.structural_revision);
  hash_claim(h, t.ceiling);
  hash_claim(h, t.current);
  h.u32(t.active_nodes);
  h.u64(t.state_digest);
  h.u64(t.token_integrity);
  for (int l = 0; l < GLACIER_HIP_PUBLICATION_WIDTH; ++l) {
    const glacier_hip_resource_commitment_v3_t &r = p.resources[l];
    h.u64(r.abi_version);
    h.u32(r.lane_index);
    u8(h, (uint8_t)r.lifecycle);
    h.u64(r.coordinator_instance);
    h.u64(r.cache_instance);
    h.u32(r.scope_index);
    h.u64(r.scope_generation);
    hash_root(h, r.root);
    h.update(r.kv_state_chain_after, 32);
    u8(h, r.has_canonical_after ? 1 : 0);
    h.update(r.canonical_after_sha256, 32);
    u8(h, r.has_terminal_generation ? 1 : 0);
    h.u64(r.terminal_generation);
    u8(h, r.has_binding_summary ? 1 : 0);
    h.u32(r.binding_summary.count);
    h.u64(r.binding_summary.payload_bytes);
    h.update(r.binding_summary.digest, 32);
    h.u64(r.allocation_set.abi_version);
    h.u32(r.allocation_set.count);
    h.u64(r.allocation_set.payload_bytes);
    h.update(r.allocation_set.sha256, 32);
  }
  for (int l = 0; l < GLACIER_HIP_PUBLICATION_WIDTH; ++l) {
    const glacier_hip_lane_proposal_v3_t &lane = p.lanes[l];
    h.u32(lane.lane_index);
    h.u64(lane.step_index);
    h.u64(lane.prompt_len);
    h.u64(lane.kv_before);
    h.u64(lane.kv_after);
    u8(h, lane.has_kv_transition ? 1 : 0);
    hash_transition(h, lane.kv_transition);
    h.u64(lane.output_before);
    h.u64(lane.output_after);
    h.update(lane.output_sha256, 32);
    for (int i = 0; i < 4; ++i) h.u64(lane.rng_before[i]);
    for (int i = 0; i < 4; ++i) h.u64(lane.rng_after[i]);
    h.u64(lane.sampling_calls_before);
    h.u64(lane.sampling_calls_after);
    h.u32(lane.token_id);
    u8(h, (uint8_t)lane.terminal_reason);
  }
  h.final(out);
}

void commit_v3_sha256(const uint8_t proposal_sha[32], const glacier_hip_prepare_ack_v1_t &ack,
                      uint8_t out[32]) {
  static const char d[] = "glacier-paged-lease-token-txn-commit-v3";
  gh::Sha256 h;
  h.update(d, sizeof d);  // with its NUL
  h.u64(kCommitReceiptV3Abi);
  h.update(proposal_sha, 32);
  h.u64(ack.abi_version);
  h.update(ack.proposal_sha256, 32);
  h.u64(ack.sink_epoch);
  h.u64(ack.reservation_id);
  h.final(out);
}

}  // namespace gpub

extern "C" {

int glacier_hip_token_proposal_sha256(const glacier_hip_token_proposal_v1_t *proposal,
                                      uint8_t out[32]) {
  if (!proposal || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  gpub::proposal_sha256(*proposal, out);
  return GLACIER_HIP_OK;
}

int glacier_hip_token_commit_sha256(const uint8_t proposal_sha256[32],
                                    const glacier_hip_prepare_ack_v1_t *ack, uint8_t out[32]) {
  if (!proposal_sha256 || !ack || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  gpub::commit_sha256(proposal_sha256, *ack, out);
  return GLACIER_HIP_OK;
}

int glacier_hip_token_proposal_v3_sha256(const glacier_hip_token_proposal_v3_t *proposal,
                                         uint8_t out[32]) {
  if (!proposal || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  gpub::proposal_v3_sha256(*proposal, out);
  return GLACIER_HIP_OK;
}

int glacier_hip_token_commit_v3_sha256(const uint8_t proposal_sha256[32],
                                       const glacier_hip_prepare_ack_v1_t *ack, uint8_t out[32]) {
  if (!proposal_sha256 || !ack || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  gpub::commit_v3_sha256(proposal_sha256, *ack, out);
  return GLACIER_HIP_OK;
}

int glacier_hip_token_sequence_sha256(const uint32_t *tokens, uint64_t count, uint8_t out[32]) {
  if (!out || (count && !tokens)) return GLACIER_HIP_INVALID_ARGUMENT;
  gh::token_sequence_sha256(tokens, (size_t)count, out);
  return GLACIER_HIP_OK;
}

}  // extern "C"
