// publication.h — the per-token publication transaction's digests
// (src/paged_token_txn.zig) over the C-ABI proposal records.
#pragma once
#include <stdint.h>

#include "../../include/glacier_hip.h"
#include "paged_kv.h"

namespace gpub {

constexpr uint64_t kProposalAbi = 0x4750545800000001ull;        // paged_token_txn.zig:18
constexpr uint64_t kSinkAbi = 0x4750545300000001ull;            // :19
constexpr uint64_t kPrepareAckAbi = 0x4750544100000001ull;      // :20
constexpr uint64_t kCommitReceiptAbi = 0x4750544300000001ull;   // :21
constexpr uint64_t kPageTransitionAbi = 0x4750545200000001ull;  // :22
constexpr uint64_t kResourceBankAbi = 0x4752424B00000001ull;    // resource_bank.zig:12
constexpr uint64_t kPublicationFenceAbi = 0x4752505500000001ull;  // resource_bank.zig:14

void initial_state_chain(const uint8_t logical_kv_sha256[32], const glacier_hip_page_map_root_t &root,
                         uint8_t out[32]);
void appended_state_chain(const uint8_t chain_before[32], const glacier_hip_page_map_root_t &before,
                          const glacier_hip_page_map_root_t &after,
                          const glacier_hip_row_txn_mark_t &mark, const uint8_t row_payload_sha256[32],
                          uint8_t out[32]);
void proposal_sha256(const glacier_hip_token_proposal_v1_t &p, uint8_t out[32]);
void commit_sha256(const uint8_t proposal_sha[32], const glacier_hip_prepare_ack_v1_t &ack,
                   uint8_t out[32]);
// A lane slot / proposal with only its ABI fields set (the reference's
// default-initialised RootTransitionV1 / ProposalV1).
void empty_transition(glacier_hip_root_transition_v1_t &t);
void empty_proposal(glacier_hip_token_proposal_v1_t &p);

// paged_lease_token_txn.zig (ProposalV3): ABIs, the v3 KV state chain
// (initialStateChain :533-543, appendedStateChain :545-564) and the v3
// proposal / commit digests (:1013-1098).
constexpr uint64_t kProposalV3Abi = 0x47504C5800000004ull;         // paged_lease_token_txn.zig:16
constexpr uint64_t kPrepareAckV3Abi = 0x47504C4100000003ull;       // :18
constexpr uint64_t kCommitReceiptV3Abi = 0x47504C4300000004ull;    // :19
constexpr uint64_t kPageTransitionV3Abi = 0x47504C5200000003ull;   // :20
constexpr uint64_t kResourceCommitmentAbi = 0x47504C4300000005ull; // :21
constexpr uint64_t kTreeCommitmentAbi = 0x47504C5400000003ull;     // :22
constexpr uint64_t kLeaseTreeAbi = 0x47524C5400000001ull;          // resource_bank.zig:27
constexpr uint64_t kLeasedPagedKvAbi = 0x47504C4300000002ull;      // leased_paged_kv_cache.zig:24
constexpr uint64_t kAllocationSetAbi = 0x47504C4100000002ull;      // leased_paged_kv_cache.zig:29
void initial_state_chain_v3(const uint8_t logical_kv_sha256[32],
                            const glacier_hip_page_map_root_t &root, uint8_t out[32]);
void appended_state_chain_v3(const uint8_t chain_before[32], const glacier_hip_page_map_root_t &before,
                             const glacier_hip_page_map_root_t &after,
                             const glacier_hip_row_txn_mark_t &mark,
                             const uint8_t row_payload_sha256[32], uint8_t out[32]);
void proposal_v3_sha256(const glacier_hip_token_proposal_v3_t &p, uint8_t out[32]);
void commit_v3_sha256(const uint8_t proposal_sha[32], const glacier_hip_prepare_ack_v1_t &ack,
                      uint8_t out[32]);

}  // namespace gpub
