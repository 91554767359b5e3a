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

}  // namespace gpub
