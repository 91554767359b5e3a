"""Restatement of the per-token publication digests of the reference.

TEST INFRASTRUCTURE ONLY: the checker for the product's staged publication
(glacier_hip_session_step_prepare / _commit, csrc/publication.cpp). Only
tests/ use it.

Follows /root/reference/src/paged_token_txn.zig:
  hashRoot             :762-772
  initialStateChain    :774-786
  appendedStateChain   :788-808
  proposalSha256       :1064-1130  (ProposalV1 :110-131, LaneProposalV1 :91-108,
                                    RootTransitionV1 :61-89; u8 fields live_mask,
                                    live_lane_count, bools as one byte)
  commitSha256         :1132-1148
and src/paged_kv_cache.zig logicalRowTxnSha256 :1366-1384 (row payload digest);
the leased v3 wave (src/paged_lease_token_txn.zig):
  initialStateChain    :532-543  (v3 domain)
  appendedStateChain   :545-564  (v3 domain)
  proposalSha256       :1013-1082 (ProposalV3 :162-180, ResourceCommitmentV3
                                   :141-160, LeaseTreeCommitmentV3 :127-139,
                                   LaneProposalV3 :107-124; lifecycle and
                                   terminal reason as one byte, the reason as
                                   0 or 1 + TerminalReason)
  commitSha256         :1084-1096
and src/leased_paged_kv_cache.zig allocationSetCommitmentForState :1253-1291
(with hashLeaseNode :1597-1616).
Integers little-endian, SHA-256 from hashlib. A record here is the ctypes
structure of the product's header read field by field, so the byte layout
this module hashes is written from the reference's field list, not from the
product's code.
"""
import hashlib
import struct

PAGE_MAP_ROOT_ABI = 0x47504D5200000001
PAGE_REF_ABI = 0x4750524600000001


def _u64(v):
    return struct.pack("<Q", v)


def _u32(v):
    return struct.pack("<I", v)


def _u8(v):
    return struct.pack("<B", v)


def root_bytes(generation, committed_len, committed_pages, ownership, cache_instance):
    """hashRoot: abi, instance, generation, len, pages, ownership digest."""
    return (_u64(PAGE_MAP_ROOT_ABI) + _u64(cache_instance) + _u64(generation) +
            _u64(committed_len) + _u64(committed_pages) + bytes(ownership))


def initial_state_chain_preimage(logical_kv_sha256, root):
    return b"glacier-paged-token-kv-chain-seed-v1\x00" + bytes(logical_kv_sha256) + root


def initial_state_chain(logical_kv_sha256, root):
    return hashlib.sha256(initial_state_chain_preimage(logical_kv_sha256, root)).digest()


def appended_state_chain_preimage(chain_before, root_before, root_after, cache_instance,
                                  logical_page, ownership_generation, row_txn_generation,
                                  row_payload_sha256):
    return (b"glacier-paged-token-kv-chain-append-v1\x00" + bytes(chain_before) + root_before +
            root_after + _u64(PAGE_REF_ABI) + _u64(cache_instance) + _u64(logical_page) +
            _u64(ownership_generation) + _u64(row_txn_generation) + bytes(row_payload_sha256))


def appended_state_chain(*args):
    return hashlib.sha256(appended_state_chain_preimage(*args)).digest()


def row_payload_sha256(num_layers, dim, base_len, rows_f32):
    """logicalRowTxnSha256: rows_f32 = [K_0, V_0, K_1, V_1, ...] f32 rows."""
    h = hashlib.sha256(b"glacier-paged-kv-row-v1\x00" + _u64(num_layers) + _u64(dim) +
                       _u64(base_len))
    for r in rows_f32:
        h.update(bytes(memoryview(r.astype("<f4")).cast("B")))
    return h.digest()


_PROPOSAL_HEAD = ("abi_version", "resource_bank_abi", "resource_publication_fence_abi",
                  "paged_kv_abi", "page_map_root_abi", "page_ref_abi", "page_transition_abi",
                  "kv_row_txn_abi", "execution_abi", "request_epoch", "transaction_sequence",
                  "resource_permit_generation")
_CLAIM = ("capsule_bytes", "kv_bytes", "activation_bytes", "partial_bytes", "logits_bytes",
          "output_journal_bytes", "staging_bytes", "device_bytes", "io_bytes", "queue_slots")
_TRANSITION_U64 = ("abi_version", "kv_row_txn_abi", "page_map_root_abi", "page_ref_abi",
                   "cache_instance", "row_txn_generation", "root_before_generation",
                   "root_after_generation", "root_before_len", "root_after_len",
                   "root_before_pages", "root_after_pages")


def proposal_preimage(p):
    """The bytes proposalSha256 hashes for a ProposalV1 record (any object with the fields)."""
    b = bytearray(b"glacier-paged-token-txn-proposal-v1\x00")
    for f in _PROPOSAL_HEAD:
        b += _u64(getattr(p, f))
    b += _u8(p.live_mask) + _u8(p.live_lane_count) + _u64(p.kv_capacity_bytes)
    r = p.receipt
    b += _u64(r.bank_epoch) + _u32(r.slot_index) + _u64(r.generation) + _u64(r.owner_key)
    for f in _CLAIM:
        b += _u64(getattr(r.claim, f))
    b += _u64(r.integrity)
    for lane in p.lanes:
        b += _u32(lane.lane_index)
        for f in ("step_index", "prompt_len", "kv_before", "kv_after", "kv_capacity_bytes"):
            b += _u64(getattr(lane, f))
        b += _u8(1 if lane.has_kv_transition else 0)
        t = lane.kv_transition
        for f in _TRANSITION_U64:
            b += _u64(getattr(t, f))
        b += bytes(t.root_before_ownership_sha256) + bytes(t.root_after_ownership_sha256)
        b += _u64(t.logical_page) + _u64(t.page_ownership_generation)
        b += _u8(1 if t.installs_new_page else 0)
        b += (bytes(t.initial_logical_kv_sha256) + bytes(t.row_payload_sha256) +
              bytes(t.state_chain_before) + bytes(t.state_chain_after))
        b += _u64(lane.output_before) + _u64(lane.output_after)
        for w in lane.rng_before:
            b += _u64(w)
        for w in lane.rng_after:
            b += _u64(w)
        b += _u64(lane.sampling_calls_before) + _u64(lane.sampling_calls_after)
        b += _u32(lane.token_id) + _u8(1 if lane.terminal else 0)
    return bytes(b)


def proposal_sha256(p):
    return hashlib.sha256(proposal_preimage(p)).digest()


COMMIT_RECEIPT_ABI = 0x4750544300000001


def commit_preimage(proposal_sha, ack_abi, ack_proposal_sha, sink_epoch, reservation_id):
    return (b"glacier-paged-token-txn-commit-v1\x00" + _u64(COMMIT_RECEIPT_ABI) +
            bytes(proposal_sha) + _u64(ack_abi) + bytes(ack_proposal_sha) + _u64(sink_epoch) +
            _u64(reservation_id))


def commit_sha256(*args):
    return hashlib.sha256(commit_preimage(*args)).digest()


# ---- leased v3 waves (paged_lease_token_txn.zig) ----
PROPOSAL_V3_ABI = 0x47504C5800000004
COMMIT_RECEIPT_V3_ABI = 0x47504C4300000004
PREPARE_ACK_V3_ABI = 0x47504C4100000003
PAGE_TRANSITION_V3_ABI = 0x47504C5200000003
RESOURCE_COMMITMENT_ABI = 0x47504C4300000005
TREE_COMMITMENT_ABI = 0x47504C5400000003
ALLOCATION_SET_ABI = 0x47504C4100000002
LEASED_PAGED_KV_ABI = 0x47504C4300000002
LEASE_TREE_ABI = 0x47524C5400000001


def initial_state_chain_v3(logical_kv_sha256, root):
    return hashlib.sha256(b"glacier-paged-lease-token-kv-chain-seed-v3\x00" +
                          bytes(logical_kv_sha256) + root).digest()


def appended_state_chain_v3(chain_before, root_before, root_after, cache_instance, logical_page,
                            ownership_generation, row_txn_generation, row_payload_sha256):
    return hashlib.sha256(
        b"glacier-paged-lease-token-kv-chain-append-v3\x00" + bytes(chain_before) + root_before +
        root_after + _u64(PAGE_REF_ABI) + _u64(cache_instance) + _u64(logical_page) +
        _u64(ownership_generation) + _u64(row_txn_generation) +
        bytes(row_payload_sha256)).digest()


def _claim(c):
    return b"".join(_u64(getattr(c, f)) for f in _CLAIM)


def _receipt(r):
    return (_u64(r.bank_epoch) + _u32(r.slot_index) + _u64(r.generation) + _u64(r.owner_key) +
            _claim(r.claim) + _u64(r.integrity))


def _root(r):
    return (_u64(r.abi_version) + _u64(r.cache_instance) + _u64(r.generation) +
            _u64(r.committed_len) + _u64(r.committed_pages) + bytes(r.ownership_sha256))


def lease_node_bytes(n):
    """hashLeaseNode: the node's ABI, parent receipt, tree identity, index,
    generation, parent link, keys, kind byte, ceiling, claim and integrity."""
    return (_u64(n.abi_version) + _receipt(n.parent) + _u64(n.tree_key) +
            _u64(n.tree_identity_generation) + _u32(n.node_index) + _u64(n.generation) +
            _u32(n.parent_index) + _u64(n.parent_generation) + _u64(n.node_key) +
            _u64(n.tenant_key) + _u64(n.binding_key) + _u8(n.kind) + _claim(n.ceiling) +
            _claim(n.claim) + _u64(n.integrity))


def allocation_set_preimage(instance, cache_instance, scope, bindings):
    """allocationSetCommitmentForState's hashed bytes: the coordinator and
    cache instances, the sidecar's length and scope node, then each non-free
    binding (its index and fields, the state as one byte) with its leaf."""
    b = bytearray(b"glacier-paged-lease-allocation-set-v2\x00")
    b += _u64(ALLOCATION_SET_ABI) + _u64(instance) + _u64(cache_instance) + _u64(len(bindings))
    b += lease_node_bytes(scope)
    for i, x in enumerate(bindings):
        if x.state == 0:  # BindingState.free
            continue
        b += (_u64(i) + _u64(x.abi_version) + _u8(x.state) + _u64(x.cache_instance) +
              _u64(x.logical_page) + _u64(x.payload_bytes) + _u32(x.scope_index) +
              _u64(x.scope_generation) + _u64(x.integrity) + lease_node_bytes(x.leaf))
    return bytes(b)


def allocation_set_sha256(*args):
    return hashlib.sha256(allocation_set_preimage(*args)).digest()


_PROPOSAL_V3_HEAD = ("abi_version", "resource_bank_abi", "resource_lease_tree_abi",
                     "resource_publication_fence_abi", "leased_paged_kv_abi", "paged_kv_abi",
                     "page_transition_abi", "execution_abi", "request_epoch",
                     "transaction_sequence", "resource_permit_generation")


def _transition(t):
    b = bytearray()
    for f in _TRANSITION_U64:
        b += _u64(getattr(t, f))
    b += bytes(t.root_before_ownership_sha256) + bytes(t.root_after_ownership_sha256)
    b += _u64(t.logical_page) + _u64(t.page_ownership_generation)
    b += _u8(1 if t.installs_new_page else 0)
    b += (bytes(t.initial_logical_kv_sha256) + bytes(t.row_payload_sha256) +
          bytes(t.state_chain_before) + bytes(t.state_chain_after))
    return bytes(b)


def proposal_v3_preimage(p):
    """The bytes proposalSha256 (v3) hashes for a ProposalV3 record."""
    b = bytearray(b"glacier-paged-lease-token-txn-proposal-v3\x00")
    for f in _PROPOSAL_V3_HEAD:
        b += _u64(getattr(p, f))
    b += _u8(p.live_mask) + _u8(p.live_lane_count) + _receipt(p.parent_receipt)
    t = p.tree
    b += (_u64(t.abi_version) + _u64(t.tree_key) + _u64(t.identity_generation) +
          _u64(t.generation) + _u64(t.structural_revision) + _claim(t.ceiling) +
          _claim(t.current) + _u32(t.active_nodes) + _u64(t.state_digest) +
          _u64(t.token_integrity))
    for r in p.resources:
        b += (_u64(r.abi_version) + _u32(r.lane_index) + _u8(r.lifecycle) +
              _u64(r.coordinator_instance) + _u64(r.cache_instance) + _u32(r.scope_index) +
              _u64(r.scope_generation) + _root(r.root) + bytes(r.kv_state_chain_after) +
              _u8(1 if r.has_canonical_after else 0) + bytes(r.canonical_after_sha256) +
              _u8(1 if r.has_terminal_generation else 0) + _u64(r.terminal_generation) +
              _u8(1 if r.has_binding_summary else 0))
        s = r.binding_summary
        b += _u32(s.count) + _u64(s.payload_bytes) + bytes(s.digest)
        a = r.allocation_set
        b += _u64(a.abi_version) + _u32(a.count) + _u64(a.payload_bytes) + bytes(a.sha256)
    for lane in p.lanes:
        b += _u32(lane.lane_index)
        for f in ("step_index", "prompt_len", "kv_before", "kv_after"):
            b += _u64(getattr(lane, f))
        b += _u8(1 if lane.has_kv_transition else 0) + _transition(lane.kv_transition)
        b += _u64(lane.output_before) + _u64(lane.output_after) + bytes(lane.output_sha256)
        for w in lane.rng_before:
            b += _u64(w)
        for w in lane.rng_after:
            b += _u64(w)
        b += _u64(lane.sampling_calls_before) + _u64(lane.sampling_calls_after)
        b += _u32(lane.token_id) + _u8(lane.terminal_reason)
    return bytes(b)


def proposal_v3_sha256(p):
    return hashlib.sha256(proposal_v3_preimage(p)).digest()


def commit_v3_preimage(proposal_sha, ack_abi, ack_proposal_sha, sink_epoch, reservation_id):
    return (b"glacier-paged-lease-token-txn-commit-v3\x00" + _u64(COMMIT_RECEIPT_V3_ABI) +
            bytes(proposal_sha) + _u64(ack_abi) + bytes(ack_proposal_sha) + _u64(sink_epoch) +
            _u64(reservation_id))


def commit_v3_sha256(*args):
    return hashlib.sha256(commit_v3_preimage(*args)).digest()
