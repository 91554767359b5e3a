"""Pins of the leased v3 wave digests (paged_lease_token_txn.zig) and of the
leased coordinator's allocation-set commitment
(leased_paged_kv_cache.zig:1253-1291), none of which the reference holds a
vector or a runnable restatement for.

As for the v1 digests (tests/test_publication_pins.py), following the
reference's own digest test ("proposal digest binds binding summary and
terminal generation", paged_lease_token_txn.zig:1927-1955): every field the
reference hashes moves the digest, the preimage length equals the byte count
of the reference's field list (ProposalV3 :162-180, ResourceCommitmentV3
:141-160, LeaseTreeCommitmentV3 :127-139, LaneProposalV3 :107-124,
RootTransitionV3 :83-105, AllocationSetCommitmentV2 and BindingSummaryV1
leased_paged_kv_cache.zig:74-90, LeaseNodeV1 resource_bank.zig), integers
hash at the reference's width, bools and enums as one byte. The product's
host functions must equal the oracle on random records, and a host leased
coordinator's allocation set must equal the oracle's restatement over the
coordinator's own binding sidecar and scope node.
"""
import ctypes as C
import hashlib
import random

import pytest

from oracle import publication as opub
from test_publication_pins import _leaves

U64, U32, U8, DIGEST = 8, 4, 1, 32
CLAIM = 10 * U64
RECEIPT = U64 + U32 + U64 + U64 + CLAIM + U64
ROOT = 5 * U64 + DIGEST
TRANSITION = 12 * U64 + 2 * DIGEST + 2 * U64 + U8 + 4 * DIGEST
TREE = 5 * U64 + 2 * CLAIM + U32 + 2 * U64
SUMMARY = U32 + U64 + DIGEST
ALLOC = U64 + U32 + U64 + DIGEST
RESOURCE = (U64 + U32 + U8 + 2 * U64 + U32 + U64 + ROOT + DIGEST + U8 + DIGEST + U8 + U64 + U8 +
            SUMMARY + ALLOC)
LANE = U32 + 4 * U64 + U8 + TRANSITION + 2 * U64 + DIGEST + 8 * U64 + 2 * U64 + U32 + U8
WIDTH = 4
PROPOSAL = (len(b"glacier-paged-lease-token-txn-proposal-v3\x00") + 11 * U64 + 2 * U8 + RECEIPT +
            TREE + WIDTH * RESOURCE + WIDTH * LANE)
COMMIT = len(b"glacier-paged-lease-token-txn-commit-v3\x00") + U64 + DIGEST + U64 + DIGEST + 2 * U64
NODE = U64 + RECEIPT + 2 * U64 + U32 + U64 + U32 + 4 * U64 + U8 + 2 * CLAIM + U64  # hashLeaseNode
BINDING = 2 * U64 + U8 + 3 * U64 + U32 + 2 * U64 + NODE  # one non-free binding + its leaf

BOOLS = {"has_kv_transition", "installs_new_page", "has_canonical_after",
         "has_terminal_generation", "has_binding_summary"}
REF_BITS = {"slot_index": 32, "lane_index": 32, "token_id": 32, "live_mask": 8,
            "live_lane_count": 8, "lifecycle": 8, "terminal_reason": 8, "active_nodes": 32,
            "scope_index": 32, "count": 32}


def _bits(obj, name):
    return REF_BITS.get(name, 8 * C.sizeof(dict(type(obj)._fields_)[name]))


def _random_proposal(gh, rng):
    p = gh.TokenProposalV3()
    for _, obj, name, kind in _leaves(p):
        if kind == "digest":
            getattr(obj, name)[:] = list(rng.randbytes(32))
        elif kind == "array":
            arr = getattr(obj, name)
            for i in range(len(arr)):
                arr[i] = rng.getrandbits(64)
        elif name in BOOLS:
            setattr(obj, name, rng.getrandbits(1))
        else:
            setattr(obj, name, rng.getrandbits(_bits(obj, name)))
    return p


def _owner(p, path):
    o = p
    for part in path.split(".")[:-1]:
        if "[" in part:
            n, i = part[:-1].split("[")
            o = getattr(o, n)[int(i)]
        else:
            o = getattr(o, part)
    return o


def test_v3_preimage_lengths_match_the_reference_field_lists(gh):
    p = _random_proposal(gh, random.Random(1))
    assert len(opub.proposal_v3_preimage(p)) == PROPOSAL == 3504
    sha = opub.proposal_v3_sha256(p)
    assert len(opub.commit_v3_preimage(sha, 1, sha, 2, 3)) == COMMIT
    node = gh.LeaseNode()
    assert len(opub.lease_node_bytes(node)) == NODE
    b = (gh.PageLeaseBinding * 3)()
    b[1].state = 1
    head = len(b"glacier-paged-lease-allocation-set-v2\x00") + 4 * U64 + NODE
    assert len(opub.allocation_set_preimage(7, 8, node, b)) == head + BINDING
    b[2].state = 1
    assert len(opub.allocation_set_preimage(7, 8, node, b)) == head + 2 * BINDING


@pytest.mark.parametrize("seed", [2, 3])
def test_every_v3_proposal_field_moves_the_digest(gh, seed):
    p = _random_proposal(gh, random.Random(seed))
    base = opub.proposal_v3_sha256(p)
    seen = 0
    for path, _, name, kind in list(_leaves(p)):
        q = gh.TokenProposalV3.from_buffer_copy(p)
        o = _owner(q, path)
        if kind == "digest":
            getattr(o, name)[31] ^= 0x80
        elif kind == "array":
            getattr(o, name)[3] ^= 1 << 63
        elif name in BOOLS:
            setattr(o, name, 1 - getattr(o, name))
        else:
            setattr(o, name, getattr(o, name) ^ (1 << (_bits(o, name) - 1)))
        assert opub.proposal_v3_sha256(q) != base, path
        seen += 1
    # head 11 + masks 2 + receipt 15 + tree 28; per resource 26 (7 identity
    # fields, 6 root fields, chain, 2 canonical, 2 terminal, has_summary,
    # 3 summary, 4 allocation set); per lane 36
    assert seen == 11 + 2 + 15 + 28 + WIDTH * 26 + WIDTH * 36


def test_v3_bools_and_enums_hash_as_one_byte(gh):
    p = _random_proposal(gh, random.Random(4))
    for r in p.resources:
        r.has_canonical_after = r.has_terminal_generation = r.has_binding_summary = 1
        r.lifecycle = 3
    for lane in p.lanes:
        lane.has_kv_transition = lane.kv_transition.installs_new_page = 1
        lane.terminal_reason = 2
    base = opub.proposal_v3_sha256(p)
    out = (C.c_uint8 * 32)()
    assert gh.lib().glacier_hip_token_proposal_v3_sha256(C.byref(p), out) == 0
    assert bytes(out) == base
    for r in p.resources:
        r.has_canonical_after = 2
        r.has_terminal_generation = 0x10
        r.has_binding_summary = 0xFF
    for lane in p.lanes:
        lane.has_kv_transition = 7
        lane.kv_transition.installs_new_page = 9
    assert opub.proposal_v3_sha256(p) == base
    assert gh.lib().glacier_hip_token_proposal_v3_sha256(C.byref(p), out) == 0
    assert bytes(out) == base
    p.lanes[0].terminal_reason = 0  # no reason hashes as 0, eos as 1
    assert opub.proposal_v3_sha256(p) != base


def test_v3_chain_domains_differ_from_v1():
    sha = hashlib.sha256(b"k").digest()
    root = opub.root_bytes(1, 2, 3, sha, 4)
    assert opub.initial_state_chain_v3(sha, root) != opub.initial_state_chain(sha, root)
    args = (sha, root, root, 1, 2, 3, 4, sha)
    assert opub.appended_state_chain_v3(*args) != opub.appended_state_chain(*args)
    for i in range(len(args)):
        a = list(args)
        a[i] = bytes([a[i][0] ^ 1]) + a[i][1:] if isinstance(a[i], bytes) else a[i] ^ (1 << 63)
        assert opub.appended_state_chain_v3(*a) != opub.appended_state_chain_v3(*args), i


@pytest.mark.parametrize("seed", range(5, 13))
def test_product_v3_digests_equal_the_oracle_on_random_records(gh, seed):
    rng = random.Random(seed)
    p = _random_proposal(gh, rng)
    out = (C.c_uint8 * 32)()
    assert gh.lib().glacier_hip_token_proposal_v3_sha256(C.byref(p), out) == 0
    sha = bytes(out)
    assert sha == opub.proposal_v3_sha256(p)
    ack = gh.PrepareAck(rng.getrandbits(64), (C.c_uint8 * 32)(*rng.randbytes(32)),
                        rng.getrandbits(64), rng.getrandbits(64))
    assert gh.lib().glacier_hip_token_commit_v3_sha256((C.c_uint8 * 32)(*sha), C.byref(ack),
                                                       out) == 0
    assert bytes(out) == opub.commit_v3_sha256(sha, ack.abi_version, bytes(ack.proposal_sha256),
                                               ack.sink_epoch, ack.reservation_id)
    assert bytes(out) != opub.commit_sha256(sha, ack.abi_version, bytes(ack.proposal_sha256),
                                            ack.sink_epoch, ack.reservation_id)


def test_host_coordinator_allocation_set_equals_the_oracle(gh):
    """A host leased coordinator (one 16-row page = 128 payload bytes) after
    0, 1 and 17 committed rows: its allocation set is the oracle's
    restatement over the coordinator's binding sidecar and scope node, its
    count and bytes are the binding summary's, and an edited live binding is
    refused as the summary refuses it."""
    bank = gh.LeaseBank(1, 8, 0x4C504341, kv_bytes=512, queue_slots=1)
    parent = bank.commit(bank.reserve(1, queue_slots=1))
    tree = bank.open_tree(parent, 0x74726565, 0x61757468, kv_bytes=512)
    scope = bank.open_scope(tree, 10, 100, kv_bytes=256)
    epoch, sid = 0x4C504342, 0x5E55_1001
    seq = C.c_uint64(0)
    bank.bind_session(tree, epoch, sid)
    pages = gh.KvPages(1, 1, 33, 8)
    lk = gh.LeasedKV(bank, tree, scope, pages, epoch, sid, seq)
    instance = lk.plan_next_row().coordinator_instance
    seen = set()
    for rows in (0, 1, 17):
        while pages.root().committed_len < rows:
            txn = lk.begin_row(lk.plan_next_row())
            lk.append_row(txn, 0, [1.0], [-1.0])
            lk.commit_row(txn)
        a = lk.allocation_set()
        s = lk.binding_summary()
        assert a.abi_version == opub.ALLOCATION_SET_ABI
        assert (a.count, a.payload_bytes) == (s.count, s.payload_bytes) == \
            ((rows + 15) // 16, 128 * ((rows + 15) // 16))
        want = opub.allocation_set_sha256(instance, pages.root().cache_instance, lk.scope,
                                          lk.bindings)
        assert bytes(a.sha256) == want
        seen.add(want)
    assert len(seen) == 3
    lk.bindings[0].payload_bytes += 1
    with pytest.raises(gh.LeaseError):
        lk.allocation_set()
    lk.bindings[0].payload_bytes -= 1
    assert bytes(lk.allocation_set().sha256) == want
