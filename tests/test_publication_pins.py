"""Pins of the per-token publication digests (paged_token_txn.zig) for which
the reference holds no vector and no runnable restatement: proposalSha256
(:1064-1130), commitSha256 (:1132-1148) and the KV state chain
(initialStateChain :774-786, appendedStateChain :788-808).

Following the reference's own digest tests ("proposal digest binds binding
summary and terminal generation", paged_lease_token_txn.zig:1927-1955), every
field the reference hashes must move the digest; in addition the preimage
length must equal the byte count of the reference's field list (ProposalV1
:110-131, LaneProposalV1 :91-108, RootTransitionV1 :61-89, Receipt and Claim
resource_bank.zig:61-71,506-513), each integer must be hashed at its full
width, and a bool must hash as its truth value (@intFromBool). A dropped,
duplicated or narrowed field fails one of these; the relative order of two
fields of equal width is the one property left unpinned. The product's host
functions (glacier_hip_token_proposal_sha256 / _commit_sha256) must equal the
oracle on random records.
"""
import ctypes as C
import hashlib
import random

import pytest

from oracle import publication as opub

U64, U32, U8, DIGEST = 8, 4, 1, 32
CLAIM_FIELDS = 10  # resource_bank.zig:61-71
RECEIPT = U64 + U32 + U64 + U64 + CLAIM_FIELDS * U64 + U64  # :506-513
TRANSITION = 12 * U64 + 2 * DIGEST + 2 * U64 + U8 + 4 * DIGEST  # :61-89
LANE = U32 + 5 * U64 + U8 + TRANSITION + 2 * U64 + 8 * U64 + 2 * U64 + U32 + U8  # :91-108
WIDTH = 4
PROPOSAL = (len(b"glacier-paged-token-txn-proposal-v1\x00") + 12 * U64 + 2 * U8 + U64 + RECEIPT +
            WIDTH * LANE)  # :110-131 hashed as :1064-1130
COMMIT = len(b"glacier-paged-token-txn-commit-v1\x00") + U64 + DIGEST + U64 + DIGEST + 2 * U64
ROOT = 5 * U64 + DIGEST  # hashRoot :762-772
CHAIN_SEED = len(b"glacier-paged-token-kv-chain-seed-v1\x00") + DIGEST + ROOT
CHAIN_APPEND = len(b"glacier-paged-token-kv-chain-append-v1\x00") + DIGEST + 2 * ROOT + 5 * U64 + \
    DIGEST

# ProposalV1 fields the reference declares as bool (hashed through @intFromBool)
BOOLS = {"has_kv_transition", "installs_new_page", "terminal"}
# fields the reference declares narrower than u64 (the C records widen some)
REF_BITS = {"slot_index": 32, "lane_index": 32, "token_id": 32, "live_mask": 8,
            "live_lane_count": 8}


def _bits(obj, name):
    return REF_BITS.get(name, 8 * C.sizeof(_ctype(obj, name)))


def _random_proposal(gh, rng):
    p = gh.TokenProposal()
    for path, obj, name, kind in _leaves(p):
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


def _ctype(obj, name):
    return dict(type(obj)._fields_)[name]


def _leaves(obj, path=""):
    """(path, owner, field, kind) for every field of a ctypes record, nested
    records and lane arrays expanded; `reserved` padding is not a field of
    the reference's records."""
    for name, t in type(obj)._fields_:
        if name.startswith("reserved"):
            continue
        val = getattr(obj, name)
        if isinstance(val, C.Structure):
            yield from _leaves(val, f"{path}{name}.")
        elif isinstance(val, C.Array) and isinstance(val[0], C.Structure):
            for i in range(len(val)):
                yield from _leaves(val[i], f"{path}{name}[{i}].")
        elif isinstance(val, C.Array):
            yield (path + name, obj, name, "digest" if t._type_ is C.c_uint8 else "array")
        else:
            yield (path + name, obj, name, "int")


def test_preimage_lengths_match_the_reference_field_lists(gh):
    rng = random.Random(1)
    p = _random_proposal(gh, rng)
    assert len(opub.proposal_preimage(p)) == PROPOSAL == 2062
    sha = opub.proposal_sha256(p)
    assert len(opub.commit_preimage(sha, 1, sha, 2, 3)) == COMMIT
    root = opub.root_bytes(1, 2, 3, bytes(32), 4)
    assert len(root) == ROOT
    assert len(opub.initial_state_chain_preimage(bytes(32), root)) == CHAIN_SEED
    assert len(opub.appended_state_chain_preimage(bytes(32), root, root, 1, 2, 3, 4,
                                                  bytes(32))) == CHAIN_APPEND


@pytest.mark.parametrize("seed", [2, 3])
def test_every_proposal_field_moves_the_digest(gh, seed):
    rng = random.Random(seed)
    p = _random_proposal(gh, rng)
    base = opub.proposal_sha256(p)
    seen = 0
    for path, obj, name, kind in list(_leaves(p)):
        q = gh.TokenProposal.from_buffer_copy(p)
        # the same field of the copy
        owner = q
        for part in path.split(".")[:-1]:
            if "[" in part:
                n, i = part[:-1].split("[")
                owner = getattr(owner, n)[int(i)]
            else:
                owner = getattr(owner, part)
        if kind == "digest":
            getattr(owner, name)[31] ^= 0x80
        elif kind == "array":
            getattr(owner, name)[3] ^= 1 << 63
        elif name in BOOLS:
            setattr(owner, name, 1 - getattr(owner, name))
        else:  # the top bit of the field's width in the reference
            setattr(owner, name, getattr(owner, name) ^ (1 << (_bits(owner, name) - 1)))
        assert opub.proposal_sha256(q) != base, path
        seen += 1
    # head, masks, capacity, receipt; per lane: index + 5 counters, has_kv_transition,
    # 21 transition fields, outputs, the two RNG states, sampler counters, token + terminal
    assert seen == 12 + 2 + 1 + (4 + CLAIM_FIELDS + 1) + WIDTH * (6 + 1 + 21 + 2 + 2 + 2 + 2)


def test_bools_hash_as_their_truth_value(gh):
    rng = random.Random(4)
    p = _random_proposal(gh, rng)
    for lane in p.lanes:
        lane.has_kv_transition = 1
        lane.terminal = 1
        lane.kv_transition.installs_new_page = 1
    base = opub.proposal_sha256(p)
    for lane in p.lanes:
        lane.has_kv_transition = 2
        lane.terminal = 5
        lane.kv_transition.installs_new_page = 0xFF
    assert opub.proposal_sha256(p) == base
    out = (C.c_uint8 * 32)()
    assert gh.lib().glacier_hip_token_proposal_sha256(C.byref(p), out) == 0
    assert bytes(out) == base


def test_commit_and_chain_arguments_each_move_the_digest():
    sha = hashlib.sha256(b"p").digest()
    args = [sha, 11, sha, 12, 13]
    base = opub.commit_sha256(*args)
    for i in range(len(args)):
        a = list(args)
        a[i] = bytes([a[i][0] ^ 1]) + a[i][1:] if isinstance(a[i], bytes) else a[i] ^ (1 << 63)
        assert opub.commit_sha256(*a) != base, i
    root = opub.root_bytes(5, 6, 7, sha, 8)
    for i in range(5):
        r = list((5, 6, 7, sha, 8))
        r[i] = bytes([r[i][0] ^ 1]) + r[i][1:] if isinstance(r[i], bytes) else r[i] ^ (1 << 63)
        assert opub.root_bytes(*r) != root
    chain = [sha, root, root, 1, 2, 3, 4, sha]
    base = opub.appended_state_chain(*chain)
    for i in range(len(chain)):
        a = list(chain)
        a[i] = bytes([a[i][0] ^ 1]) + a[i][1:] if isinstance(a[i], bytes) else a[i] ^ (1 << 63)
        assert opub.appended_state_chain(*a) != base, i
    assert opub.initial_state_chain(sha, root) != opub.initial_state_chain(bytes(32), root)


@pytest.mark.parametrize("seed", range(5, 15))
def test_product_digests_equal_the_oracle_on_random_records(gh, seed):
    rng = random.Random(seed)
    p = _random_proposal(gh, rng)
    out = (C.c_uint8 * 32)()
    assert gh.lib().glacier_hip_token_proposal_sha256(C.byref(p), out) == 0
    sha = bytes(out)
    assert sha == opub.proposal_sha256(p)
    ack = gh.PrepareAck(rng.getrandbits(64), (C.c_uint8 * 32)(*rng.randbytes(32)),
                        rng.getrandbits(64), rng.getrandbits(64))
    assert gh.lib().glacier_hip_token_commit_sha256((C.c_uint8 * 32)(*sha), C.byref(ack), out) == 0
    assert bytes(out) == opub.commit_sha256(sha, ack.abi_version, bytes(ack.proposal_sha256),
                                            ack.sink_epoch, ack.reservation_id)
