"""Paged-KV row transaction: the oracle (oracle/paged_kv.py) and the product's
host page map (glacier_hip_kv_pages_*, csrc/paged_kv.cpp) against the
reference's own tests in /root/reference/src/paged_kv_cache.zig, then against
each other on a seeded trace of begin / commit / abort / reset.

The KATs are restated from the reference tests cited on each function; the
trace uses the reference's LCG from its 10k-transition test (:2351-2400).
No GPU is needed: the page map is host state."""
import hashlib
import struct

import pytest

from oracle import paged_kv as opk


# ---------------------------------------------------------------------------------
# an adapter so the same KAT bodies run on the oracle and on the product
# ---------------------------------------------------------------------------------
class OracleCache:
    def __init__(self, layers, dim, max_seq):
        self.c = opk.PagedKVCache(layers, dim, max_seq)

    def begin(self):
        return self.c.begin_row()

    def commit(self, m):
        self.c.commit_row(m)

    def abort(self, m):
        self.c.abort_row(m)

    def reset(self):
        self.c.reset()

    def root(self):
        return self.c.root().key()

    def payload(self, page):
        return self.c.payload[page]

    def gen(self, m):
        return m.ownership_generation

    def row_gen(self, m):
        return m.generation

    def ref_ok(self, page, gen):
        try:
            self.c.validate_committed_page_ref(self.c.instance_id, page, gen)
            return True
        except opk.PagedError:
            return False

    def ledger(self):
        return self.c.resident_ledger()

    @property
    def len(self):
        return self.c.len

    def expect_error(self, fn, name):
        with pytest.raises(opk.PagedError) as e:
            fn()
        assert str(e.value) == name


class ProductCache:
    def __init__(self, gh, layers, dim, max_seq):
        self.gh = gh
        self.p = gh.KvPages(layers, dim, max_seq, pool_pages=-(-max_seq // 16))

    def begin(self):
        rc, m = self.p.begin_row()
        if rc:
            raise RuntimeError(rc)
        return m

    def commit(self, m):
        assert self.p.commit_row(m) == 0

    def abort(self, m):
        assert self.p.abort_row(m) == 0

    def reset(self):
        assert self.p.reset() == 0

    def root(self):
        r = self.p.root()
        return (r.abi_version, r.cache_instance, r.generation, r.committed_len,
                r.committed_pages, bytes(r.ownership_sha256))

    def payload(self, page):
        p, _ = self.p.page(page)
        return None if p < 0 else p

    def gen(self, m):
        return m.page_ref.ownership_generation

    def row_gen(self, m):
        return m.generation

    def ref_ok(self, page, gen):
        ref = self.gh.PageRef(0x4750524600000001, self.p.root().cache_instance, page, gen)
        return self.p.validate_page_ref(ref) == 0

    def ledger(self):
        return self.p.ledger()

    @property
    def len(self):
        return self.p.root().committed_len

    def expect_error(self, fn, name):
        codes = {"InvalidTransaction": self.gh.INVALID_TRANSACTION,
                 "TransactionActive": self.gh.TRANSACTION_ACTIVE,
                 "CacheFull": self.gh.CACHE_FULL}
        with pytest.raises(RuntimeError) as e:
            fn()
        assert e.value.args[0] == codes[name]


@pytest.fixture(params=["oracle", "product"])
def make_cache(request, gh):
    if request.param == "oracle":
        return OracleCache
    return lambda *a: ProductCache(gh, *a)


# ---------------------------------------------------------------------------------
# reference KATs (paged_kv_cache.zig tests)
# ---------------------------------------------------------------------------------
def test_boundary_abort_reuses_payload_with_fresh_ownership_and_rejects_aba(make_cache):
    """paged_kv_cache.zig:1946-1985."""
    c = make_cache(1, 2, 2)
    root_before = c.root()
    first = c.begin()
    payload = c.payload(0)
    c.abort(first)
    assert c.root() == root_before and c.len == 0
    led = c.ledger()
    assert (led["allocated_pages"], led["reusable_pages"]) == (1, 1)
    if isinstance(c, OracleCache):
        c.expect_error(lambda: c.abort(first), "InvalidTransaction")
    else:
        assert c.p.abort_row(first) == c.gh.INVALID_TRANSACTION
    assert not c.ref_ok(0, c.gen(first))
    retry = c.begin()
    assert c.payload(0) == payload                  # same payload
    assert c.gen(retry) != c.gen(first)              # fresh ownership: no ABA
    if isinstance(c, OracleCache):
        c.expect_error(lambda: c.commit(first), "InvalidTransaction")
    else:
        assert c.p.commit_row(first) == c.gh.INVALID_TRANSACTION
    c.commit(retry)
    assert c.ref_ok(0, c.gen(retry))
    assert not c.ref_ok(0, c.gen(first))
    assert c.ledger()["reusable_pages"] == 0


def test_reset_invalidates_roots_and_page_refs_keeping_payloads(make_cache):
    """paged_kv_cache.zig:1987-2014."""
    c = make_cache(1, 1, 17)
    for _ in range(17):
        c.commit(c.begin())
    old_root = c.root()
    # the page ref of logical page 0 is (instance, 0, generation 1)
    before = c.ledger()
    c.reset()
    assert c.len == 0 and c.root() != old_root
    assert not c.ref_ok(0, 1)
    after = c.ledger()
    assert before["allocated_pages"] == after["allocated_pages"] == after["reusable_pages"]
    assert before["resident_allocation_bytes"] == after["resident_allocation_bytes"]
    m0 = c.begin()
    assert c.gen(m0) != 1
    c.commit(m0)


def test_commit_keeps_prepare_private_and_rejects_second_begin(make_cache):
    """paged_kv_cache.zig:1913-1944 (the page-map half: a second begin while a
    row is staged is TransactionActive; the root changes only at commit)."""
    c = make_cache(2, 2, 4)
    root_before = c.root()
    m = c.begin()
    c.expect_error(c.begin, "TransactionActive")
    assert c.root() == root_before and c.len == 0
    c.commit(m)
    assert c.len == 1 and c.root() != root_before


def test_cache_full_at_max_seq(make_cache):
    c = make_cache(1, 1, 3)
    for _ in range(3):
        c.commit(c.begin())
    c.expect_error(c.begin, "CacheFull")


def _ten_thousand_transitions(c):
    """paged_kv_cache.zig:2351-2400: the reference's LCG picks abort (state & 3
    == 0) or commit; a full cache is reset."""
    state = 0x123456789ABCDEF0
    committed = 0
    M64 = (1 << 64) - 1
    trace = []
    for _ in range(10_000):
        if committed == 64:
            stale = c.root()
            c.reset()
            assert c.root() != stale
            committed = 0
        root_before = c.root()
        m = c.begin()
        state = (state * 6364136223846793005 + 1442695040888963407) & M64
        if state & 3 == 0:
            c.abort(m)
            assert c.root() == root_before and c.len == committed
        else:
            assert c.root() == root_before
            c.commit(m)
            committed += 1
            assert c.len == committed and c.root()[3] == committed  # committed_len
        led = c.ledger()
        assert led["committed_pages"] == c.len // 16 + (1 if c.len % 16 else 0)
        trace.append((c.root(), c.gen(m), c.row_gen(m)))
    return trace


def test_ten_thousand_commit_abort_reset_transitions(make_cache):
    c = make_cache(2, 3, 64)
    _ten_thousand_transitions(c)


def test_product_page_map_equals_oracle_on_the_reference_trace(gh):
    """Every root (generation, length, pages, ownership chain), page ownership
    generation and row generation of the product equals the oracle's over the
    10k-transition trace (same cache instance for both)."""
    prod = ProductCache(gh, 2, 3, 64)
    inst = prod.p.root().cache_instance
    ora = OracleCache(2, 3, 64)
    ora.c = opk.PagedKVCache(2, 3, 64, instance=inst)
    tp = _ten_thousand_transitions(prod)
    to = _ten_thousand_transitions(ora)
    assert len(tp) == len(to)
    for i, (a, b) in enumerate(zip(tp, to)):
        assert a == b, i


def test_oracle_digests_match_c_oracle_and_product(gh, ora):
    """The three SHA-256 implementations (hashlib in oracle/paged_kv.py, the C
    oracle, the product's host SHA-256) agree on the ownership chain."""
    d0 = opk.empty_ownership_digest(7, 24, 128, 4096)
    assert d0 == ora.empty_ownership_digest(7, 24, 128, 4096)
    d1 = opk.append_ownership_digest(d0, 7, 0, 1)
    assert d1 == ora.append_ownership_digest(d0, 7, 0, 1)
    p = gh.KvPages(24, 128, 4096, pool_pages=4)
    r = p.root()
    assert bytes(r.ownership_sha256) == opk.empty_ownership_digest(r.cache_instance, 24, 128, 4096)
    rc, m = p.begin_row()
    assert rc == 0
    rc, b, a = p.staged_roots(m)
    assert rc == 0 and bytes(b.ownership_sha256) == bytes(r.ownership_sha256)
    assert bytes(a.ownership_sha256) == opk.append_ownership_digest(
        bytes(r.ownership_sha256), r.cache_instance, 0, 1)
    assert (a.generation, a.committed_len, a.committed_pages) == (2, 1, 1)


def test_product_pool_exhaustion_is_cache_full_without_mutation(gh):
    """A begin that needs a payload from an empty pool fails before any state
    changes (validate-before-write, paged_kv_cache.zig:2167 second-page OOM)."""
    p = gh.KvPages(1, 2, 64, pool_pages=1)
    for _ in range(16):
        rc, m = p.begin_row()
        assert rc == 0 and p.commit_row(m) == 0
    root = bytes(p.root())
    led = p.ledger()
    rc, _ = p.begin_row()
    assert rc == gh.CACHE_FULL
    assert bytes(p.root()) == root and p.ledger() == led
    assert p.page(1) == (-1, 0)


# ---------------------------------------------------------------------------------
# per-token publication digests (paged_token_txn.zig:762-808, 1064-1148)
# ---------------------------------------------------------------------------------
def _random_proposal(gh, rng):
    p = gh.TokenProposal()
    for f, _ in gh.TokenProposal._fields_:
        if f in ("receipt", "lanes"):
            continue
        setattr(p, f, int(rng.integers(0, 1 << 63)) if f not in ("live_mask", "live_lane_count")
                else int(rng.integers(0, 16)))
    for f, _ in gh.BankReceipt._fields_:
        if f == "claim":
            for g, _ in gh.Claim._fields_:
                setattr(p.receipt.claim, g, int(rng.integers(0, 1 << 62)))
        else:
            setattr(p.receipt, f, int(rng.integers(0, 1 << 32 if f == "slot_index" else 1 << 62)))
    for lane in p.lanes:
        for f, t in gh.LaneProposal._fields_:
            if f == "kv_transition":
                for g, tt in gh.RootTransition._fields_:
                    if tt == C.c_uint64:
                        setattr(lane.kv_transition, g, int(rng.integers(0, 1 << 62)))
                    elif tt == C.c_uint32:
                        setattr(lane.kv_transition, g, int(rng.integers(0, 2)))
                    else:
                        getattr(lane.kv_transition, g)[:] = rng.integers(0, 256, 32).tolist()
            elif f in ("rng_before", "rng_after"):
                getattr(lane, f)[:] = [int(x) for x in rng.integers(0, 1 << 62, 4)]
            elif t == C.c_uint32:
                setattr(lane, f, int(rng.integers(0, 1 << 31)) if f in ("lane_index", "token_id")
                        else int(rng.integers(0, 2)))
            else:
                setattr(lane, f, int(rng.integers(0, 1 << 62)))
    return p


import ctypes as C  # noqa: E402


@pytest.mark.parametrize("seed", range(4))
def test_product_proposal_and_commit_digests_equal_oracle(gh, seed):
    """The product's proposalSha256 / commitSha256 (csrc/publication.cpp)
    equal the oracle's restatement (oracle/publication.py, written from the
    reference's field list) on random records; a one-byte change of any lane
    field changes the digest."""
    import numpy as np

    from oracle import publication as opub

    rng = np.random.default_rng(seed)
    p = _random_proposal(gh, rng)
    out = (C.c_uint8 * 32)()
    assert gh.lib().glacier_hip_token_proposal_sha256(C.byref(p), out) == 0
    sha = bytes(out)
    assert sha == opub.proposal_sha256(p)
    p.lanes[3].token_id ^= 1
    assert gh.lib().glacier_hip_token_proposal_sha256(C.byref(p), out) == 0
    assert bytes(out) != sha and bytes(out) == opub.proposal_sha256(p)
    ack = gh.PrepareAck(gh.PREPARE_ACK_ABI, (C.c_uint8 * 32)(*sha), 0x50414745, 7)
    assert gh.lib().glacier_hip_token_commit_sha256((C.c_uint8 * 32)(*sha), C.byref(ack), out) == 0
    assert bytes(out) == opub.commit_sha256(sha, gh.PREPARE_ACK_ABI, sha, 0x50414745, 7)
