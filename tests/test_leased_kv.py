"""Leased paged KV: page payloads charged through a LeaseTree
(glacier_hip_lease_* / glacier_hip_leased_kv_* over host page maps).

The reference's own scenarios (leased_paged_kv_cache.zig:1709-2056 "two
leased lanes share current tree and reclaim exact physical pages",
:2058-2178 "leased allocation OOM aborts Bank reservation and can retry",
:2302-2388 "teardown reclaims active reusable and empty leased scopes") run
step for step against both the oracle restatement (oracle/leased_kv.py) and
the product through the C ABI; every expected error name and every charge
the reference asserts is asserted on both. A randomized run then drives both
with the same operations and compares outcomes, charges, bank counters,
binding summaries, tree generations and page-map roots after every step.
Cases the C ABI cannot express (copies of the address-bound coordinator
object) are the reference's copy fences; the ABI hands out opaque handles.
"""
import ctypes as C
import random

import pytest

from oracle import leased_kv as ol

PB = 128  # one page payload: 1 layer x K,V x 16 rows x 1 f32


class Product:
    name = "product"

    def __init__(self, gh):
        self.gh = gh
        self.Error = gh.LeaseError

    def bank(self, slots, nodes, epoch, **lim):
        return self.gh.LeaseBank(slots, nodes, epoch, **lim)

    def pages(self, layers, dim, max_seq, pool):
        return self.gh.KvPages(layers, dim, max_seq, pool)

    def seq(self):
        return C.c_uint64(0)

    def leased(self, bank, tree, scope, pages, epoch, session, seq):
        return self.gh.LeasedKV(bank, tree, scope, pages, epoch, session, seq)

    def plan(self, lk):
        return lk.plan_next_row()

    def begin(self, lk, plan):
        return lk.begin_row(plan)

    def append(self, lk, txn, value):
        lk.append_row(txn, 0, [value], [-value])

    def commit(self, lk, txn):
        return lk.commit_row(txn)

    def abort(self, lk, txn):
        lk.abort_row(txn)

    def summary(self, lk):
        s = lk.binding_summary()
        return s.count, s.payload_bytes

    def root(self, pages):
        return pages.root()

    def root_key(self, r):
        return (r.generation, r.committed_len, r.committed_pages)

    def kv(self, pages):
        return pages.kv_sha256()

    def tree_kv(self, tree):
        return tree.current.kv_bytes

    def tree_gens(self, tree):
        return (tree.identity_generation, tree.generation, tree.structural_revision,
                tree.active_nodes)

    def allocated(self, pages):
        return pages.ledger()["allocated_pages"]

    def retired(self, pages):
        return pages.is_retired()

    def page_ref_valid(self, pages, txn):
        return pages.validate_page_ref(txn.mark.page_ref) == 0

    def swap_bindings(self, lk, i, j):
        a, b = self.gh.PageLeaseBinding(), self.gh.PageLeaseBinding()
        C.memmove(C.byref(a), C.byref(lk.bindings[i]), C.sizeof(a))
        C.memmove(C.byref(b), C.byref(lk.bindings[j]), C.sizeof(b))
        lk.bindings[i], lk.bindings[j] = b, a

    def take_binding(self, lk, i):
        saved = self.gh.PageLeaseBinding()
        C.memmove(C.byref(saved), C.byref(lk.bindings[i]), C.sizeof(saved))
        lk.bindings[i] = self.gh.PageLeaseBinding(abi_version=0x47504C4200000001,
                                                  scope_index=0xFFFFFFFF)
        return saved

    def put_binding(self, lk, i, saved):
        lk.bindings[i] = saved

    def forge_extra(self, lk, src, dst):
        b = self.gh.PageLeaseBinding()
        C.memmove(C.byref(b), C.byref(lk.bindings[src]), C.sizeof(b))
        b.logical_page = dst
        lk.bindings[dst] = b

    def forge_seal_scope(self, seal, scope_index):
        s = self.gh.TerminalSeal()
        C.memmove(C.byref(s), C.byref(seal), C.sizeof(s))
        s.scope_index = scope_index
        return s

    def forge_freed(self, freed):
        f = self.gh.FreedPayload()
        C.memmove(C.byref(f), C.byref(freed), C.sizeof(f))
        f.payload_bytes += 1
        return f

    def seal_count(self, seal):
        return seal.bindings.count, seal.bindings.payload_bytes

    def alloc_bytes(self, plan):
        return plan.cache_plan.allocation_bytes


class Oracle(Product):
    name = "oracle"

    def __init__(self):
        self.Error = ol.LeaseFailure

    def bank(self, slots, nodes, epoch, **lim):
        return ol.Bank(slots, nodes, epoch, **lim)

    def pages(self, layers, dim, max_seq, pool):
        return ol.Pages(layers, dim, max_seq, pool)

    def seq(self):
        class Cell:
            value = 0
        return Cell()

    def leased(self, bank, tree, scope, pages, epoch, session, seq):
        return ol.Leased(bank, tree, scope, pages, epoch, session, seq)

    def append(self, lk, txn, value):
        lk.append_row(txn, 0, [value], [-value])

    def summary(self, lk):
        return lk.binding_summary()

    def root(self, pages):
        return pages.cache.root()

    def kv(self, pages):
        return pages.kv_sha256()

    def tree_kv(self, tree):
        return tree.current.kv_bytes

    def tree_gens(self, tree):
        return (tree.identity_generation, tree.generation, tree.structural_revision,
                tree.active_nodes)

    def allocated(self, pages):
        return pages.cache.allocated_pages

    def retired(self, pages):
        return pages.retired

    def page_ref_valid(self, pages, mark):
        try:
            pages.cache.validate_committed_page_ref(mark.cache_instance, mark.logical_page,
                                                    mark.ownership_generation)
            return True
        except Exception:
            return False

    def swap_bindings(self, lk, i, j):
        lk.bindings[i], lk.bindings[j] = lk.bindings[j], lk.bindings[i]

    def take_binding(self, lk, i):
        saved, lk.bindings[i] = lk.bindings[i], None
        return saved

    def put_binding(self, lk, i, saved):
        lk.bindings[i] = saved

    def forge_extra(self, lk, src, dst):
        lk.bindings[dst] = list(lk.bindings[src])

    def forge_seal_scope(self, seal, scope_index):
        return dict(seal, scope=scope_index)

    def forge_freed(self, freed):
        return dict(freed, bytes=freed["bytes"] + 1)

    def seal_count(self, seal):
        return seal["bindings"]

    def alloc_bytes(self, plan):
        return plan["allocation_bytes"]


@pytest.fixture(params=["oracle", "product"])
def impl(request):
    if request.param == "oracle":
        return Oracle()
    import glacier_hip as gh
    try:
        gh.lib()
    except RuntimeError as e:
        pytest.fail(str(e))
    return Product(gh)


def reason(impl, fn, *a, **kw):
    with pytest.raises(impl.Error) as e:
        fn(*a, **kw)
    return e.value.reason


def scalar_row(impl, lk, value):
    txn = impl.begin(lk, impl.plan(lk))
    impl.append(lk, txn, value)
    impl.commit(lk, txn)
    return txn


def test_two_lanes_share_tree_and_reclaim_exact_pages(impl):
    """leased_paged_kv_cache.zig:1709-2056."""
    bank = impl.bank(1, 8, 0x4C504341, kv_bytes=512, queue_slots=1)
    parent = bank.commit(bank.reserve(1, queue_slots=1))
    tree = bank.open_tree(parent, 0x74726565, 0x61757468, kv_bytes=512)
    left_scope = bank.open_scope(tree, 10, 100, kv_bytes=256)
    right_scope = bank.open_scope(tree, 11, 101, kv_bytes=256)
    epoch, sid = 0x4C504342, 0x5E55_1001
    seq = impl.seq()
    bank.bind_session(tree, epoch, sid)
    left_pages = impl.pages(1, 1, 33, 8)
    right_pages = impl.pages(1, 1, 17, 8)
    left = impl.leased(bank, tree, left_scope, left_pages, epoch, sid, seq)
    # a second coordinator cannot take the same page map
    assert reason(impl, impl.leased, bank, tree, left_scope, left_pages, epoch, sid,
                  seq) == "InvalidCoordinator"
    right = impl.leased(bank, tree, right_scope, right_pages, epoch, sid, seq)

    stale_left_plan = impl.plan(left)
    scalar_row(impl, right, 2.0)  # the sibling changed the shared tree
    assert reason(impl, impl.begin, left, stale_left_plan) == "InvalidLeasedPlan"
    left_empty_root = impl.root(left_pages)
    left_txn = impl.begin(left, impl.plan(left))
    impl.append(left, left_txn, 1.0)
    impl.commit(left, left_txn)
    assert reason(impl, impl.commit, left, left_txn) == "InvalidLeasedTransaction"
    for i in range(1, 17):
        second = scalar_row(impl, left, float(i + 1))
    left_root = impl.root(left_pages)
    assert impl.tree_kv(tree) == 3 * PB
    assert impl.summary(left) == (2, 2 * PB) and impl.summary(right) == (1, PB)
    assert impl.allocated(left_pages) == 2 and impl.allocated(right_pages) == 1

    # membership is exact: order, omission and an extra forged entry fail
    impl.swap_bindings(left, 0, 1)
    assert reason(impl, impl.summary, left) == "InvalidBinding"
    impl.swap_bindings(left, 0, 1)
    saved = impl.take_binding(left, 1)
    assert reason(impl, impl.summary, left) == "InvalidBinding"
    impl.put_binding(left, 1, saved)
    impl.forge_extra(left, 1, 2)
    assert reason(impl, impl.summary, left) == "InvalidBinding"
    impl.take_binding(left, 2)
    assert impl.summary(left) == (2, 2 * PB)

    # a mutation after planning is rejected before the map or the bank changes
    plan = impl.plan(left)
    root_before = impl.root_key(impl.root(left_pages))
    used_before = bank.snapshot()["used"]["kv_bytes"]
    saved = impl.take_binding(left, 1)
    assert reason(impl, impl.begin, left, plan) == "InvalidBinding"
    impl.put_binding(left, 1, saved)
    assert impl.root_key(impl.root(left_pages)) == root_before
    assert bank.snapshot()["used"]["kv_bytes"] == used_before

    left_digest = impl.kv(left_pages)
    assert reason(impl, left.seal_terminal, left_empty_root, left_digest, 0, 0, 9) == "InvalidRoot"
    assert reason(impl, left.seal_terminal, left_root, bytes(32), 0, 0, 9) == "InvalidTerminalSeal"
    left_seal = left.seal_terminal(left_root, left_digest, 0, 0, 9)
    assert impl.seal_count(left_seal) == (2, 2 * PB)
    assert seq.value == 1
    assert reason(impl, right.begin_reclaim, left_seal, 1) == "TerminalRequired"
    forged = impl.forge_seal_scope(left_seal, right_scope.node_index)
    assert reason(impl, left.begin_reclaim, forged, 1) == "InvalidTerminalSeal"

    right_seal = right.seal_terminal(impl.root(right_pages), impl.kv(right_pages), 1, 1, 10)
    assert impl.seal_count(right_seal) == (1, PB)
    assert seq.value == 2

    # left published first; its reclaim takes the cohort's current sequence
    left_freed = left.begin_reclaim(left_seal, 2)
    assert impl.retired(left_pages)
    assert impl.root_key(impl.root(left_pages)) != impl.root_key(left_root)
    assert not impl.page_ref_valid(left_pages, second if impl.name == "product" else second)
    assert impl.allocated(left_pages) == 0
    snap = bank.snapshot()
    assert snap["used"]["kv_bytes"] == 3 * PB and snap["free_authorized_allocations"] == 2
    assert reason(impl, left.commit_reclaim, impl.forge_freed(left_freed)) == "InvalidFreedPayload"
    assert bank.snapshot()["used"]["kv_bytes"] == 3 * PB
    left.commit_reclaim(left_freed)
    assert reason(impl, left.commit_reclaim, left_freed) == "ReclaimComplete"
    snap = bank.snapshot()
    assert snap["used"]["kv_bytes"] == PB and snap["live_allocations"] == 1

    assert reason(impl, left.begin_reclaim, right_seal, 2) == "InvalidTerminalSeal"
    right_freed = right.begin_reclaim(right_seal, 2)
    right.commit_reclaim(right_freed)
    assert impl.tree_kv(tree) == 0
    bank.close_session(parent, epoch, sid, seq.value)
    bank.close_tree(tree)
    bank.release(parent)
    snap = bank.snapshot()
    assert not any(snap["used"].values())
    assert snap["lease_reclaim_commits"] == 2 and snap["lease_allocation_materializations"] == 3


def test_allocation_failure_aborts_the_charge_and_retries(impl):
    """leased_paged_kv_cache.zig:2058-2178."""
    bank = impl.bank(1, 3, 0x4C504343, kv_bytes=256, queue_slots=1)
    parent = bank.commit(bank.reserve(1, queue_slots=1))
    tree = bank.open_tree(parent, 1, 2, kv_bytes=256)
    scope = bank.open_scope(tree, 3, 4, kv_bytes=256)
    epoch, sid = 5, 0x5E55_2002
    seq = impl.seq()
    bank.bind_session(tree, epoch, sid)
    pages = impl.pages(1, 1, 16, 1)
    lk = impl.leased(bank, tree, scope, pages, epoch, sid, seq)
    failed_plan = impl.plan(lk)
    pages.set_pool_capacity(0)  # the allocator refuses the next payload
    assert reason(impl, impl.begin, lk, failed_plan) == "OutOfMemory"
    assert impl.summary(lk) == (0, 0) and impl.allocated(pages) == 0
    snap = bank.snapshot()
    assert snap["used"]["kv_bytes"] == 0
    assert snap["lease_allocation_reserves"] == 1 and snap["lease_allocation_aborts"] == 1
    assert reason(impl, impl.begin, lk, failed_plan) == "InvalidLeasedPlan"

    pages.set_pool_capacity(1)
    aborted = impl.begin(lk, impl.plan(lk))
    impl.abort(lk, aborted)
    assert impl.summary(lk) == (1, PB)
    assert bank.snapshot()["used"]["kv_bytes"] == PB
    assert not impl.page_ref_valid(pages, aborted)
    assert impl.alloc_bytes(impl.plan(lk)) == 0  # the payload is reused, no new charge
    scalar_row(impl, lk, 7.0)
    assert impl.allocated(pages) == 1
    seal = lk.seal_terminal(impl.root(pages), impl.kv(pages), 0, 2, 0)
    freed = lk.begin_reclaim(seal, 1)
    assert impl.allocated(pages) == 0
    assert bank.snapshot()["used"]["kv_bytes"] == PB
    lk.commit_reclaim(freed)
    bank.close_session(parent, epoch, sid, seq.value)
    bank.close_tree(tree)
    bank.release(parent)
    assert not any(bank.snapshot()["used"].values())


def test_teardown_reclaims_active_and_empty_scopes(impl):
    """leased_paged_kv_cache.zig:2302-2388."""
    bank = impl.bank(1, 5, 0x4C504351, kv_bytes=512, queue_slots=1)
    parent = bank.commit(bank.reserve(31, queue_slots=1))
    tree = bank.open_tree(parent, 32, 33, kv_bytes=512)
    live_scope = bank.open_scope(tree, 34, 35, kv_bytes=256)
    empty_scope = bank.open_scope(tree, 36, 37, kv_bytes=256)
    epoch, sid = 38, 0x5E55_3003
    seq = impl.seq()
    bank.bind_session(tree, epoch, sid)
    live_pages, empty_pages = impl.pages(1, 1, 16, 1), impl.pages(1, 1, 16, 1)
    live = impl.leased(bank, tree, live_scope, live_pages, epoch, sid, seq)
    empty = impl.leased(bank, tree, empty_scope, empty_pages, epoch, sid, seq)
    txn = impl.begin(live, impl.plan(live))
    impl.append(live, txn, 5.0)  # staged, never committed
    assert bank.snapshot()["used"]["kv_bytes"] != 0
    live.reclaim_for_teardown(seq.value)
    empty.reclaim_for_teardown(seq.value)
    assert impl.retired(live_pages) and impl.retired(empty_pages)
    assert impl.tree_kv(tree) == 0
    bank.close_session(parent, epoch, sid, seq.value)
    bank.close_tree(tree)
    bank.release(parent)
    assert not any(bank.snapshot()["used"].values())


def test_bank_rejects_like_the_reference(impl):
    """Receipt and tree rules the leased path leans on: zero claims, capacity,
    slots, scope ceilings, node exhaustion, stale trees, close ordering
    (resource_bank.zig:976-1044, :1404-1514, :2582-2622, :3166-3184)."""
    bank = impl.bank(1, 2, 7, kv_bytes=300, queue_slots=1)
    assert reason(impl, bank.reserve, 0, queue_slots=1) == "InvalidClaim"
    assert reason(impl, bank.reserve, 1) == "InvalidClaim"
    assert reason(impl, bank.reserve, 1, queue_slots=2) == "CapacityExceeded"
    res = bank.reserve(1, queue_slots=1)
    assert reason(impl, bank.reserve, 2, kv_bytes=1) == "ReservationSlotsExhausted"
    assert reason(impl, bank.open_tree, res, 1, 2, kv_bytes=256) in ("InvalidTransition",
                                                                     "StaleReservation")
    parent = bank.commit(res)
    assert reason(impl, bank.commit, res) == "StaleReservation"
    assert reason(impl, bank.open_tree, parent, 0, 2, kv_bytes=256) == "InvalidClaim"
    tree = bank.open_tree(parent, 1, 2, kv_bytes=256)
    old = impl_copy_tree(impl, tree)
    assert reason(impl, bank.open_scope, tree, 3, 4, kv_bytes=257) == "InvalidTransition"
    bank.open_scope(tree, 3, 4, kv_bytes=128)
    assert reason(impl, bank.open_scope, tree, 3, 5, kv_bytes=128) == "InvalidTransition"
    assert reason(impl, bank.open_scope, old, 9, 5, kv_bytes=128) == "StaleReservation"
    bank.open_scope(tree, 6, 7, kv_bytes=128)
    assert reason(impl, bank.open_scope, tree, 8, 9, kv_bytes=128) == "LeaseNodesExhausted"
    assert reason(impl, bank.release, parent) == "InvalidTransition"  # the tree is live
    bank.close_tree(tree)
    bank.release(parent)
    snap = bank.snapshot()
    assert snap["lease_tree_opens"] == 1 and snap["lease_scope_opens"] == 2
    assert snap["lease_tree_closes"] == 1 and snap["rejected_lease_nodes"] == 1


def impl_copy_tree(impl, tree):
    if impl.name == "product":
        t = impl.gh.LeaseTree()
        C.memmove(C.byref(t), C.byref(tree), C.sizeof(t))
        return t
    import copy
    return copy.deepcopy(tree)


def _drive(impl, ops):
    """Runs an operation list on one implementation; returns the trace."""
    bank = impl.bank(1, 16, 0x52414E44, kv_bytes=8 * PB, queue_slots=1)
    parent = bank.commit(bank.reserve(9, queue_slots=1))
    tree = bank.open_tree(parent, 11, 12, kv_bytes=8 * PB)
    scopes = [bank.open_scope(tree, 20 + i, 30 + i, kv_bytes=4 * PB) for i in range(2)]
    epoch, sid = 41, 0x5E55_4004
    seq = impl.seq()
    bank.bind_session(tree, epoch, sid)
    pages = [impl.pages(1, 1, 64, 5), impl.pages(1, 1, 64, 5)]
    lanes = [impl.leased(bank, tree, scopes[i], pages[i], epoch, sid, seq) for i in range(2)]
    staged = [None, None]
    seals = [None, None]
    freed = [None, None]
    trace = []
    for op, lane, arg in ops:
        lk, pg = lanes[lane], pages[lane]
        try:
            if op == "row":
                if staged[lane] is None:
                    staged[lane] = impl.begin(lk, impl.plan(lk))
                    impl.append(lk, staged[lane], float(arg))
                else:
                    impl.commit(lk, staged[lane])
                    staged[lane] = None
            elif op == "abort" and staged[lane] is not None:
                impl.abort(lk, staged[lane])
                staged[lane] = None
            elif op == "cap":
                pg.set_pool_capacity(max(arg, impl.allocated(pg)))
            elif op == "seal":
                seals[lane] = lk.seal_terminal(impl.root(pg), lk.kv_sha256(), seq.value, 0, arg)
            elif op == "reclaim" and seals[lane] is not None:
                freed[lane] = lk.begin_reclaim(seals[lane], seq.value)
                lk.commit_reclaim(freed[lane])
            elif op == "teardown":
                lk.reclaim_for_teardown(seq.value)
                staged[lane] = None
            elif op == "renew" and lk.lifecycle() == "reclaimed":
                # a new request on the lane's scope: fresh page map and coordinator
                pages[lane] = pg = impl.pages(1, 1, 64, 5)
                lanes[lane] = lk = impl.leased(bank, tree, scopes[lane], pg, epoch, sid, seq)
                seals[lane] = None
            out = "ok"
        except impl.Error as e:
            out = e.reason
            if op == "row" and staged[lane] is not None and out != "ok":
                pass
        snap = bank.snapshot()
        try:
            summ = impl.summary(lk)
        except impl.Error as e:
            summ = e.reason
        trace.append((op, lane, out, impl.tree_kv(tree), impl.tree_gens(tree), summ,
                      snap["used"]["kv_bytes"], snap["live_allocations"],
                      snap["lease_allocation_aborts"], snap["lease_reclaim_commits"], seq.value,
                      impl.root_key(impl.root(pg)), impl.allocated(pg), impl.retired(pg)))
    return trace


@pytest.mark.parametrize("seed", range(6))
def test_random_operations_match_the_oracle(seed):
    import glacier_hip as gh
    rng = random.Random(seed)
    ops = []
    for _ in range(300):
        r = rng.random()
        lane = rng.randrange(2)
        if r < 0.66:
            ops.append(("row", lane, rng.randrange(1, 1000)))
        elif r < 0.76:
            ops.append(("abort", lane, 0))
        elif r < 0.84:
            ops.append(("cap", lane, rng.randrange(0, 6)))
        elif r < 0.87:
            ops.append(("seal", lane, rng.randrange(100)))
        elif r < 0.91:
            ops.append(("reclaim", lane, 0))
        elif r < 0.93:
            ops.append(("teardown", lane, 0))
        else:
            ops.append(("renew", lane, 0))
    want = _drive(Oracle(), ops)
    got = _drive(Product(gh), ops)
    for i, (w, g) in enumerate(zip(want, got)):
        assert w == g, f"step {i}: {ops[i]}\noracle  {w}\nproduct {g}"


def _oracle_lane(kv_limit, nodes, epoch):
    bank = ol.Bank(1, nodes, epoch, kv_bytes=kv_limit)
    receipt = bank.commit(bank.reserve(1, queue_slots=1))
    tree = bank.open_tree(receipt, 1, 2, kv_bytes=128)
    scope = bank.open_scope(tree, 3, 4, kv_bytes=128)
    bank.bind_session(tree, 5, 0x5E55)
    return bank, receipt, tree, scope


def oreason(fn, *a):
    with pytest.raises(ol.LeaseFailure) as e:
        fn(*a)
    return e.value.reason


def test_oracle_aborted_reservation_stays_charged_until_abort():
    """resource_bank.zig:6348-6435 on the oracle (the product runs the same
    bank code through the leased-cache scenarios above)."""
    bank, receipt, tree, scope = _oracle_lane(128, 3, 0x50324343)
    batch, leaves = bank.reserve_allocations(tree, 5, 0x5E55, 0, [(scope, 6, 7, ol.Claim(kv_bytes=64))])
    forged = dict(batch, claim=ol.Claim(kv_bytes=63))
    assert oreason(bank.abort_allocations, forged, tree) == "StaleReservation"
    assert bank.snapshot()["used"]["kv_bytes"] == 64
    bank.abort_allocations(batch, tree)
    assert tree.current.kv_bytes == 0
    assert oreason(bank.abort_allocations, batch, tree) == "InvalidTransition"
    assert oreason(bank._node, tree, leaves[0]) == "StaleReservation"
    second, leaves2 = bank.reserve_allocations(tree, 5, 0x5E55, 0,
                                               [(scope, 8, 9, ol.Claim(kv_bytes=32))])
    assert leaves2[0].generation != leaves[0].generation
    bank.abort_allocations(second, tree)
    bank.close_session(receipt, 5, 0x5E55, 0)
    bank.close_tree(tree)
    bank.release(receipt)
    snap = bank.snapshot()
    assert not any(snap["used"].values()) and snap["lease_allocation_aborts"] == 2


def test_oracle_capacity_and_node_exhaustion_are_atomic_and_distinct():
    """resource_bank.zig:6437-6514 on the oracle: too many leaves for the
    node pool, then a leaf past the bank's capacity, each refused with its
    own error and counter and nothing charged."""
    bank, receipt, tree, scope = _oracle_lane(64, 2, 0x50324344)
    before = tree.key()
    two = [(scope, 6, 7, ol.Claim(kv_bytes=16)), (scope, 8, 9, ol.Claim(kv_bytes=16))]
    assert oreason(bank.reserve_allocations, tree, 5, 0x5E55, 0, two) == "LeaseNodesExhausted"
    bank._tree(tree)
    assert tree.key() == before
    snap = bank.snapshot()
    assert snap["used"]["kv_bytes"] == 0 and snap["rejected_lease_nodes"] == 1
    big = [(scope, 10, 11, ol.Claim(kv_bytes=65))]
    assert oreason(bank.reserve_allocations, tree, 5, 0x5E55, 0, big) == "CapacityExceeded"
    snap = bank.snapshot()
    assert snap["used"]["kv_bytes"] == 0 and snap["rejected_lease_capacity"] == 1
    batch, _ = bank.reserve_allocations(tree, 5, 0x5E55, 0, [(scope, 12, 13, ol.Claim(kv_bytes=64))])
    bank.commit_allocations(batch, tree)
    assert bank.snapshot()["used"]["kv_bytes"] == 64


def test_oracle_retire_cancel_and_forged_permit_keep_the_charge():
    """resource_bank.zig:6516-6605 on the oracle: a cancelled retirement
    keeps the charge and its ticket can no longer authorize; an authorized
    one can no longer cancel; a forged free permit (the reference alters its
    node-set digest, here its node count) is stale and uncharges nothing."""
    bank, receipt, tree, scope = _oracle_lane(128, 3, 0x50324345)
    batch, _ = bank.reserve_allocations(tree, 5, 0x5E55, 0, [(scope, 6, 7, ol.Claim(kv_bytes=64))])
    bank.commit_allocations(batch, tree)
    first = bank.begin_retire(tree, scope, 5, 0x5E55, 0)
    bank.cancel_retire(first, tree)
    assert bank.snapshot()["used"]["kv_bytes"] == 64
    assert oreason(bank.authorize_free, first, tree) == "InvalidTransition"
    second = bank.begin_retire(tree, scope, 5, 0x5E55, 0)
    permit = bank.authorize_free(second, tree)
    assert oreason(bank.cancel_retire, second, tree) == "InvalidTransition"
    assert oreason(bank.commit_free, dict(permit, count=permit["count"] + 1), tree) == "StaleReservation"
    assert bank.snapshot()["used"]["kv_bytes"] == 64
    bank.commit_free(permit, tree)
    bank.close_session(receipt, 5, 0x5E55, 0)
    bank.close_tree(tree)
    bank.release(receipt)
    snap = bank.snapshot()
    assert not any(snap["used"].values())
    assert (snap["lease_reclaim_prepares"], snap["lease_reclaim_authorizations"],
            snap["lease_reclaim_cancels"], snap["lease_reclaim_commits"]) == (2, 1, 1, 1)


def _bound_tree(gh, bank, owner, epoch, session):
    parent = bank.commit(bank.reserve(owner, queue_slots=4))
    tree = bank.open_tree(parent, owner + 1, owner + 2, queue_slots=4)
    bank.bind_session(tree, epoch, session)
    return parent, tree


def _reason(gh, fn, *args):
    with pytest.raises(gh.LeaseError) as e:
        fn(*args)
    return e.value.reason


def test_publication_permit_lifecycle(gh):
    """resource_bank.zig:5019-5077 ("publication session permits are exact and
    single-use"), with the session bound through a LeaseTree: one live permit
    per receipt, abort and commit each take it once, commit advances the
    sequence, a retry gets a new generation."""
    bank = gh.LeaseBank(1, 4, 21, queue_slots=4)
    parent, tree = _bound_tree(gh, bank, 7, 99, 0x51)
    assert _reason(gh, bank.bind_session, tree, 99, 0x51) == "InvalidTransition"
    first = bank.begin_publication(tree, 99, 0x51, 0)
    assert _reason(gh, bank.begin_publication, tree, 99, 0x51, 0) == "InvalidTransition"
    assert _reason(gh, bank.close_session, parent, 99, 0x51, 0) == "InvalidTransition"
    bank.abort_publication(first)
    assert _reason(gh, bank.abort_publication, first) == "InvalidTransition"
    retry = bank.begin_publication(tree, 99, 0x51, 0)
    assert retry.generation != first.generation
    bank.commit_publication(retry)
    assert _reason(gh, bank.commit_publication, retry) == "InvalidTransition"
    assert _reason(gh, bank.begin_publication, tree, 99, 0x51, 0) == "InvalidTransition"
    second = bank.begin_publication(tree, 99, 0x51, 1)
    bank.abort_publication(second)
    bank.close_session(parent, 99, 0x51, 1)
    bank.close_tree(tree)
    bank.release(parent)
    bank.close()


def test_publication_permit_rejects_forged_identity(gh):
    """resource_bank.zig:5126-5163 ("publication permit rejects wrong
    coordinator and forged identity"): a permit copied with another session,
    another sequence, epoch or generation, or a flipped integrity word is
    refused by abort and by commit and changes nothing; the real permit
    still aborts."""
    bank = gh.LeaseBank(1, 4, 22, queue_slots=4)
    parent, tree = _bound_tree(gh, bank, 8, 100, 0xA1)
    assert _reason(gh, bank.begin_publication, tree, 100, 0xA2, 0) == "InvalidTransition"
    permit = bank.begin_publication(tree, 100, 0xA1, 0)
    for field, delta in (("session_id", 1), ("integrity", 1), ("sequence", 1),
                         ("request_epoch", 1), ("generation", 1)):
        forged = gh.PublicationPermit.from_buffer_copy(permit)
        setattr(forged, field, getattr(forged, field) ^ delta)
        assert _reason(gh, bank.abort_publication, forged) == "InvalidTransition", field
        assert _reason(gh, bank.commit_publication, forged) == "InvalidTransition", field
    bank.abort_publication(permit)
    assert _reason(gh, bank.close_session, parent, 100, 0xA2, 0) == "InvalidTransition"
    bank.close_session(parent, 100, 0xA1, 0)
    bank.close_tree(tree)
    bank.release(parent)
    bank.close()


def test_publication_close_is_terminal_and_prevents_replay(gh):
    """resource_bank.zig:5165-5211 ("publication close is terminal for one
    receipt and prevents replay ABA"): after close the receipt cannot bind
    again; once the receipt is released a permit from it is a stale
    reservation, even when a new receipt takes the same slot."""
    bank = gh.LeaseBank(1, 4, 24, queue_slots=4)
    parent, tree = _bound_tree(gh, bank, 9, 101, 0xB1)
    stale = bank.begin_publication(tree, 101, 0xB1, 0)
    bank.abort_publication(stale)
    bank.close_session(parent, 101, 0xB1, 0)
    assert _reason(gh, bank.bind_session, tree, 101, 0xB1) == "InvalidTransition"
    bank.close_tree(tree)
    bank.release(parent)
    parent2, tree2 = _bound_tree(gh, bank, 10, 101, 0xB1)
    current = bank.begin_publication(tree2, 101, 0xB1, 0)
    assert current.receipt.generation != stale.receipt.generation
    assert _reason(gh, bank.abort_publication, stale) == "StaleReservation"
    bank.abort_publication(current)
    bank.close_session(parent2, 101, 0xB1, 0)
    bank.close_tree(tree2)
    bank.release(parent2)
    bank.close()
