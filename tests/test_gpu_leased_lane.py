"""Leased session lanes (glacier_hip_leased_kv_create_for_lane): the device
page payloads of one lane charged through a LeaseTree as the reference's
LeasedPagedKVCache charges its allocator pages (leased_paged_kv_cache.zig
:482-565), sealed (:691-757) and reclaimed back to the session's pool
(:918-1080).

A leased lane decodes exactly what an unleased lane decodes (same tokens,
same KV digest); every page it takes is one exact kv_bytes leaf of its scope
from the step that takes it; a step whose new page the lease refuses fails
with OUT_OF_MEMORY and publishes nothing (root, charge and published tokens
unchanged); seal + reclaim return the lane's pages to the pool and the
charge to zero; the lane cannot start a new request while leased and can
once the coordinator is gone. Staged publication waves over leased lanes
take one cohort permit per wave (paged_lease_token_txn.zig)."""
import ctypes as C

import pytest

pytestmark = pytest.mark.gpu

TINY = dict(num_layers=2, dim=256, hidden_dim=512, num_heads=4, num_kv_heads=2, head_dim=64,
            vocab_size=4096, group_size=32, rms_eps=1e-6, rope_theta=1e6)
SEED = 0x4C454153
MAXPOS = 96
PAGES = MAXPOS // 16
PB = TINY["num_layers"] * 2 * 16 * TINY["num_kv_heads"] * TINY["head_dim"] * 2  # fp16 payload


@pytest.fixture(scope="module")
def model(gh, gctx):
    m = gh.Model(gctx, TINY)
    m.init_random(SEED)
    yield m
    m.close()


def _cohort(gh, scope_pages):
    bank = gh.LeaseBank(2, 16, 0x4C4C, kv_bytes=64 * PB, queue_slots=4)
    parent = bank.commit(bank.reserve(1, queue_slots=1))
    tree = bank.open_tree(parent, 2, 3, kv_bytes=16 * PB)
    scope = bank.open_scope(tree, 4, 5, kv_bytes=scope_pages * PB)
    seq = C.c_uint64(0)
    bank.bind_session(tree, 6, 0x5E55)
    return bank, parent, tree, scope, seq


def _decode(sess, lane, prompt, n):
    toks = [sess.prefill(lane, prompt)]
    for _ in range(n):
        toks.append(int(sess.step([lane], [toks[-1]])[0]))
    return toks


def test_leased_lane_charges_pages_and_reclaims(gh, model):
    sess = gh.Session(model, max_lanes=2, max_positions=MAXPOS, kv_dtype=gh.F16)
    try:
        bank, parent, tree, scope, seq = _cohort(gh, PAGES)
        prompt = gh.synth_tokens(SEED, 1, TINY["vocab_size"], 21)
        sess.begin(0, seed=3)
        sess.begin(1, seed=3)
        print("leased lane: create", flush=True)
        lk = gh.LeasedKV(bank, tree, scope, sess, 6, 0x5E55, seq, lane=0, binding_count=PAGES)
        assert lib_rc(gh, sess, 0) == gh.INVALID_TRANSACTION  # no new request while leased
        first = sess.prefill(0, prompt)
        assert tree.current.kv_bytes == 2 * PB  # 21 rows: two pages, each charged once
        s = lk.binding_summary()
        assert (s.count, s.payload_bytes) == (2, 2 * PB)
        toks = [first]
        for i in range(16):  # to 37 positions: the third page from the step at row 32
            toks.append(int(sess.step([0], [toks[-1]])[0]))
            assert tree.current.kv_bytes == (3 if 21 + i + 1 > 32 else 2) * PB
        assert toks == _decode(sess, 1, prompt, 16)  # the unleased lane decodes the same
        assert sess.kv_sha256(0) == sess.kv_sha256(1) == lk.kv_sha256()
        snap = bank.snapshot()
        assert snap["used"]["kv_bytes"] == 3 * PB and snap["live_allocations"] == 3
        # the prompt's two pages are one allocation wave, the decode page another
        assert snap["lease_allocation_materializations"] == 2

        root = lk.root()
        seal = lk.seal_terminal(root, lk.kv_sha256(), 0, 0, toks[-1])
        assert seq.value == 1 and seal.bindings.count == 3
        rc, _ = sess.step([0], [toks[-1]], raise_on_error=False)
        assert rc != gh.OK  # a sealed lane takes no more rows
        freed = lk.begin_reclaim(seal, 1)
        assert freed.payload_bytes == 3 * PB
        assert all(sess.page_of(0, p) == -1 for p in range(PAGES))  # back in the pool
        assert bank.snapshot()["used"]["kv_bytes"] == 3 * PB  # charged until the commit
        lk.commit_reclaim(freed)
        assert tree.current.kv_bytes == 0 and lk.lifecycle() == "reclaimed"
        lk.close()
        sess.begin(0, seed=3)  # unleased: a new request
        assert _decode(sess, 0, prompt, 4) == toks[:5]
        bank.close_session(parent, 6, 0x5E55, seq.value)
        bank.close_tree(tree)
        bank.release(parent)
        assert not any(bank.snapshot()["used"].values())
    finally:
        sess.close()


def test_two_leased_lanes_on_one_tree_take_pages_in_one_step(gh, model):
    """Two leased lanes of one LeaseTree (one scope each) whose rows cross a
    page boundary in the same decode step: each lane's page is reserved,
    taken and settled before the next lane reserves (beginRowPlanned per
    coordinator, leased_paged_kv_cache.zig:482-565), so the step succeeds and
    both lanes decode as unleased lanes do. At the next boundary the second
    lane's scope is full: the step fails, nothing is published on either
    lane, and the first lane's new page stays charged with its logical page
    (abortRowTxn), which that lane then continues onto."""
    sess = gh.Session(model, max_lanes=4, max_positions=MAXPOS, kv_dtype=gh.F16)
    try:
        bank = gh.LeaseBank(2, 16, 0x4C4C, kv_bytes=64 * PB, queue_slots=4)
        parent = bank.commit(bank.reserve(1, queue_slots=1))
        tree = bank.open_tree(parent, 2, 3, kv_bytes=16 * PB)
        scopes = [bank.open_scope(tree, 4, 5, kv_bytes=PAGES * PB),
                  bank.open_scope(tree, 6, 7, kv_bytes=2 * PB)]
        seq = C.c_uint64(0)
        bank.bind_session(tree, 6, 0x5E55)
        prompts = [gh.synth_tokens(SEED, 40 + i, TINY["vocab_size"], 15) for i in range(2)]
        for lane in range(4):
            sess.begin(lane, seed=lane % 2)
        lks = [gh.LeasedKV(bank, tree, scopes[lane], sess, 6, 0x5E55, seq, lane=lane,
                           binding_count=PAGES) for lane in range(2)]
        toks = [sess.prefill(lane, prompts[lane]) for lane in range(2)]
        ref = [sess.prefill(2 + lane, prompts[lane]) for lane in range(2)]
        assert toks == ref and tree.current.kv_bytes == 2 * PB
        print("two leased lanes: steps over a page boundary", flush=True)
        for row in range(15, 32):  # row 16 takes a new page on both lanes in one step
            toks = [int(t) for t in sess.step([0, 1], toks)]
            ref = [int(t) for t in sess.step([2, 3], ref)]
            assert toks == ref
            assert tree.current.kv_bytes == (4 if row >= 16 else 2) * PB
        assert lks[0].binding_summary().count == lks[1].binding_summary().count == 2
        root0, root1, state1 = sess.root(0), sess.root(1), sess.state(1)
        # row 32: lane 0's third page is charged and taken, lane 1's scope
        # refuses its third: the step fails and publishes nothing
        rc, _ = sess.step([0, 1], toks, raise_on_error=False)
        assert rc == gh.OUT_OF_MEMORY
        assert sess.root(0).committed_len == root0.committed_len == 32
        assert sess.root(1).committed_len == root1.committed_len == 32
        assert sess.state(1).published_tokens == state1.published_tokens
        assert tree.current.kv_bytes == 5 * PB
        assert lks[0].binding_summary().count == 3 and lks[1].binding_summary().count == 2
        # lane 0 alone continues onto the page it already holds
        assert int(sess.step([0], toks[:1])[0]) == int(sess.step([2], ref[:1])[0])
        assert tree.current.kv_bytes == 5 * PB
        assert sess.kv_sha256(0) == sess.kv_sha256(2)
        for lk in lks:
            lk.reclaim_for_teardown(seq.value)
            lk.close()
        assert tree.current.kv_bytes == 0
        bank.close_session(parent, 6, 0x5E55, seq.value)
        bank.close_tree(tree)
        bank.release(parent)
        assert not any(bank.snapshot()["used"].values())
    finally:
        sess.close()


def lib_rc(gh, sess, lane):
    return gh.lib().glacier_hip_session_lane_begin(sess.h, lane, 0)


def test_refused_page_publishes_nothing(gh, model):
    sess = gh.Session(model, max_lanes=1, max_positions=MAXPOS, kv_dtype=gh.F16)
    try:
        bank, parent, tree, scope, seq = _cohort(gh, 1)  # the scope holds one page
        sess.begin(0, seed=9)
        lk = gh.LeasedKV(bank, tree, scope, sess, 6, 0x5E55, seq, lane=0, binding_count=PAGES)
        prompt = gh.synth_tokens(SEED, 2, TINY["vocab_size"], 14)
        tok = sess.prefill(0, prompt)
        tok = int(sess.step([0], [tok])[0])
        tok = int(sess.step([0], [tok])[0])  # 16 rows: the page is full
        root, state = sess.root(0), sess.state(0)
        print("leased lane: refused page", flush=True)
        rc, _ = sess.step([0], [tok], raise_on_error=False)
        assert rc == gh.OUT_OF_MEMORY
        after = sess.root(0)
        assert (after.generation, after.committed_len) == (root.generation, root.committed_len)
        assert sess.state(0).published_tokens == state.published_tokens
        snap = bank.snapshot()
        assert snap["used"]["kv_bytes"] == PB and snap["lease_allocation_reserves"] == 1
        assert tree.current.kv_bytes == PB
        lk.reclaim_for_teardown(seq.value)
        assert tree.current.kv_bytes == 0
        lk.close()
    finally:
        sess.close()


def _wave_binding(gh, slots, seq, terminal=()):
    b = gh.PublicationBinding()
    b.execution_abi = 0x5042544553540001
    b.request_epoch = 6
    b.transaction_sequence = seq
    b.resource_permit_generation = 999  # replaced by the cohort permit's generation
    b.kv_capacity_bytes = 2 * PAGES * PB
    b.receipt.bank_epoch = 0x4C4C
    for i, sl in enumerate(slots):
        b.lane_index[i] = sl
        b.terminal[i] = 1 if sl in terminal else 0
    return b


def _ack(gh, sha, rid):
    return gh.PrepareAck(gh.PREPARE_ACK_ABI, (C.c_uint8 * 32)(*sha), 0x50414745, rid)


def test_leased_waves_publish_under_one_cohort_permit(gh, model):
    """paged_lease_token_txn.zig: one Bank publication permit fences a whole
    staged wave of leased lanes (its generation is the proposal's permit
    generation); commit advances the cohort's sequence once, a sink rejection
    or abort leaves it for the retry, a wrong sequence is refused before any
    permit; a lane whose terminal token the wave publishes is sealed with the
    wave's proposal and commit digests and reclaims from that seal."""
    sess = gh.Session(model, max_lanes=2, max_positions=MAXPOS, kv_dtype=gh.F16)
    try:
        bank = gh.LeaseBank(2, 16, 0x4C4C, kv_bytes=64 * PB, queue_slots=4)
        parent = bank.commit(bank.reserve(1, queue_slots=1))
        tree = bank.open_tree(parent, 2, 3, kv_bytes=16 * PB)
        scopes = [bank.open_scope(tree, 4 + i, 5 + i, kv_bytes=PAGES * PB) for i in range(2)]
        seq = C.c_uint64(0)
        bank.bind_session(tree, 6, 0x5E55)
        lks = []
        for lane in range(2):
            sess.begin(lane, seed=lane)
            lks.append(gh.LeasedKV(bank, tree, scopes[lane], sess, 6, 0x5E55, seq, lane=lane,
                                   binding_count=PAGES))
            sess.prefill_staged(lane, gh.synth_tokens(SEED, 10 + lane, TINY["vocab_size"], 20))
        assert tree.current.kv_bytes == 4 * PB
        print("leased waves: first tokens", flush=True)
        rc, _, _, _ = sess.step_prepare([0, 1], None, _wave_binding(gh, [0, 1], 5))
        assert rc == gh.INVALID_TRANSACTION and seq.value == 0  # not the cohort's sequence
        rc, prop, sha, toks = sess.step_prepare([0, 1], None, _wave_binding(gh, [0, 1], 0))
        assert rc == gh.OK and prop.resource_permit_generation == 1
        rc, _ = sess.step_commit(_ack(gh, sha, 1))
        assert rc == gh.OK and seq.value == 1
        toks = [int(t) for t in toks]
        # abort, then a rejected ack: the sequence stays, each retry takes a new permit
        rc, prop, sha, _ = sess.step_prepare([0, 1], toks, _wave_binding(gh, [0, 1], 1))
        assert rc == gh.OK and prop.resource_permit_generation == 2
        assert sess.step_abort() == gh.OK and seq.value == 1
        rc, prop, sha, _ = sess.step_prepare([0, 1], toks, _wave_binding(gh, [0, 1], 1))
        assert rc == gh.OK and prop.resource_permit_generation == 3
        rc, _ = sess.step_commit(_ack(gh, bytes(32), 2))
        assert rc == gh.INVALID_TRANSACTION and seq.value == 1
        for wave in range(14):  # wave 12 writes row 32: both lanes take a page in one wave
            terminal = (1,) if wave == 13 else ()
            rc, prop, sha, nxt = sess.step_prepare([0, 1], toks,
                                                   _wave_binding(gh, [0, 1], seq.value, terminal))
            assert rc == gh.OK
            rc, rec = sess.step_commit(_ack(gh, sha, 10 + wave))
            assert rc == gh.OK
            toks = [int(t) for t in nxt]
        assert seq.value == 15
        # 20 prompt rows + 14 decode rows (the first-token wave writes none):
        # 34 rows, three pages per lane
        assert tree.current.kv_bytes == 6 * PB
        seal, psha, csha = lks[1].terminal_seal()
        assert psha == sha and csha == bytes(rec.commit_sha256)
        assert seal.transaction_sequence == 14 and seal.terminal_token == toks[1]
        assert seal.bindings.count == 3
        assert lks[0].lifecycle() == "live" and lks[1].lifecycle() == "terminal_retained"
        with pytest.raises(gh.LeaseError) as e:
            lks[1].begin_reclaim(seal, 14)  # the reclaim comes after the terminal sequence
        assert e.value.reason == "InvalidTerminalSeal"
        freed = lks[1].begin_reclaim(seal, 15)
        lks[1].commit_reclaim(freed)
        assert tree.current.kv_bytes == 3 * PB
        # lane 0 publishes on alone; then teardown
        rc, prop, sha, nxt = sess.step_prepare([0], toks[:1], _wave_binding(gh, [0], 15))
        assert rc == gh.OK
        assert sess.step_commit(_ack(gh, sha, 99))[0] == gh.OK and seq.value == 16
        lks[0].reclaim_for_teardown(seq.value)
        assert tree.current.kv_bytes == 0
        for lk in lks:
            lk.close()
        bank.close_session(parent, 6, 0x5E55, seq.value)
        bank.close_tree(tree)
        bank.release(parent)
        assert not any(bank.snapshot()["used"].values())
    finally:
        sess.close()


def test_coordinator_gone_mid_wave_aborts_the_wave(gh, model):
    """A leased lane's coordinator destroyed between step_prepare and
    step_commit aborts the prepared wave: its permit goes back to the bank
    (the cohort's sequence stays), its rows are aborted, and the other lane
    publishes the next wave at the same sequence."""
    sess = gh.Session(model, max_lanes=2, max_positions=MAXPOS, kv_dtype=gh.F16)
    try:
        bank = gh.LeaseBank(2, 16, 0x4C4C, kv_bytes=64 * PB, queue_slots=4)
        parent = bank.commit(bank.reserve(1, queue_slots=1))
        tree = bank.open_tree(parent, 2, 3, kv_bytes=16 * PB)
        scopes = [bank.open_scope(tree, 4 + i, 5 + i, kv_bytes=PAGES * PB) for i in range(2)]
        seq = C.c_uint64(0)
        bank.bind_session(tree, 6, 0x5E55)
        lks = []
        for lane in range(2):
            sess.begin(lane, seed=lane)
            lks.append(gh.LeasedKV(bank, tree, scopes[lane], sess, 6, 0x5E55, seq, lane=lane,
                                   binding_count=PAGES))
            sess.prefill_staged(lane, gh.synth_tokens(SEED, 20 + lane, TINY["vocab_size"], 18))
        rc, _, sha, toks = sess.step_prepare([0, 1], None, _wave_binding(gh, [0, 1], 0))
        assert rc == gh.OK and sess.step_commit(_ack(gh, sha, 1))[0] == gh.OK
        toks = [int(t) for t in toks]
        root1 = sess.root(1)
        rc, _, sha, _ = sess.step_prepare([0, 1], toks, _wave_binding(gh, [0, 1], 1))
        assert rc == gh.OK
        print("coordinator gone mid-wave", flush=True)
        lks[0].close()  # lane 0's coordinator goes away inside the prepared wave
        rc, _ = sess.step_commit(_ack(gh, sha, 2))
        assert rc == gh.INVALID_TRANSACTION and seq.value == 1
        after = sess.root(1)
        assert (after.generation, after.committed_len) == (root1.generation, root1.committed_len)
        rc, _, sha, _ = sess.step_prepare([1], toks[1:], _wave_binding(gh, [1], 1))
        assert rc == gh.OK and sess.step_commit(_ack(gh, sha, 3))[0] == gh.OK
        assert seq.value == 2
        lks[1].reclaim_for_teardown(seq.value)
        lks[1].close()
    finally:
        sess.close()


def _v3_binding(gh, parent, slots, seq):
    b = _wave_binding(gh, slots, seq)
    C.memmove(C.byref(b.receipt), C.byref(parent), C.sizeof(b.receipt))
    return b


def _ack3(gh, sha, rid):
    return gh.PrepareAck(gh.PREPARE_ACK_V3_ABI, (C.c_uint8 * 32)(*sha), 0x50414745, rid)


def _troot(opub, t, side):
    return opub.root_bytes(getattr(t, f"root_{side}_generation"), getattr(t, f"root_{side}_len"),
                           getattr(t, f"root_{side}_pages"),
                           bytes(getattr(t, f"root_{side}_ownership_sha256")), t.cache_instance)


def _rbytes(opub, r):
    return opub.root_bytes(r.generation, r.committed_len, r.committed_pages,
                           bytes(r.ownership_sha256), r.cache_instance)


def test_leased_v3_waves_commit_tree_and_resources(gh, model):
    """ProposalV3 (paged_lease_token_txn.zig:107-180, Batch.begin :1117-1250,
    collectResourceSnapshot :765-896): each v3 wave's digest equals the
    oracle's over the returned record; its tree commitment is the cohort
    tree's redacted fields; each live lane's resource names its coordinator,
    cache instance, scope, the page-map root and v3 KV chain after the wave,
    the canonical logical-KV digest after a first or terminal row, the
    terminal seal's generation, and its binding summary and allocation set
    (equal to the coordinator's own and to the oracle's restatement over the
    lane's sidecar); a terminal-retained lane is committed from its seal and
    a reclaimed one by its seal's root. Slots are fixed, live lanes cannot
    sit out, lanes chain under one ABI, and the v3 ack / commit digests are
    the v3 ones."""
    import oracle as ora
    from oracle import publication as opub

    V = TINY["vocab_size"]
    sess = gh.Session(model, max_lanes=3, max_positions=MAXPOS, kv_dtype=gh.F16)
    try:
        bank = gh.LeaseBank(2, 16, 0x4C4C, kv_bytes=64 * PB, queue_slots=4)
        parent = bank.commit(bank.reserve(1, queue_slots=1))
        tree = bank.open_tree(parent, 2, 3, kv_bytes=16 * PB)
        scopes = [bank.open_scope(tree, 4 + i, 5 + i, kv_bytes=PAGES * PB) for i in range(2)]
        seq = C.c_uint64(0)
        bank.bind_session(tree, 6, 0x5E55)
        lks, outs = [], [[], []]
        slots = [2, 0]  # lane 0 publishes in slot 2, lane 1 in slot 0
        for lane in range(2):
            sess.begin(lane, seed=lane)
            lks.append(gh.LeasedKV(bank, tree, scopes[lane], sess, 6, 0x5E55, seq, lane=lane,
                                   binding_count=PAGES))
            sess.prefill_staged(lane, gh.synth_tokens(SEED, 30 + lane, V, 14))
        sess.begin(2, seed=9)
        sess.prefill_staged(2, gh.synth_tokens(SEED, 40, V, 5))
        rc, *_ = sess.step_prepare_v3([2], None, _v3_binding(gh, parent, [1], 0))
        assert rc == gh.INVALID_ARGUMENT  # v3 waves publish leased lanes only
        bad = _v3_binding(gh, parent, slots, 0)
        bad.receipt.integrity ^= 1
        rc, *_ = sess.step_prepare_v3([0, 1], None, bad)
        assert rc == gh.INVALID_TRANSACTION and seq.value == 0  # not the tree's parent

        def check_wave(prop, sha, lanes, toks, first, reasons):
            assert sha == opub.proposal_v3_sha256(prop)
            assert prop.abi_version == opub.PROPOSAL_V3_ABI
            assert prop.page_transition_abi == opub.PAGE_TRANSITION_V3_ABI
            assert prop.live_lane_count == len(lanes)
            assert prop.live_mask == sum(1 << slots[ln] for ln in lanes)
            assert bytes(prop.parent_receipt) == bytes(parent)
            t = prop.tree
            assert (t.tree_key, t.identity_generation, t.generation, t.structural_revision,
                    t.active_nodes, t.state_digest, t.token_integrity) == (
                tree.tree_key, tree.identity_generation, tree.generation,
                tree.structural_revision, tree.active_nodes, tree.state_digest, tree.integrity)
            assert bytes(t.current) == bytes(tree.current)
            for i, ln in enumerate(lanes):
                sl = slots[ln]
                r, lp = prop.resources[sl], prop.lanes[sl]
                tr = lp.kv_transition
                assert r.lane_index == sl and r.lifecycle == gh.LIFECYCLE_LIVE
                assert r.scope_index == scopes[ln].node_index
                assert r.scope_generation == scopes[ln].generation
                assert r.cache_instance == sess.root(ln).cache_instance == tr.cache_instance
                assert _rbytes(opub, r.root) == _troot(opub, tr, "after")
                assert bytes(r.binding_summary) == bytes(lks[ln].binding_summary())
                alloc = lks[ln].allocation_set()
                assert bytes(r.allocation_set) == bytes(alloc)
                assert bytes(alloc.sha256) == opub.allocation_set_sha256(
                    r.coordinator_instance, r.cache_instance, lks[ln].scope, lks[ln].bindings)
                assert bytes(lp.output_sha256) == ora.token_sequence_sha256(
                    outs[ln] + [int(toks[i])])
                assert lp.terminal_reason == reasons[i]
                assert bool(r.has_terminal_generation) == bool(reasons[i])
                assert bool(r.has_canonical_after) == (first or bool(reasons[i]))
                if first:
                    assert bytes(r.canonical_after_sha256) == sess.kv_sha256(ln)
                    assert bytes(tr.state_chain_after) == opub.initial_state_chain_v3(
                        bytes(r.canonical_after_sha256), _troot(opub, tr, "after"))
                else:
                    assert bytes(tr.state_chain_after) == opub.appended_state_chain_v3(
                        bytes(tr.state_chain_before), _troot(opub, tr, "before"),
                        _troot(opub, tr, "after"), tr.cache_instance, tr.logical_page,
                        tr.page_ownership_generation, tr.row_txn_generation,
                        bytes(tr.row_payload_sha256))
                assert bytes(r.kv_state_chain_after) == bytes(tr.state_chain_after)

        print("v3 leased waves: first tokens", flush=True)
        rc, prop, sha, toks = sess.step_prepare_v3([0, 1], None, _v3_binding(gh, parent, slots, 0))
        assert rc == gh.OK
        check_wave(prop, sha, [0, 1], toks, True, [0, 0])
        rc, _ = sess.step_commit(_ack(gh, sha, 1))  # a v1 ack does not acknowledge a v3 wave
        assert rc == gh.INVALID_TRANSACTION and seq.value == 0
        rc, prop, sha, toks = sess.step_prepare_v3([0, 1], None, _v3_binding(gh, parent, slots, 0))
        assert rc == gh.OK
        ack = _ack3(gh, sha, 1)
        rc, rec = sess.step_commit(ack)
        assert rc == gh.OK and seq.value == 1
        assert bytes(rec.commit_sha256) == opub.commit_v3_sha256(
            sha, ack.abi_version, sha, ack.sink_epoch, ack.reservation_id)
        for ln in range(2):
            outs[ln].append(int(toks[ln]))
        toks = [int(t) for t in toks]
        # slots are fixed, live lanes join every wave, lanes chain under one ABI
        rc, *_ = sess.step_prepare_v3([0, 1], toks, _v3_binding(gh, parent, [0, 2], 1))
        assert rc == gh.INVALID_ARGUMENT
        rc, *_ = sess.step_prepare_v3([0], toks[:1], _v3_binding(gh, parent, [2], 1))
        assert rc == gh.INVALID_TRANSACTION
        rc, *_ = sess.step_prepare([0, 1], toks, _wave_binding(gh, slots, 1))
        assert rc == gh.INVALID_TRANSACTION and seq.value == 1
        for wave in range(4):  # wave 2 writes row 16: both lanes take a page
            reasons = [0, 1 + gh.TERMINAL_MAX_TOKENS] if wave == 3 else [0, 0]
            rc, prop, sha, nxt = sess.step_prepare_v3([0, 1], toks,
                                                      _v3_binding(gh, parent, slots, seq.value),
                                                      terminal_reason=reasons)
            assert rc == gh.OK
            check_wave(prop, sha, [0, 1], nxt, False, reasons)
            rc, rec = sess.step_commit(_ack3(gh, sha, 10 + wave))
            assert rc == gh.OK
            for ln in range(2):
                outs[ln].append(int(nxt[ln]))
            toks = [int(t) for t in nxt]
        assert seq.value == 5
        term = prop.resources[slots[1]]
        seal, psha, csha = lks[1].terminal_seal()
        assert psha == sha and csha == bytes(rec.commit_sha256)
        assert seal.terminal_reason == gh.TERMINAL_MAX_TOKENS and seal.terminal_token == toks[1]
        assert seal.generation == term.terminal_generation
        assert bytes(seal.logical_kv_sha256) == bytes(term.canonical_after_sha256)
        assert bytes(seal.logical_kv_sha256) == sess.kv_sha256(1)
        assert seal.coordinator_instance == term.coordinator_instance
        chain1 = bytes(prop.lanes[slots[1]].kv_transition.state_chain_after)
        # lane 1 retired: lane 0 publishes alone, lane 1 committed from its seal
        rc, prop, sha, nxt = sess.step_prepare_v3([0], toks[:1], _v3_binding(gh, parent, [2], 5))
        assert rc == gh.OK
        check_wave(prop, sha, [0], nxt, False, [0])
        r1 = prop.resources[0]
        assert r1.lifecycle == gh.LIFECYCLE_TERMINAL_RETAINED
        assert bytes(r1.root) == bytes(seal.root) and bytes(r1.kv_state_chain_after) == chain1
        assert r1.has_canonical_after and r1.has_binding_summary and not r1.has_terminal_generation
        assert bytes(r1.canonical_after_sha256) == bytes(seal.logical_kv_sha256)
        assert bytes(r1.binding_summary) == bytes(seal.bindings)
        assert sess.step_commit(_ack3(gh, sha, 20))[0] == gh.OK and seq.value == 6
        outs[0].append(int(nxt[0]))
        toks = [int(nxt[0])]
        freed = lks[1].begin_reclaim(seal, 6)
        lks[1].commit_reclaim(freed)
        rc, prop, sha, nxt = sess.step_prepare_v3([0], toks, _v3_binding(gh, parent, [2], 6))
        assert rc == gh.OK
        check_wave(prop, sha, [0], nxt, False, [0])
        r1 = prop.resources[0]
        assert r1.lifecycle == gh.LIFECYCLE_RECLAIMED and bytes(r1.root) == bytes(seal.root)
        assert not r1.has_binding_summary and r1.allocation_set.count == 0
        assert r1.allocation_set.abi_version == opub.ALLOCATION_SET_ABI
        assert sess.step_commit(_ack3(gh, sha, 21))[0] == gh.OK and seq.value == 7
        lks[0].reclaim_for_teardown(seq.value)
        assert tree.current.kv_bytes == 0
        for lk in lks:
            lk.close()
        bank.close_session(parent, 6, 0x5E55, seq.value)
        bank.close_tree(tree)
        bank.release(parent)
    finally:
        sess.close()
