"""Staged per-token publication (paged_token_txn.zig:346-600) through the C
ABI on the tiny model: glacier_hip_session_prefill_staged, step_prepare,
step_commit and step_abort.

Checked against the oracle: the proposal digest (oracle/publication.py),
each lane's page-map root transition (oracle/paged_kv.py replaying the same
begin / commit / abort sequence), the KV state chain (initialStateChain /
appendedStateChain over the committed rows read back), the greedy tokens
(the oracle's generate), and the reference's own transaction tests:
  * 'commits exact root transitions through one batch fence' (:1384-1435)
  * 'sink rejection restores roots and permits generation-fenced retry' (:1437-1490)
  * 'page-boundary ack rejection reuses allocation with fresh ownership' (:1512-1600)
"""
import ctypes as C

import numpy as np
import pytest

from oracle import paged_kv as opk
from oracle import publication as opub

pytestmark = pytest.mark.gpu

TINY = dict(num_layers=2, dim=256, hidden_dim=512, num_heads=4, num_kv_heads=2, head_dim=64,
            vocab_size=4096, group_size=32, rms_eps=1e-6, rope_theta=1e6)
SEED = 0x5EED
KVD = TINY["num_kv_heads"] * TINY["head_dim"]
MAXPOS = 64


@pytest.fixture(scope="module")
def tiny(gh, gctx, ora):
    host = gh.random_model_host(TINY, SEED)
    for L in host["layers"]:
        L["input_norm"] = (L["input_norm"] + 1.0).astype(np.float32)
        L["post_attn_norm"] = (L["post_attn_norm"] + 1.0).astype(np.float32)
    host["final_norm"] = (host["final_norm"] + 1.0).astype(np.float32)
    om = ora.OracleModel(TINY, host)
    m = gh.Model(gctx, TINY)
    m.set_from_host(host)
    yield om, m
    m.close()


def _capacity():
    pages = -(-MAXPOS // 16)
    return pages * TINY["num_layers"] * 2 * 16 * KVD * 4 + pages * 16


def _binding(gh, slots, seq, terminal=()):
    b = gh.PublicationBinding()
    b.execution_abi = 0x5042544553540001
    b.request_epoch = 0x7010
    b.transaction_sequence = seq
    b.resource_permit_generation = 100 + seq
    b.kv_capacity_bytes = 4 * _capacity()
    b.receipt.bank_epoch = 701
    b.receipt.slot_index = 0
    b.receipt.generation = 1
    b.receipt.owner_key = 701 ^ 0x55AA
    b.receipt.claim.kv_bytes = 4 * _capacity()
    b.receipt.claim.queue_slots = 4
    b.receipt.integrity = 0x1234
    for i, sl in enumerate(slots):
        b.lane_index[i] = sl
        b.terminal[i] = 1 if sl in terminal else 0
    return b


def _ack(gh, sha, rid):
    return gh.PrepareAck(gh.PREPARE_ACK_ABI, (C.c_uint8 * 32)(*sha), 0x50414745, rid)


def _root(sess, lane):
    r = sess.root(lane)
    return opub.root_bytes(r.generation, r.committed_len, r.committed_pages, r.ownership_sha256,
                           r.cache_instance)


def _row_digest(sess, lane, pos):
    rows = [sess.kv_row(lane, l, v, pos, KVD) for l in range(TINY["num_layers"]) for v in (0, 1)]
    return opub.row_payload_sha256(TINY["num_layers"], KVD, pos, rows)


def _check_transition(t, before, after, inst):
    assert t.cache_instance == inst
    assert (t.root_before_generation, t.root_before_len, t.root_before_pages,
            bytes(t.root_before_ownership_sha256)) == (before.generation, before.committed_len,
                                                       before.committed_pages,
                                                       before.ownership_sha256)
    assert (t.root_after_generation, t.root_after_len, t.root_after_pages,
            bytes(t.root_after_ownership_sha256)) == (after.generation, after.committed_len,
                                                      after.committed_pages,
                                                      after.ownership_sha256)


def test_staged_waves_publish_the_oracle_tokens_and_chains(gh, tiny):
    om, m = tiny
    V = TINY["vocab_size"]
    prompts = [gh.synth_tokens(SEED, 80 + i, V, n) for i, n in enumerate([5, 16, 21, 31])]
    waves = 8
    wants = [om.generate(p, waves + 1) for p in prompts]
    sess = gh.Session(m, max_lanes=4, max_positions=MAXPOS)
    try:
        refs, chains = [], []
        for i, p in enumerate(prompts):
            sess.begin(i)
            sess.prefill_staged(i, p)
            ref = opk.PagedKVCache(TINY["num_layers"], KVD, MAXPOS,
                                   instance=sess.root(i).cache_instance)
            for _ in range(len(p)):
                ref.commit_row(ref.begin_row())
            refs.append(ref)
            assert sess.state(i).published_tokens == 0  # held back
        # first wave: no KV row, initial transitions
        rc, prop, sha, first = sess.step_prepare([0, 1, 2, 3], None, _binding(gh, [0, 1, 2, 3], 0))
        assert rc == 0
        assert sha == opub.proposal_sha256(prop)
        assert (prop.live_mask, prop.live_lane_count) == (0b1111, 4)
        for i in range(4):
            lp = prop.lanes[i]
            t = lp.kv_transition
            kv = sess.kv_sha256(i)
            assert lp.has_kv_transition == 0 and lp.step_index == 0
            assert lp.kv_before == lp.kv_after == len(prompts[i]) == lp.prompt_len
            assert bytes(t.initial_logical_kv_sha256) == kv
            chain = opub.initial_state_chain(kv, _root(sess, i))
            assert bytes(t.state_chain_before) == bytes(t.state_chain_after) == chain
            assert (lp.output_before, lp.output_after) == (0, 1)
            assert (lp.sampling_calls_before, lp.sampling_calls_after) == (0, 1)
            assert lp.token_id == first[i] == wants[i][0][0]
            chains.append(chain)
        rc, rec = sess.step_commit(_ack(gh, sha, 1))
        assert rc == 0
        assert bytes(rec.commit_sha256) == opub.commit_sha256(sha, gh.PREPARE_ACK_ABI, sha,
                                                               0x50414745, 1)
        toks = [[int(x)] for x in first]
        for w in range(1, waves + 1):
            roots_before = [refs[i].root() for i in range(4)]
            rc, prop, sha, nxt = sess.step_prepare([0, 1, 2, 3], [t[-1] for t in toks],
                                                   _binding(gh, [0, 1, 2, 3], w))
            assert rc == 0 and sha == opub.proposal_sha256(prop)
            marks = [refs[i].begin_row() for i in range(4)]
            for i in range(4):
                lp = prop.lanes[i]
                t = lp.kv_transition
                before, after, installs = refs[i].prepare_commit(marks[i])
                assert before == roots_before[i]
                _check_transition(t, before, after, refs[i].instance_id)
                assert t.row_txn_generation == marks[i].generation
                assert t.page_ownership_generation == marks[i].ownership_generation
                assert (t.logical_page, bool(t.installs_new_page)) == (marks[i].logical_page,
                                                                       installs)
                assert lp.has_kv_transition == 1 and lp.step_index == w
                assert bytes(t.state_chain_before) == chains[i]
                assert lp.token_id == nxt[i]
                # nothing is visible before the commit
                assert sess.root(i).committed_len == before.committed_len
                assert sess.state(i).published_tokens == w
            rc, _ = sess.step_commit(_ack(gh, sha, w + 1))
            assert rc == 0
            for i in range(4):
                refs[i].commit_row(marks[i])
                t = prop.lanes[i].kv_transition
                digest = _row_digest(sess, i, marks[i].base_len)
                assert bytes(t.row_payload_sha256) == digest
                chain = opub.appended_state_chain(
                    chains[i], opub.root_bytes(t.root_before_generation, t.root_before_len,
                                               t.root_before_pages, t.root_before_ownership_sha256,
                                               t.cache_instance),
                    opub.root_bytes(t.root_after_generation, t.root_after_len,
                                    t.root_after_pages, t.root_after_ownership_sha256,
                                    t.cache_instance),
                    t.cache_instance, t.logical_page, t.page_ownership_generation,
                    t.row_txn_generation, digest)
                assert bytes(t.state_chain_after) == chain
                chains[i] = chain
                toks[i].append(int(nxt[i]))
        for i in range(4):
            assert toks[i] == wants[i][0].tolist(), i
            st = sess.state(i)
            assert bytes(st.output_sha256) == wants[i][3]
            assert st.sampling_calls == waves + 1 and st.published_tokens == waves + 1
            r = sess.root(i)
            assert (r.generation, r.committed_len, r.committed_pages,
                    bytes(r.ownership_sha256)) == refs[i].root().key()[2:]
    finally:
        sess.close()


def test_sink_rejection_publishes_nothing_and_retry_takes_fresh_generations(gh, tiny):
    """A rejected proposal (the host's sink refused it, so it aborts) leaves
    roots, RNG, sampler counter and outputs unchanged; the retry's row
    transaction and, at a page boundary, its page ownership generation are
    fresh while the page payload is reused."""
    om, m = tiny
    prompt = gh.synth_tokens(SEED, 90, TINY["vocab_size"], 16)
    want = om.generate(prompt, 3)[0].tolist()
    sess = gh.Session(m, max_lanes=1, max_positions=MAXPOS)
    try:
        sess.begin(0)
        sess.prefill_staged(0, prompt)
        rc, prop, sha, first = sess.step_prepare([0], None, _binding(gh, [2], 0))
        assert rc == 0 and prop.live_mask == 0b100 and prop.lanes[2].token_id == want[0]
        assert sess.step_commit(_ack(gh, sha, 1))[0] == 0
        root0, state0 = bytes(sess.root(0)), bytes(sess.state(0))
        # row 16 installs logical page 1; the sink rejects
        rc, rej, rsha, _ = sess.step_prepare([0], [int(first[0])], _binding(gh, [2], 1))
        assert rc == 0
        rt = rej.lanes[2].kv_transition
        assert rt.installs_new_page == 1 and rt.logical_page == 1
        page = sess.page_of(0, 1)
        assert sess.step_abort() == 0
        assert bytes(sess.root(0)) == root0 and bytes(sess.state(0)) == state0
        assert sess.page_of(0, 1) == page >= 0 and sess.page_generation(0, 1) == 0
        # the retry: same payload, fresh row and ownership generations
        rc, ok, osha, nxt = sess.step_prepare([0], [int(first[0])], _binding(gh, [2], 1))
        assert rc == 0
        ot = ok.lanes[2].kv_transition
        assert ot.row_txn_generation > rt.row_txn_generation
        assert ot.page_ownership_generation > rt.page_ownership_generation
        assert ot.root_after_generation > rt.root_after_generation
        assert osha != rsha
        assert sess.page_of(0, 1) == page
        assert sess.step_commit(_ack(gh, osha, 2))[0] == 0
        assert sess.page_generation(0, 1) == ot.page_ownership_generation
        assert int(nxt[0]) == want[1]
        # an invalid ack aborts: nothing published, the next wave proceeds
        root1, state1 = bytes(sess.root(0)), bytes(sess.state(0))
        rc, p3, sha3, n3 = sess.step_prepare([0], [int(nxt[0])], _binding(gh, [2], 2, terminal=(2,)))
        assert rc == 0 and p3.lanes[2].terminal == 1
        bad = bytearray(sha3)
        bad[0] ^= 1
        assert sess.step_commit(_ack(gh, bytes(bad), 3))[0] == gh.INVALID_TRANSACTION
        assert bytes(sess.root(0)) == root1 and bytes(sess.state(0)) == state1
        assert sess.step_commit(_ack(gh, sha3, 3))[0] == gh.INVALID_TRANSACTION  # already aborted
        rc, p3, sha3, n3 = sess.step_prepare([0], [int(nxt[0])], _binding(gh, [2], 2, terminal=(2,)))
        assert rc == 0
        # while a wave is prepared every other step is fenced
        assert sess.step([0], [int(nxt[0])], raise_on_error=False)[0] == gh.TRANSACTION_ACTIVE
        assert sess.step_commit(_ack(gh, sha3, 4))[0] == 0
        assert int(n3[0]) == want[2]
        assert sess.state(0).published_tokens == 3
        # a terminal lane accepts no further wave
        assert sess.step_prepare([0], [int(n3[0])], _binding(gh, [2], 3))[0] == gh.INVALID_TRANSACTION
    finally:
        sess.close()
