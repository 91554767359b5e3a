"""BASELINE config 5 at its workload on the GPU: 32 lanes of the
Qwen2.5-7B-shaped model (tests/golden/q7b_case.py) admitted to LaneWeave
with the bench's admission set (bench.c5_workload: prompt lengths drawn from
U[64, 4096] by seed, weights 1..4, each lane's fp16 KV pages charged to the
scheduler's Bank), prefilled, then served in LaneWeave device waves
(glacier_hip_session_lane_weave_wave: the next IWRR quanta of distinct lanes
in one device step, committed in scheduler order) through the eligible
argmax over an all-ones mask of all 152064 ids, 16 decode quanta per lane.

Checks (lane_weave_qos.zig:1196-1270 serveOne, sampling.zig:55-105):
  * every lane's 17 tokens equal its own batch-1 run (a fresh one-lane
    session, plain greedy argmax), so batching lanes of 64-4096 positions
    into one wave changes no lane's tokens;
  * the scheduler's event chain equals the oracle scheduler's
    (oracle/lane_weave.py) event for event: every admission, every service
    quantum in wave order, every retirement and the close.
f32 activations (the reference's int4_activation = .f32) make the model's
arithmetic continuous, so batch-1 and batched steps agree token for token;
the Q8 mode's batch-1 parity is covered by tests/test_gpu_7b.py.
"""
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(HERE, "golden"), os.path.dirname(HERE)]
import q7b_case  # noqa: E402

CFG = q7b_case.Q7B
V = CFG["vocab_size"]
GEN = 17  # the first token from prefill + 16 decode quanta


@pytest.fixture(scope="module")
def q7b(gh, gctx):
    print("building the 7B test model", flush=True)
    host = q7b_case.make_host(gh)
    m = gh.Model(gctx, CFG)
    m.set_from_host(host)
    del host
    yield m
    m.close()


def test_c5_lane_weave_waves_match_batch1_and_oracle_chain(gh, q7b):
    import bench
    from oracle import lane_weave as olw

    wl = bench.c5_workload(CFG, gen=GEN)
    lanes, plens = wl["lanes"], wl["plens"]
    assert lanes == 32 and sum(p >= 2048 for p in plens) >= 8
    prompts = [gh.synth_tokens(bench.SEED, 0x4C414E45 + i, V, plens[i]) for i in range(lanes)]
    W = (V + 63) // 64
    elig = np.full((lanes, W), ~np.uint64(0), np.uint64)
    if V % 64:
        elig[:, -1] = np.uint64((1 << (V % 64)) - 1)

    # batch-1 runs, one fresh lane each
    want = []
    one = gh.Session(q7b, max_lanes=1, max_positions=wl["prompt_hi"] + GEN + 8, kv_dtype=gh.F16,
                     layer_activation=gh.ACT_F32, head_activation=gh.ACT_F32, prefill_chunk=2048)
    try:
        for i in range(lanes):
            one.begin(0, seed=i)
            t = [one.prefill(0, prompts[i])]
            for _ in range(GEN - 1):
                t.append(int(one.step([0], [t[-1]])[0]))
            want.append(t)
        print(f"batch-1 runs done (prompts {min(plens)}..{max(plens)})", flush=True)
    finally:
        one.close()

    sess = gh.Session(q7b, max_lanes=lanes, max_positions=wl["prompt_hi"] + GEN + 8,
                      kv_dtype=gh.F16, total_pages=sum(wl["pages"]), prefill_chunk=2048,
                      layer_activation=gh.ACT_F32, head_activation=gh.ACT_F32)
    sched = gh.LaneWeave(lanes, wl["bank"], bank_epoch=wl["bank_epoch"],
                         scheduler_epoch=wl["scheduler_epoch"], max_weight=wl["max_weight"])
    ref = olw.Scheduler(olw.Bank(lanes, olw.limits(**wl["bank"]), wl["bank_epoch"]), lanes,
                        wl["scheduler_epoch"], bytes([0xA5]) + bytes(31), wl["max_weight"],
                        1_000_000, 1_000_000)
    try:
        tokens = np.zeros(lanes, np.uint32)
        got = [[] for _ in range(lanes)]
        for i, sp in enumerate(wl["specs"]):
            ok, _, ev = sched.admit(gh.LaneWeave.spec(
                sp["tenant_key"], sp["request_key"], sp["request_generation"],
                sp["resource_owner_key"], sp["weight"], sp["work_quanta"], sp["deadline_tick"],
                sp["claim"]))
            r_ok, _, r_ev = ref.admit(dict(sp, claim=olw.claim(**sp["claim"])))
            assert ok and r_ok and bytes(ev.event_sha256) == r_ev["event_sha256"]
            sess.begin(i, seed=i)
            tokens[i] = sess.prefill(i, prompts[i])
            got[i].append(int(tokens[i]))
        print("32 lanes admitted and prefilled", flush=True)
        waves = sizes = 0
        while True:
            try:
                slots, evs = sched.wave(sess, list(range(lanes)), tokens, elig)
            except gh.GlacierHipError as e:
                assert e.code == gh.NO_RUNNABLE
                break
            waves += 1
            sizes += len(slots)
            assert len(set(slots)) == len(slots)
            for slot, ev in zip(slots, evs):
                got[slot].append(int(tokens[slot]))
                assert bytes(ev.event_sha256) == ref.serve_one()["event_sha256"]
            for slot, ev in zip(slots, evs):
                if ev.remaining_after == 0:
                    want_retire = ref.retire(ref.handle_for(slot))["event_sha256"]
                    rc, rev = sched.retire(ev.handle)
                    assert rc == 0 and bytes(rev.event_sha256) == want_retire
        rc, cev = sched.close()
        assert rc == 0 and bytes(cev.event_sha256) == ref.close()["event_sha256"]
        assert sizes == lanes * (GEN - 1) and waves < sizes
        bad = [i for i in range(lanes) if got[i] != want[i]]
        print(f"{waves} waves (mean {sizes / waves:.1f} lanes); lanes differing from their "
              f"batch-1 run: {bad}", flush=True)
        assert not bad
    finally:
        sess.close()
