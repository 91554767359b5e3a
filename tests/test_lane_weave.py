"""LaneWeave QoS v1 (BASELINE config 5's scheduler): the oracle restatement
and the product scheduler (glacier_hip_lane_weave_*, host C++ in
libglacier_hip.so) against the reference's own known answers, and against
each other on random traces.

Reference known answers (src/core/lane_weave_qos.zig):
  * IWRR golden order and final close-event SHA-256 (:4436-4474)
  * deadline_infeasible before Bank mutation (:4476-4493)
  * projection budgets: quanta, operations, scan (:4495-4554)
  * resource capacity (:4556-4570)
  * stale handle after slot reuse (:4572-4586)
"""
import random

import pytest

from oracle import lane_weave as lw

GOLDEN_ORDER = [1, 2, 3, 2, 3, 3, 3, 1, 2, 3, 2, 3, 3, 3]
GOLDEN_CLOSE = "9cffc54d7a146c3a69cebb386a189dd1d3efffec3fba25c8ecadef8ab3c96785"


# ---------------------------------------------------------------- oracle ----
def test_oracle_iwrr_golden_order_and_close_hash():
    f = lw.test_fixture(3, 4)
    for key, weight, work in ((1, 1, 2), (2, 2, 4), (3, 4, 8)):
        ok, _, ev = f.admit(lw.test_spec(key, weight, work, 0))
        assert ok and ev["kind"] == lw.ADMISSION_ACCEPTED
    order = []
    for _ in GOLDEN_ORDER:
        ev = f.serve_one()
        assert ev["kind"] == lw.SERVICE
        assert ev["wait_quanta"] <= ev["maximum_service_gap"]
        assert ev["event_sha256"] == lw.event_sha256(ev)
        order.append(ev["handle"]["tenant_key"])
    assert order == GOLDEN_ORDER
    for i in range(3):
        f.retire(f.handle_for(i))
    final = f.close()
    assert final["kind"] == lw.CLOSE
    assert final["event_sha256"].hex() == GOLDEN_CLOSE
    assert lw.claim_is_zero(f.bank.used) and f.bank.committed_receipts() == 0


def _bank_state(f):
    return (dict(f.bank.used), [dict(s) for s in f.bank.slots], f.bank.next_generation)


def test_oracle_rejects_infeasible_deadline_before_bank_mutation():
    f = lw.test_fixture(2, 2)
    assert f.admit(lw.test_spec(1, 1, 2, 2))[0]
    before = _bank_state(f)
    ok, _, ev = f.admit(lw.test_spec(2, 1, 1, 1))
    assert not ok and ev["rejection_reason"] == lw.DEADLINE_INFEASIBLE
    assert _bank_state(f) == before


@pytest.mark.parametrize("cap,mw,pq,po,spec", [
    (1, 1, 2, 100, (1, 1, 3, 10)),     # quanta budget
    (8, 8, 100, 32, (1, 1, 4, 20)),    # operation budget
    (8, 8, 100, 1, (1, 1, 1, 0)),      # scan budget
])
def test_oracle_projection_budgets_reject_before_bank_mutation(cap, mw, pq, po, spec):
    f = lw.test_fixture(cap, mw, pq, po)
    before = _bank_state(f)
    ok, _, ev = f.admit(lw.test_spec(*spec))
    assert not ok and ev["rejection_reason"] == lw.PROJECTION_LIMIT
    assert _bank_state(f) == before


def test_oracle_rejects_resource_capacity():
    f = lw.test_fixture(2, 2)
    sp = lw.test_spec(1, 1, 1, 0)
    sp["claim"]["kv_bytes"] = (1 << 20) + 1
    before = _bank_state(f)
    ok, _, ev = f.admit(sp)
    assert not ok and ev["rejection_reason"] == lw.RESOURCE_LIMIT
    assert _bank_state(f) == before


def test_oracle_stale_handle_cannot_cancel_reused_slot():
    f = lw.test_fixture(1, 1)
    ok, first, _ = f.admit(lw.test_spec(1, 1, 1, 0))
    f.cancel(first)
    ok, second, _ = f.admit(lw.test_spec(2, 1, 1, 0))
    assert second["slot_generation"] != first["slot_generation"]
    with pytest.raises(lw.LaneWeaveError, match="StaleHandle"):
        f.cancel(first)
    f.cancel(second)
    f.close()


# --------------------------------------------------------------- product ----
FIXTURE_LIMITS = lambda cap: dict(host_bytes=1 << 20, kv_bytes=1 << 20, queue_slots=cap)  # noqa: E731


def _product(gh, cap, mw, pq=10_000, po=1_000_000):
    return gh.LaneWeave(cap, FIXTURE_LIMITS(cap), bank_epoch=0x42414E4B,
                        scheduler_epoch=0x51534553, challenge=bytes([0xA5]) + bytes(31),
                        max_weight=mw, max_projection_quanta=pq, max_projection_operations=po)


def _pspec(gh, sp):
    return gh.LaneWeave.spec(sp["tenant_key"], sp["request_key"], sp["request_generation"],
                             sp["resource_owner_key"], sp["weight"], sp["work_quanta"],
                             sp["deadline_tick"], {k: v for k, v in sp["claim"].items() if v})


def test_product_iwrr_golden_order_and_close_hash(gh):
    p = _product(gh, 3, 4)
    for key, weight, work in ((1, 1, 2), (2, 2, 4), (3, 4, 8)):
        ok, _, ev = p.admit(_pspec(gh, lw.test_spec(key, weight, work, 0)))
        assert ok and ev.kind == lw.ADMISSION_ACCEPTED
    order = []
    for _ in GOLDEN_ORDER:
        ev = p.serve_one()
        assert ev.kind == lw.SERVICE and ev.wait_quanta <= ev.maximum_service_gap
        order.append(ev.handle.tenant_key)
    assert order == GOLDEN_ORDER
    for i in range(3):
        rc, _ = p.retire(p.slot(i)[0])
        assert rc == 0
    rc, final = p.close()
    assert rc == 0 and bytes(final.event_sha256).hex() == GOLDEN_CLOSE


@pytest.mark.parametrize("cap,mw,pq,po,first,spec,reason", [
    (2, 2, 10_000, 1_000_000, (1, 1, 2, 2), (2, 1, 1, 1), lw.DEADLINE_INFEASIBLE),
    (1, 1, 2, 100, None, (1, 1, 3, 10), lw.PROJECTION_LIMIT),
    (8, 8, 100, 32, None, (1, 1, 4, 20), lw.PROJECTION_LIMIT),
    (8, 8, 100, 1, None, (1, 1, 1, 0), lw.PROJECTION_LIMIT),
])
def test_product_rejections_match_reference(gh, cap, mw, pq, po, first, spec, reason):
    p = _product(gh, cap, mw, pq, po)
    if first:
        assert p.admit(_pspec(gh, lw.test_spec(*first)))[0]
    ok, h, ev = p.admit(_pspec(gh, lw.test_spec(*spec)))
    assert not ok and h is None
    assert ev.kind == lw.ADMISSION_REJECTED and ev.rejection_reason == reason
    assert list(ev.bank_used_before.__reduce__()[1]) == list(ev.bank_used_after.__reduce__()[1])


def test_product_resource_limit_and_stale_handle(gh):
    p = _product(gh, 2, 2)
    sp = lw.test_spec(1, 1, 1, 0)
    sp["claim"]["kv_bytes"] = (1 << 20) + 1
    ok, _, ev = p.admit(_pspec(gh, sp))
    assert not ok and ev.rejection_reason == lw.RESOURCE_LIMIT
    q = _product(gh, 1, 1)
    ok, first, _ = q.admit(_pspec(gh, lw.test_spec(1, 1, 1, 0)))
    assert q.cancel(first)[0] == 0
    ok, second, _ = q.admit(_pspec(gh, lw.test_spec(2, 1, 1, 0)))
    assert second.slot_generation != first.slot_generation
    assert q.cancel(first)[0] == gh.STALE_HANDLE
    assert q.cancel(second)[0] == 0
    assert q.close()[0] == 0


def test_product_rejects_malformed_spec_without_event(gh):
    p = _product(gh, 2, 2)
    head = p.chain_head()
    bad = lw.test_spec(1, 3, 1, 0)  # weight above max_weight
    with pytest.raises(gh.GlacierHipError):
        p.admit(_pspec(gh, bad))
    assert p.chain_head() == head


def _random_trace(seed, cap=6, steps=400):
    """A random mix of admissions (weights, deadlines, oversize claims,
    duplicate tenants), services, retires and cancels."""
    rng = random.Random(seed)
    ops, next_key = [], 1
    for _ in range(steps):
        r = rng.random()
        if r < 0.25:
            key = next_key if rng.random() < 0.9 else max(1, next_key - 1)
            next_key += 1
            deadline = 0 if rng.random() < 0.6 else rng.randint(1, 60)
            ops.append(("admit", key, rng.randint(1, 4), rng.randint(1, 12), deadline,
                        rng.random() < 0.05))
        elif r < 0.85:
            ops.append(("serve",))
        elif r < 0.95:
            ops.append(("retire", rng.randrange(cap)))
        else:
            ops.append(("cancel", rng.randrange(cap)))
    return ops


@pytest.mark.parametrize("seed", range(6))
def test_product_matches_oracle_on_random_traces(gh, seed):
    cap, mw = 6, 4
    o = lw.test_fixture(cap, mw, 200, 100_000)
    p = _product(gh, cap, mw, 200, 100_000)
    n_events = 0
    for op in _random_trace(seed, cap):
        if op[0] == "admit":
            _, key, weight, work, deadline, big = op
            sp = lw.test_spec(key, weight, work, deadline)
            if big:
                sp["claim"]["kv_bytes"] = 1 << 19
            try:
                o_ok, o_h, o_ev = o.admit(sp)
            except lw.LaneWeaveError:  # e.g. a deadline already in the past
                with pytest.raises(gh.GlacierHipError):
                    p.admit(_pspec(gh, sp))
                continue
            p_ok, p_h, p_ev = p.admit(_pspec(gh, sp))
            assert o_ok == p_ok
            assert bytes(p_ev.event_sha256) == o_ev["event_sha256"]
        elif op[0] == "serve":
            plan = p.plan_wave(cap)
            try:
                o_ev = o.serve_one()
            except lw.LaneWeaveError:
                with pytest.raises(gh.GlacierHipError):
                    p.serve_one()
                assert plan == []
                continue
            p_ev = p.serve_one()
            assert plan and plan[0] == p_ev.handle.slot_index
            assert bytes(p_ev.event_sha256) == o_ev["event_sha256"]
        else:
            idx = op[1]
            handle = o.handle_for(idx)
            try:
                o_ev = o.retire(handle) if op[0] == "retire" else o.cancel(handle)
            except lw.LaneWeaveError:
                ph = p.slot(idx)[0]
                rc, _ = p.retire(ph) if op[0] == "retire" else p.cancel(ph)
                assert rc == gh.STALE_HANDLE
                continue
            ph = p.slot(idx)[0]
            rc, p_ev = p.retire(ph) if op[0] == "retire" else p.cancel(ph)
            assert rc == 0 and bytes(p_ev.event_sha256) == o_ev["event_sha256"]
        n_events += 1
        assert p.chain_head() == o.chain_head
    assert n_events > 100


@pytest.mark.parametrize("weights", [(1, 1, 1, 1), (1, 2, 4, 3), (4, 4, 1, 2, 3, 1, 2)])
def test_plan_wave_is_the_next_serial_selections(gh, weights):
    """A planned wave lists exactly the slots the following serve_one calls
    select, with no slot twice; committing it reproduces the serial chain."""
    cap = len(weights)
    p = _product(gh, cap, 4)
    o = lw.test_fixture(cap, 4)
    for i, w in enumerate(weights):
        sp = lw.test_spec(i + 1, w, 3 + 2 * i, 0)
        assert p.admit(_pspec(gh, sp))[0] and o.admit(sp)[0]
    while True:
        plan = p.plan_wave(cap)
        if not plan:
            break
        assert len(set(plan)) == len(plan)
        for slot in plan:
            ev = p.serve_one()
            assert ev.handle.slot_index == slot
            assert bytes(ev.event_sha256) == o.serve_one()["event_sha256"]
    assert p.chain_head() == o.chain_head


def test_c5_schedule_replays_on_oracle(gh):
    """BASELINE config 5's scheduler trace, model-free: the 32 admissions of
    bench.c5_workload, decode waves (the next IWRR quanta of distinct lanes,
    served in plan order), the retire of each lane once its last quantum is
    served, then close. The product's event chain equals the oracle's event
    for event, and its close event is the chain head the bench's device
    waves report (the device step does not change the schedule)."""
    import bench

    wl = bench.c5_workload(bench.CFG_7B)
    lanes = wl["lanes"]
    p = gh.LaneWeave(lanes, wl["bank"], bank_epoch=wl["bank_epoch"],
                     scheduler_epoch=wl["scheduler_epoch"], max_weight=wl["max_weight"])
    o = lw.Scheduler(lw.Bank(lanes, lw.limits(**wl["bank"]), wl["bank_epoch"]), lanes,
                     wl["scheduler_epoch"], bytes([0xA5]) + bytes(31), wl["max_weight"],
                     1_000_000, 1_000_000)
    for sp in wl["specs"]:
        o_ok, _, o_ev = o.admit(dict(sp, claim=lw.claim(**sp["claim"])))
        p_ok, _, p_ev = p.admit(_pspec(gh, dict(sp, claim=lw.claim(**sp["claim"]))))
        assert o_ok and p_ok and bytes(p_ev.event_sha256) == o_ev["event_sha256"]
    waves = quanta = 0
    while True:
        plan = p.plan_wave(lanes)
        if not plan:
            break
        waves += 1
        finished = []
        for slot in plan:
            p_ev, o_ev = p.serve_one(), o.serve_one()
            assert p_ev.handle.slot_index == slot
            assert bytes(p_ev.event_sha256) == o_ev["event_sha256"]
            quanta += 1
            if p_ev.remaining_after == 0:
                finished.append(slot)
        for slot in finished:
            rc, p_ev = p.retire(p.slot(slot)[0])
            o_ev = o.retire(o.handle_for(slot))
            assert rc == 0 and bytes(p_ev.event_sha256) == o_ev["event_sha256"]
    rc, p_close = p.close()
    o_close = o.close()
    assert rc == 0 and bytes(p_close.event_sha256) == o_close["event_sha256"]
    assert quanta == lanes * (wl["gen"] - 1)
    print("waves", waves, "close", bytes(p_close.event_sha256).hex())
    # the chain head of the bench's config-5 run on the GPU (device waves)
    assert bytes(p_close.event_sha256).hex() == \
        "7d027cdf284a5173360b19e40f9ba7099533958d46b50fd56d83b44e4b36c06f"


# ------------------------------------------------------ prepared service ----
# The reference's prepared-service tests (lane_weave_qos.zig:6156-6282,
# :6652-6766) on the oracle and on the product. Permits are process-local
# (coordinator id and address), so their digests are compared only with the
# same implementation's recomputation.
class _OracleSched:
    def __init__(self, cap, mw):
        self.f = lw.test_fixture(cap, mw)

    def admit(self, key, weight, work):
        ok, _, ev = self.f.admit(lw.test_spec(key, weight, work, 0))
        assert ok
        return ev["handle"]

    def call(self, name, *args):
        try:
            return "OK", getattr(self.f, name)(*args)
        except lw.LaneWeaveError as e:
            return str(e), None

    def state(self):
        return self.f.state_sha256(), self.f.chain_head, dict(self.f.bank.used)

    def event_sha(self, ev):
        return ev["event_sha256"]

    def mutate(self, p, field, how):
        q = __import__("copy").deepcopy(p)
        if field.startswith("handle."):
            q["handle"][field[7:]] = (q["handle"][field[7:]] + 1) & lw.U64_MAX
        elif field.startswith("resource_receipt."):
            q["resource_receipt"][field[17:]] = (q["resource_receipt"][field[17:]] + 1) & lw.U64_MAX
        elif field.endswith("sha256"):
            q[field] = bytes([q[field][0] ^ 0xFF]) + q[field][1:]
        else:
            q[field] = (q[field] + 1) & lw.U64_MAX
        if how == "resealed":
            q["permit_sha256"] = lw.service_permit_sha256(q)
        return q


class _ProductSched:
    names = {0: "OK", 16: "NoRunnableRequest", 18: "SchedulerClosed", 19: "InvariantViolation",
             23: "ServiceInFlight", 24: "StaleServicePermit", 15: "StaleHandle",
             17: "IncompleteDrain"}

    def __init__(self, gh, cap, mw):
        self.gh = gh
        self.f = _product(gh, cap, mw)

    def admit(self, key, weight, work):
        ok, h, ev = self.f.admit(_pspec(self.gh, lw.test_spec(key, weight, work, 0)))
        assert ok
        return h

    def call(self, name, *args):
        f = self.f
        if name == "prepare_service":
            rc, p = f.prepare_service()
            return self.names.get(rc, rc), p
        if name in ("commit_service", "serve_one", "close"):
            rc, ev = (f.commit_service(*args) if name == "commit_service" else
                      f._ev(getattr(self.gh.lib(), "glacier_hip_lane_weave_" + name)))
            return self.names.get(rc, rc), ev
        if name == "abort_service":
            return self.names.get(f.abort_service(*args), None), None
        if name in ("cancel", "retire"):
            rc, ev = getattr(f, name)(*args)
            return self.names.get(rc, rc), ev
        if name == "admit":
            import ctypes as C
            ok, h, e = C.c_int(0), self.gh.LaneHandle(), self.gh.LaneEvent()
            rc = self.gh.lib().glacier_hip_lane_weave_admit(
                f.h, C.byref(_pspec(self.gh, args[0])), C.byref(ok), C.byref(h), C.byref(e))
            return self.names.get(rc, rc), e
        raise AssertionError(name)

    def state(self):
        return self.f.state_sha256(), self.f.chain_head()

    def event_sha(self, ev):
        return bytes(ev.event_sha256)

    def mutate(self, p, field, how):
        import ctypes as C
        q = self.gh.ServicePermit.from_buffer_copy(p)
        if field.startswith("handle."):
            setattr(q.handle, field[7:], getattr(q.handle, field[7:]) + 1)
        elif field.startswith("resource_receipt."):
            setattr(q.resource_receipt, field[17:], getattr(q.resource_receipt, field[17:]) + 1)
        elif field.endswith("sha256"):
            getattr(q, field)[0] ^= 0xFF
        else:
            setattr(q, field, (getattr(q, field) + 1) & ((1 << 64) - 1))
        if how == "resealed":
            out = (C.c_uint8 * 32)()
            self.gh.lib().glacier_hip_service_permit_sha256(C.byref(q), out)
            q.permit_sha256[:] = list(bytes(out))
        return q


@pytest.fixture(params=["oracle", "product"])
def sched(request, gh):
    return (lambda cap, mw: _OracleSched(cap, mw)) if request.param == "oracle" else \
        (lambda cap, mw: _ProductSched(gh, cap, mw))


def test_service_abort_preserves_state_and_refuses_stale_permits(sched):
    """:6156-6211: prepare changes nothing; abort restores nothing because
    nothing moved; a second permit has a later generation and another
    digest; the aborted first permit is stale for commit and abort."""
    s = sched(2, 2)
    h = s.admit(1, 2, 3)
    before = s.state()
    rc, first = s.call("prepare_service")
    assert rc == "OK" and s.state() == before
    assert s.call("abort_service", first)[0] == "OK" and s.state() == before
    rc, second = s.call("prepare_service")
    assert rc == "OK"
    g = (lambda p: p["permit_generation"]) if isinstance(first, dict) else \
        (lambda p: p.permit_generation)
    d = (lambda p: p["permit_sha256"]) if isinstance(first, dict) else \
        (lambda p: bytes(p.permit_sha256))
    assert g(second) > g(first) and d(second) != d(first)
    assert s.call("commit_service", first)[0] == "StaleServicePermit"
    assert s.call("abort_service", first)[0] == "StaleServicePermit"
    assert s.call("abort_service", second)[0] == "OK"
    assert s.call("cancel", h)[0] == "OK"
    assert s.call("close")[0] == "OK"


def test_prepared_commit_is_byte_identical_to_serve_one(sched):
    """:6253-6282: prepareService + commitService emits the event serveOne
    emits on an identical scheduler."""
    a, b = sched(2, 2), sched(2, 2)
    ha, hb = a.admit(1, 2, 2), b.admit(1, 2, 2)
    rc, legacy = a.call("serve_one")
    rc2, p = b.call("prepare_service")
    rc3, prepared = b.call("commit_service", p)
    assert (rc, rc2, rc3) == ("OK", "OK", "OK")
    assert a.event_sha(legacy) == b.event_sha(prepared) and a.state() == b.state()
    a.call("cancel", ha)
    b.call("cancel", hb)


def test_pending_service_blocks_every_logical_mutator(sched):
    """:6652-6697."""
    s = sched(2, 2)
    h1, h2 = s.admit(1, 1, 2), s.admit(2, 2, 2)
    rc, p = s.call("prepare_service")
    before = s.state()
    assert s.call("prepare_service")[0] == "ServiceInFlight"
    assert s.call("serve_one")[0] == "ServiceInFlight"
    assert s.call("admit", lw.test_spec(3, 1, 1, 0))[0] == "ServiceInFlight"
    assert s.call("cancel", h1)[0] == "ServiceInFlight"
    assert s.call("cancel", h2)[0] == "ServiceInFlight"
    assert s.call("retire", h1)[0] == "ServiceInFlight"
    assert s.call("close")[0] == "ServiceInFlight"
    assert s.state() == before
    assert s.call("abort_service", p)[0] == "OK"
    assert s.call("cancel", h1)[0] == "OK" and s.call("cancel", h2)[0] == "OK"
    assert s.call("close")[0] == "OK"


MUTATIONS = ["abi_version", "scheduler_epoch", "coordinator_id", "coordinator_address",
             "permit_generation", "event_sequence", "handle.request_key", "logical_tick_before",
             "cursor_before", "level_before", "cursor_after", "level_after", "remaining_before",
             "wait_quanta", "maximum_service_gap", "state_before_sha256",
             "chain_head_before_sha256", "resource_receipt.owner_key", "resource_receipt_sha256",
             "permit_sha256"]


def test_mutated_and_foreign_permits_reject_without_consumption(sched):
    """:6699-6766: each of the 20 single-field mutations is stale for commit;
    a mutation resealed with its own digest is stale for abort; another
    scheduler's permit is stale; the real permit then commits once."""
    s, foreign = sched(1, 1), sched(1, 1)
    h = s.admit(1, 1, 2)
    fh = foreign.admit(1, 1, 2)
    rc, p = s.call("prepare_service")
    for field in MUTATIONS:
        assert s.call("commit_service", s.mutate(p, field, "raw"))[0] == "StaleServicePermit", field
    assert s.call("abort_service", s.mutate(p, "remaining_before", "resealed"))[0] == \
        "StaleServicePermit"
    assert foreign.call("commit_service", p)[0] == "StaleServicePermit"
    assert s.call("commit_service", p)[0] == "OK"
    assert s.call("commit_service", p)[0] == "StaleServicePermit"
    assert s.call("abort_service", p)[0] == "StaleServicePermit"
    assert s.call("cancel", h)[0] == "OK" and s.call("close")[0] == "OK"
    rc, fp = foreign.call("prepare_service")
    assert foreign.call("abort_service", fp)[0] == "OK"
    assert foreign.call("cancel", fh)[0] == "OK" and foreign.call("close")[0] == "OK"


def test_permit_of_an_earlier_scheduler_is_stale(sched):
    """:6213-6251: a scheduler's lifetime fences its permits (a later
    scheduler gets another coordinator id)."""
    old = sched(1, 1)
    old.admit(1, 1, 1)
    rc, stale = old.call("prepare_service")
    new = sched(1, 1)
    h = new.admit(1, 1, 1)
    rc, fresh = new.call("prepare_service")
    cid = (lambda p: p["coordinator_id"]) if isinstance(fresh, dict) else \
        (lambda p: p.coordinator_id)
    assert cid(stale) != cid(fresh)
    assert new.call("commit_service", stale)[0] == "StaleServicePermit"
    assert new.call("abort_service", stale)[0] == "StaleServicePermit"
    assert new.call("commit_service", fresh)[0] == "OK"
    assert new.call("retire", h)[0] == "OK" and new.call("close")[0] == "OK"
