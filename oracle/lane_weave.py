"""LaneWeave QoS v1 and the flat ResourceBank it admits against, restated in
Python from the reference.

TEST INFRASTRUCTURE ONLY: tests/ and bench.py's cpu_baseline leg use it as the
checker of the product scheduler (glacier_hip_lane_weave_*); the product never
imports it.

Restated from src/core/lane_weave_qos.zig and src/core/resource_bank.zig:
  * Claim / Limits / Receipt field order          resource_bank.zig:61-125, 497-515
  * mix64, tokenIntegrity, domains                resource_bank.zig:4159-4160, 4877-4903
  * Bank.reserve / commit / release (flat slots)  resource_bank.zig:976-1070, 3166
  * Scheduler.init (maximum service gap, root)    lane_weave_qos.zig:634-735, 4040-4064
  * admitLocked (rejection order, projection)     lane_weave_qos.zig:748-900, 3145-3290
  * serveOne / prepareService+commitService       lane_weave_qos.zig:1131-1290, 2617-2662
  * retire / cancel / close                       lane_weave_qos.zig:1454-1490, 1923-2014
  * IWRR selection                                lane_weave_qos.zig:3429-3512
  * state digest, event digest, receipt digest    lane_weave_qos.zig:2801-2815, 3399-3427,
                                                  3994-4038, 4066-4146
Pinned by the reference's own tests (tests/test_lane_weave.py): the IWRR golden
order and close-event SHA-256 (lane_weave_qos.zig:4436-4474), the deadline,
projection-budget and resource-limit rejections (:4476-4570) and stale-handle
fencing (:4572-4586).
"""
import copy
import hashlib
import struct

MASK64 = (1 << 64) - 1
U64_MAX = MASK64

RESOURCE_BANK_ABI = 0x4752424B00000001
ABI = 0x474C575100000001
EVENT_ABI = 0x474C574500000001
RESERVATION_DOMAIN = 0x7265736572766531
RECEIPT_DOMAIN = 0x7265636569707431

CLAIM_FIELDS = ("capsule_bytes", "kv_bytes", "activation_bytes", "partial_bytes", "logits_bytes",
                "output_journal_bytes", "staging_bytes", "device_bytes", "io_bytes",
                "queue_slots")
HOST_FIELDS = CLAIM_FIELDS[:7]
LIMIT_FIELDS = ("host_bytes",) + CLAIM_FIELDS

# EventKind / RejectionReason / SlotState enum values (lane_weave_qos.zig:262-300)
ADMISSION_ACCEPTED, ADMISSION_REJECTED, SERVICE, CANCEL, RETIRE, CLOSE = range(6)
NONE, NO_SLOT, DUPLICATE_TENANT, RESOURCE_LIMIT, PROJECTION_LIMIT, DEADLINE_INFEASIBLE = range(6)
FREE, ACTIVE, FINISHED = range(3)


SERVICE_PERMIT_ABI = 0x474C575000000001  # service_permit_abi (lane_weave_qos.zig:19)
_next_coordinator = [1]  # nextServiceCoordinatorId (:556-566)


class LaneWeaveError(Exception):
    pass


def claim(**kw):
    c = {f: 0 for f in CLAIM_FIELDS}
    c.update(kw)
    return c


def limits(**kw):
    lim = {f: U64_MAX for f in LIMIT_FIELDS}
    lim.update(kw)
    return lim


def claim_is_zero(c):
    return all(c[f] == 0 for f in CLAIM_FIELDS)


def host_bytes(c):
    t = sum(c[f] for f in HOST_FIELDS)
    if t > U64_MAX:
        raise LaneWeaveError("ClaimOverflow")
    return t


def add_claims(a, b):
    out = {f: a[f] + b[f] for f in CLAIM_FIELDS}
    if any(v > U64_MAX for v in out.values()):
        return None
    return out


def sub_claims(a, b):
    out = {f: a[f] - b[f] for f in CLAIM_FIELDS}
    if any(v < 0 for v in out.values()):
        raise LaneWeaveError("BankDrift")
    return out


def fits(lim, c):
    try:
        h = host_bytes(c)
    except LaneWeaveError:
        return False
    return h <= lim["host_bytes"] and all(c[f] <= lim[f] for f in CLAIM_FIELDS)


def mix64(v):
    v ^= v >> 30
    v = (v * 0xBF58476D1CE4E5B9) & MASK64
    v ^= v >> 27
    v = (v * 0x94D049BB133111EB) & MASK64
    v ^= v >> 31
    return v


def token_integrity(epoch, slot_index, generation, owner_key, c, domain):
    r = mix64(domain ^ epoch)
    r = mix64(r ^ slot_index)
    r = mix64(r ^ generation)
    r = mix64(r ^ owner_key)
    for f in CLAIM_FIELDS:
        r = mix64(r ^ c[f])
    return r


def zero_receipt():
    return dict(bank_epoch=0, slot_index=0, generation=0, owner_key=0, claim=claim(), integrity=0)


class Bank:
    """Flat ResourceBank (resource_bank.zig:867-3200, the parts LaneWeave uses)."""

    def __init__(self, capacity, lim, epoch):
        self.slots = [dict(state=0, generation=0, owner_key=0, claim=claim(), integrity=0)
                      for _ in range(capacity)]
        self.limits = lim
        self.epoch = epoch
        self.used = claim()
        self.next_generation = 1

    def committed_receipts(self):
        return sum(1 for s in self.slots if s["state"] == 2)

    def reserve(self, owner_key, c):
        if owner_key == 0 or claim_is_zero(c):
            raise LaneWeaveError("InvalidClaim")
        nxt = add_claims(self.used, c)
        if nxt is None or not fits(self.limits, nxt):
            raise LaneWeaveError("CapacityExceeded")
        idx = next((i for i, s in enumerate(self.slots) if s["state"] == 0), None)
        if idx is None:
            raise LaneWeaveError("ReservationSlotsExhausted")
        gen = self.next_generation
        self.next_generation += 1
        integ = token_integrity(self.epoch, idx, gen, owner_key, c, RESERVATION_DOMAIN)
        self.slots[idx] = dict(state=1, generation=gen, owner_key=owner_key, claim=dict(c),
                               integrity=integ)
        self.used = nxt
        return dict(bank_epoch=self.epoch, slot_index=idx, generation=gen, owner_key=owner_key,
                    claim=dict(c), integrity=integ)

    def commit(self, res):
        s = self.slots[res["slot_index"]]
        if s["state"] != 1 or s["generation"] != res["generation"]:
            raise LaneWeaveError("InvalidTransition")
        integ = token_integrity(self.epoch, res["slot_index"], res["generation"], res["owner_key"],
                                res["claim"], RECEIPT_DOMAIN)
        s["state"] = 2
        s["integrity"] = integ
        r = dict(res)
        r["integrity"] = integ
        return r

    def release(self, rec):
        s = self.slots[rec["slot_index"]]
        if s["state"] != 2 or s["generation"] != rec["generation"]:
            raise LaneWeaveError("StaleReservation")
        self.used = sub_claims(self.used, rec["claim"])
        self.slots[rec["slot_index"]] = dict(state=0, generation=0, owner_key=0, claim=claim(),
                                             integrity=0)


# ---- little-endian field hashing (lane_weave_qos.zig:4066-4146) -----------
def _u8(h, v):
    h.update(struct.pack("<B", v))


def _u16(h, v):
    h.update(struct.pack("<H", v))


def _u32(h, v):
    h.update(struct.pack("<I", v))


def _u64(h, v):
    h.update(struct.pack("<Q", v & MASK64))


def _claim(h, c):
    for f in CLAIM_FIELDS:
        _u64(h, c[f])


def _limits(h, lim):
    for f in LIMIT_FIELDS:
        _u64(h, lim[f])


def _spec(h, sp):
    for f in ("tenant_key", "request_key", "request_generation", "resource_owner_key"):
        _u64(h, sp[f])
    _u16(h, sp["weight"])
    _u64(h, sp["work_quanta"])
    _u64(h, sp["deadline_tick"])
    _claim(h, sp["claim"])


def _handle(h, hd):
    _u64(h, hd["scheduler_epoch"])
    _u32(h, hd["slot_index"])
    for f in ("slot_generation", "tenant_key", "request_key", "request_generation"):
        _u64(h, hd[f])


def _receipt(h, r):
    _u64(h, r["bank_epoch"])
    _u32(h, r["slot_index"])
    _u64(h, r["generation"])
    _u64(h, r["owner_key"])
    _claim(h, r["claim"])
    _u64(h, r["integrity"])


def empty_spec():
    return dict(tenant_key=0, request_key=0, request_generation=0, resource_owner_key=0, weight=0,
                work_quanta=0, deadline_tick=0, claim=claim())


def empty_handle():
    return dict(scheduler_epoch=0, slot_index=0, slot_generation=0, tenant_key=0, request_key=0,
                request_generation=0)


def resource_receipt_sha256(r):
    h = hashlib.sha256(b"glacier-lane-weave-qos-resource-receipt-v1\x00")
    _receipt(h, r)
    return h.digest()


def event_sha256(e):
    h = hashlib.sha256(b"glacier-lane-weave-qos-event-v1\x00")
    _u64(h, e["abi_version"])
    _u64(h, e["scheduler_epoch"])
    _u64(h, e["event_sequence"])
    _u8(h, e["kind"])
    _u8(h, e["rejection_reason"])
    h.update(e["previous_sha256"])
    h.update(e["state_before_sha256"])
    h.update(e["state_after_sha256"])
    _u64(h, e["logical_tick_before"])
    _u64(h, e["logical_tick_after"])
    _u32(h, e["cursor_before"])
    _u32(h, e["cursor_after"])
    _u16(h, e["level_before"])
    _u16(h, e["level_after"])
    _handle(h, e["handle"])
    _spec(h, e["spec"])
    _receipt(h, e["resource_receipt"])
    h.update(e["resource_receipt_sha256"])
    for f in ("remaining_before", "remaining_after", "wait_quanta", "maximum_service_gap"):
        _u64(h, e[f])
    for f in ("active_before", "active_after", "finished_before", "finished_after"):
        _u32(h, e[f])
    _claim(h, e["bank_used_before"])
    _claim(h, e["bank_used_after"])
    return h.digest()


class _Budget:
    def __init__(self, remaining):
        self.remaining = remaining
        self.exhausted = False

    def spend(self, amount):
        if amount > self.remaining:
            self.exhausted = True
            return False
        self.remaining -= amount
        return True


def select_iwrr(slots, cursor0, level0, max_weight, budget=None):
    """selectIWRRWithBudget (lane_weave_qos.zig:3444-3496). `slots` items
    expose active / weight. Returns (index, cursor_after, level_after) or None."""
    n = len(slots)
    if n == 0:
        return None
    if budget is not None and not budget.spend(n):
        return None
    max_active = max((w for a, w in slots if a), default=0)
    if max_active == 0:
        return None
    cursor = min(cursor0, n)
    level = 1 if level0 == 0 else level0
    if level > max_active or level > max_weight:
        level, cursor = 1, 0
    scan_limit = n * max_weight
    for _ in range(scan_limit):
        if budget is not None and not budget.spend(1):
            return None
        if cursor >= n:
            cursor = 0
            level = 1 if level >= max_active else level + 1
        idx = cursor
        cursor += 1
        active, weight = slots[idx]
        if active and weight >= level:
            return idx, cursor, level
    return None


class Scheduler:
    """LaneWeave Scheduler over a dedicated flat Bank."""

    def __init__(self, bank, capacity, scheduler_epoch, challenge, max_weight=64,
                 max_projection_quanta=1_000_000, max_projection_operations=1_000_000):
        if (capacity == 0 or len(bank.slots) != capacity or scheduler_epoch == 0 or
                max_weight == 0 or max_projection_quanta == 0 or
                max_projection_operations == 0 or challenge == bytes(32)):
            raise LaneWeaveError("InvalidConfiguration")
        self.bank = bank
        self.epoch = scheduler_epoch
        self.challenge = challenge
        self.max_weight = max_weight
        self.max_pq = max_projection_quanta
        self.max_po = max_projection_operations
        self.slots = [self._free_slot() for _ in range(capacity)]
        self.used = claim()
        self.logical_tick = 0
        self.next_event_sequence = 0
        self.next_slot_generation = 1
        self.cursor = 0
        self.level = 1
        self.poisoned = False
        self.closed = False
        self.pending_service = None
        self.next_service_permit_generation = 1
        self.service_coordinator_id = _next_coordinator[0]
        _next_coordinator[0] += 1
        self.maximum_service_gap = (capacity - 1) * max_weight + 1
        h = hashlib.sha256(b"glacier-lane-weave-qos-root-v1\x00")
        _u64(h, ABI)
        _u64(h, EVENT_ABI)
        _u64(h, RESOURCE_BANK_ABI)
        _u64(h, scheduler_epoch)
        h.update(challenge)
        _u16(h, max_weight)
        _u64(h, max_projection_quanta)
        _u64(h, max_projection_operations)
        _u32(h, capacity)
        _u64(h, bank.epoch)
        _limits(h, bank.limits)
        _u64(h, self.maximum_service_gap)
        self.chain_head = h.digest()

    @staticmethod
    def _free_slot():
        return dict(state=FREE, generation=0, spec=empty_spec(), remaining_quanta=0,
                    admitted_tick=0, last_service_tick=0, service_count=0,
                    receipt=zero_receipt(), receipt_sha256=bytes(32))

    # ---- digests ----
    def state_sha256(self):
        h = hashlib.sha256(b"glacier-lane-weave-qos-state-v1\x00")
        _u64(h, self.epoch)
        _u64(h, self.logical_tick)
        _u64(h, self.next_event_sequence)
        _u64(h, self.next_slot_generation)
        _u32(h, self.cursor)
        _u16(h, self.level)
        _u8(h, 1 if self.poisoned else 0)
        _u8(h, 1 if self.closed else 0)
        _claim(h, self.used)
        _u32(h, len(self.slots))
        for s in self.slots:
            _u8(h, s["state"])
            _u64(h, s["generation"])
            _spec(h, s["spec"])
            for f in ("remaining_quanta", "admitted_tick", "last_service_tick", "service_count"):
                _u64(h, s[f])
            _receipt(h, s["receipt"])
            h.update(s["receipt_sha256"])
        return h.digest()

    def counts(self):
        a = sum(1 for s in self.slots if s["state"] == ACTIVE)
        f = sum(1 for s in self.slots if s["state"] == FINISHED)
        return a, f

    def handle_for(self, i):
        s = self.slots[i]
        return dict(scheduler_epoch=self.epoch, slot_index=i, slot_generation=s["generation"],
                    tenant_key=s["spec"]["tenant_key"], request_key=s["spec"]["request_key"],
                    request_generation=s["spec"]["request_generation"])

    def _emit(self, kind, before_state, tick0, cursor0, level0, counts0, used0, reason=NONE,
              handle=None, spec=None, receipt=None, receipt_sha=bytes(32), remaining_before=0,
              remaining_after=0, wait=0):
        seq = self.next_event_sequence
        self.next_event_sequence += 1
        a1, f1 = self.counts()
        e = dict(abi_version=EVENT_ABI, scheduler_epoch=self.epoch, event_sequence=seq, kind=kind,
                 rejection_reason=reason, previous_sha256=self.chain_head,
                 state_before_sha256=before_state, state_after_sha256=self.state_sha256(),
                 logical_tick_before=tick0, logical_tick_after=self.logical_tick,
                 cursor_before=cursor0, cursor_after=self.cursor, level_before=level0,
                 level_after=self.level, handle=handle or empty_handle(),
                 spec=spec or empty_spec(), resource_receipt=receipt or zero_receipt(),
                 resource_receipt_sha256=receipt_sha, remaining_before=remaining_before,
                 remaining_after=remaining_after, wait_quanta=wait,
                 maximum_service_gap=self.maximum_service_gap, active_before=counts0[0],
                 active_after=a1, finished_before=counts0[1], finished_after=f1,
                 bank_used_before=used0, bank_used_after=dict(self.used))
        e["event_sha256"] = event_sha256(e)
        self.chain_head = e["event_sha256"]
        return e

    def _snapshot_before(self):
        return self.state_sha256(), self.logical_tick, self.cursor, self.level, self.counts(), dict(self.used)

    # ---- admission ----
    def _valid_spec(self, sp):
        c = sp["claim"]
        bad = (sp["tenant_key"] == 0 or sp["request_key"] == 0 or sp["request_generation"] == 0 or
               sp["resource_owner_key"] == 0 or sp["weight"] == 0 or
               sp["weight"] > self.max_weight or sp["work_quanta"] == 0 or claim_is_zero(c) or
               c["queue_slots"] != 1 or
               (sp["deadline_tick"] != 0 and sp["deadline_tick"] <= self.logical_tick))
        if bad:
            raise LaneWeaveError("InvalidRequest")
        host_bytes(c)

    def _project_prepared(self, proj, deadline_count, budget):
        if deadline_count == 0:
            return "feasible"
        tick, cursor, level, pq = self.logical_tick, self.cursor, self.level, 0
        while deadline_count:
            if pq >= self.max_pq:
                return "projection_limit"
            if not budget.spend(len(proj)):
                return "projection_limit"
            for p in proj:
                if p["active"] and p["deadline"] != 0 and tick >= p["deadline"]:
                    return "deadline_infeasible"
            sel = select_iwrr([(p["active"], p["weight"]) for p in proj], cursor, level,
                              self.max_weight, budget)
            if sel is None:
                return "projection_limit" if budget.exhausted else "deadline_infeasible"
            idx, cursor, level = sel
            p = proj[idx]
            p["remaining"] -= 1
            tick += 1
            pq += 1
            if p["remaining"] == 0:
                if p["deadline"] != 0 and tick > p["deadline"]:
                    return "deadline_infeasible"
                if p["deadline"] != 0:
                    deadline_count -= 1
                p["active"] = False
        return "feasible"

    def _project_admission(self, cand_idx, sp):
        budget = _Budget(self.max_po)
        if sp["deadline_tick"] != 0 and sp["work_quanta"] > self.max_pq:
            return "projection_limit"
        if sp["deadline_tick"] == 0:
            if not budget.spend(len(self.slots)):
                return "projection_limit"
            if not any(s["state"] == ACTIVE and s["spec"]["deadline_tick"] != 0 for s in self.slots):
                return "feasible"
        if not budget.spend(len(self.slots)):
            return "projection_limit"
        proj, dc, mq = [], 0, 0
        for s in self.slots:
            if s["state"] == ACTIVE:
                proj.append(dict(active=True, weight=s["spec"]["weight"],
                                 remaining=s["remaining_quanta"], deadline=s["spec"]["deadline_tick"]))
                if s["spec"]["deadline_tick"] != 0:
                    dc += 1
                    mq += s["remaining_quanta"]
            else:
                proj.append(dict(active=False, weight=0, remaining=0, deadline=0))
        proj[cand_idx] = dict(active=True, weight=sp["weight"], remaining=sp["work_quanta"],
                              deadline=sp["deadline_tick"])
        if sp["deadline_tick"] != 0:
            dc += 1
            mq += sp["work_quanta"]
        if mq > self.max_pq:
            return "projection_limit"
        return self._project_prepared(proj, dc, budget)

    def admit(self, sp):
        """Returns (accepted: bool, handle or None, event)."""
        if self.closed:
            raise LaneWeaveError("SchedulerClosed")
        self._require_no_service()
        self._valid_spec(sp)
        snap = self._snapshot_before()

        def reject(reason):
            return False, None, self._emit(ADMISSION_REJECTED, snap[0], snap[1], snap[2], snap[3],
                                           snap[4], snap[5], reason=reason, spec=sp)
        free = None
        for i, s in enumerate(self.slots):
            if s["state"] != FREE and s["spec"]["tenant_key"] == sp["tenant_key"]:
                return reject(DUPLICATE_TENANT)
            if s["state"] == FREE and free is None:
                free = i
        if free is None:
            return reject(NO_SLOT)
        nxt = add_claims(self.used, sp["claim"])
        if nxt is None or not fits(self.bank.limits, nxt):
            return reject(RESOURCE_LIMIT)
        out = self._project_admission(free, sp)
        if out == "projection_limit":
            return reject(PROJECTION_LIMIT)
        if out == "deadline_infeasible":
            return reject(DEADLINE_INFEASIBLE)
        gen = self.next_slot_generation
        res = self.bank.reserve(sp["resource_owner_key"], sp["claim"])
        rec = self.bank.commit(res)
        if rec["slot_index"] != free or rec["generation"] != gen:
            raise LaneWeaveError("BankDrift")
        self.next_slot_generation += 1
        rsha = resource_receipt_sha256(rec)
        self.slots[free] = dict(state=ACTIVE, generation=gen, spec=dict(sp),
                                remaining_quanta=sp["work_quanta"], admitted_tick=self.logical_tick,
                                last_service_tick=self.logical_tick, service_count=0, receipt=rec,
                                receipt_sha256=rsha)
        self.used = nxt
        handle = self.handle_for(free)
        ev = self._emit(ADMISSION_ACCEPTED, snap[0], snap[1], snap[2], snap[3], snap[4], snap[5],
                        handle=handle, spec=sp, receipt=rec, receipt_sha=rsha,
                        remaining_after=sp["work_quanta"])
        return True, handle, ev

    # ---- service ----
    def next_selection(self):
        return select_iwrr([(s["state"] == ACTIVE, s["spec"]["weight"]) for s in self.slots],
                           self.cursor, self.level, self.max_weight)

    def _require_no_service(self):
        if self.pending_service is not None:
            raise LaneWeaveError("ServiceInFlight")

    def serve_one(self):
        if self.closed:
            raise LaneWeaveError("SchedulerClosed")
        self._require_no_service()
        return self._serve_locked()

    def _serve_locked(self):
        sel = self.next_selection()
        if sel is None:
            raise LaneWeaveError("NoRunnableRequest")
        idx, cur_after, lvl_after = sel
        s = self.slots[idx]
        snap = self._snapshot_before()
        rem0 = s["remaining_quanta"]
        handle = self.handle_for(idx)
        after_tick = self.logical_tick + 1
        for j, o in enumerate(self.slots):  # selectionPreservesDeadlines
            if o["state"] != ACTIVE or o["spec"]["deadline_tick"] == 0:
                continue
            completes = j == idx and o["remaining_quanta"] == 1
            if (completes and after_tick > o["spec"]["deadline_tick"]) or (
                    not completes and after_tick >= o["spec"]["deadline_tick"]):
                self.poisoned = True
                raise LaneWeaveError("InvariantViolation")
        wait = after_tick - s["last_service_tick"]
        if wait > self.maximum_service_gap:
            self.poisoned = True
            raise LaneWeaveError("InvariantViolation")
        s["remaining_quanta"] -= 1
        s["last_service_tick"] = after_tick
        s["service_count"] += 1
        if s["remaining_quanta"] == 0:
            s["state"] = FINISHED
        self.logical_tick = after_tick
        self.cursor, self.level = cur_after, lvl_after
        return self._emit(SERVICE, snap[0], snap[1], snap[2], snap[3], snap[4], snap[5],
                          handle=handle, spec=s["spec"], receipt=s["receipt"],
                          receipt_sha=s["receipt_sha256"], remaining_before=rem0,
                          remaining_after=s["remaining_quanta"], wait=wait)

    # ---- terminal events ----
    def _finish(self, handle, kind, required_state):
        if self.closed:
            raise LaneWeaveError("SchedulerClosed")
        self._require_no_service()
        i = handle["slot_index"]
        if handle["scheduler_epoch"] != self.epoch or i >= len(self.slots):
            raise LaneWeaveError("StaleHandle")
        s = self.slots[i]
        if (s["state"] != required_state or s["generation"] != handle["slot_generation"] or
                s["spec"]["tenant_key"] != handle["tenant_key"] or
                s["spec"]["request_key"] != handle["request_key"] or
                s["spec"]["request_generation"] != handle["request_generation"]):
            raise LaneWeaveError("StaleHandle")
        snap = self._snapshot_before()
        sp, rec, rsha, rem = s["spec"], s["receipt"], s["receipt_sha256"], s["remaining_quanta"]
        self.bank.release(rec)
        self.used = sub_claims(self.used, sp["claim"])
        self.slots[i] = self._free_slot()
        return self._emit(kind, snap[0], snap[1], snap[2], snap[3], snap[4], snap[5],
                          handle=handle, spec=sp, receipt=rec, receipt_sha=rsha,
                          remaining_before=rem)

    def retire(self, handle):
        return self._finish(handle, RETIRE, FINISHED)

    def cancel(self, handle):
        return self._finish(handle, CANCEL, ACTIVE)

    def close(self):
        if self.closed:
            raise LaneWeaveError("SchedulerClosed")
        self._require_no_service()
        a, f = self.counts()
        if a or f or not claim_is_zero(self.used):
            raise LaneWeaveError("IncompleteDrain")
        snap = self._snapshot_before()
        self.closed = True
        return self._emit(CLOSE, snap[0], snap[1], snap[2], snap[3], (0, 0), snap[5])

    # ---- prepared service (prepareService :1127-1192, commitService
    # :1272-1286, abortService :1438-1452) ----
    def prepare_service(self):
        if self.closed:
            raise LaneWeaveError("SchedulerClosed")
        self._require_no_service()
        if self.logical_tick == U64_MAX:
            raise LaneWeaveError("TickOverflow")
        sel = self.next_selection()
        if sel is None:
            raise LaneWeaveError("NoRunnableRequest")
        idx, cur_after, lvl_after = sel
        s = self.slots[idx]
        after_tick = self.logical_tick + 1
        for j, o in enumerate(self.slots):  # selectionPreservesDeadlines
            if o["state"] != ACTIVE or o["spec"]["deadline_tick"] == 0:
                continue
            completes = j == idx and o["remaining_quanta"] == 1
            if (completes and after_tick > o["spec"]["deadline_tick"]) or (
                    not completes and after_tick >= o["spec"]["deadline_tick"]):
                self.poisoned = True
                raise LaneWeaveError("InvariantViolation")
        wait = after_tick - s["last_service_tick"]
        if wait > self.maximum_service_gap:
            self.poisoned = True
            raise LaneWeaveError("InvariantViolation")
        p = dict(abi_version=SERVICE_PERMIT_ABI, scheduler_epoch=self.epoch,
                 coordinator_id=self.service_coordinator_id,
                 coordinator_address=id(self) & U64_MAX,
                 permit_generation=self.next_service_permit_generation,
                 event_sequence=self.next_event_sequence, handle=self.handle_for(idx),
                 logical_tick_before=self.logical_tick, cursor_before=self.cursor,
                 level_before=self.level, cursor_after=cur_after, level_after=lvl_after,
                 remaining_before=s["remaining_quanta"], wait_quanta=wait,
                 maximum_service_gap=self.maximum_service_gap,
                 state_before_sha256=self.state_sha256(),
                 chain_head_before_sha256=self.chain_head, resource_receipt=dict(s["receipt"]),
                 resource_receipt_sha256=s["receipt_sha256"])
        p["permit_sha256"] = service_permit_sha256(p)
        self.next_service_permit_generation += 1
        self.pending_service = copy.deepcopy(p)
        return p

    def _validate_pending(self, p):
        """validatePendingService (:2461-2487)."""
        pend = self.pending_service
        if pend is None:
            raise LaneWeaveError("StaleServicePermit")
        if pend["permit_sha256"] != service_permit_sha256(pend):
            self.poisoned = True
            raise LaneWeaveError("InvariantViolation")
        if (p["abi_version"] != SERVICE_PERMIT_ABI or p["scheduler_epoch"] != self.epoch or
                p["coordinator_id"] != self.service_coordinator_id or
                p["coordinator_address"] != id(self) & U64_MAX or p["permit_generation"] == 0 or
                p["permit_sha256"] != service_permit_sha256(p) or p != pend):
            raise LaneWeaveError("StaleServicePermit")

    def _validate_before_state(self, p):
        """validateServiceBeforeState (:2512-2531)."""
        if (p["state_before_sha256"] != self.state_sha256() or
                p["event_sequence"] != self.next_event_sequence or
                p["logical_tick_before"] != self.logical_tick or
                p["chain_head_before_sha256"] != self.chain_head):
            self.poisoned = True
            raise LaneWeaveError("InvariantViolation")

    def commit_service(self, p):
        if self.closed:
            raise LaneWeaveError("SchedulerClosed")
        self._validate_pending(p)
        self._validate_before_state(p)
        sel = self.next_selection()
        if sel is None or sel[0] != p["handle"]["slot_index"] or sel[1] != p["cursor_after"] or \
                sel[2] != p["level_after"]:
            self.poisoned = True
            raise LaneWeaveError("InvariantViolation")
        self.pending_service = None
        return self._serve_locked()

    def abort_service(self, p):
        if self.closed:
            raise LaneWeaveError("SchedulerClosed")
        self._validate_pending(p)
        self._validate_before_state(p)
        self.pending_service = None


def service_permit_sha256(p):
    """servicePermitSha256 (lane_weave_qos.zig:3557-3581)."""
    h = hashlib.sha256(b"glacier-lane-weave-qos-service-permit-v1\x00")
    for f in ("abi_version", "scheduler_epoch", "coordinator_id", "coordinator_address",
              "permit_generation", "event_sequence"):
        _u64(h, p[f])
    _handle(h, p["handle"])
    _u64(h, p["logical_tick_before"])
    _u32(h, p["cursor_before"])
    _u16(h, p["level_before"])
    _u32(h, p["cursor_after"])
    _u16(h, p["level_after"])
    for f in ("remaining_before", "wait_quanta", "maximum_service_gap"):
        _u64(h, p[f])
    h.update(p["state_before_sha256"])
    h.update(p["chain_head_before_sha256"])
    _receipt(h, p["resource_receipt"])
    h.update(p["resource_receipt_sha256"])
    return h.digest()


def test_spec(key, weight, work, deadline):
    """testSpec (lane_weave_qos.zig:4198-4209)."""
    return dict(tenant_key=key, request_key=key * 10, request_generation=1,
                resource_owner_key=key * 100, weight=weight, work_quanta=work,
                deadline_tick=deadline, claim=claim(kv_bytes=64, queue_slots=1))


def test_fixture(capacity, max_weight, max_projection_quanta=10_000,
                 max_projection_operations=1_000_000):
    """TestFixture.initWithProjectionLimits (lane_weave_qos.zig:4146-4196)."""
    bank = Bank(capacity, limits(host_bytes=1 << 20, kv_bytes=1 << 20, queue_slots=capacity),
                0x42414E4B)
    challenge = bytes([0xA5]) + bytes(31)
    return Scheduler(bank, capacity, 0x51534553, challenge, max_weight, max_projection_quanta,
                     max_projection_operations)
