// lane_weave.cpp — LaneWeave QoS v1 (deterministic interleaved weighted
// round-robin multi-request scheduler) over its dedicated flat ResourceBank,
// restated from src/core/lane_weave_qos.zig and src/core/resource_bank.zig.
//
// The scheduler is host control-plane state: it decides which lane receives
// the next decode token and records every decision as a SHA-256-chained
// Event-v1 in the reference's byte format. The device never sees it; a decode
// wave runs the planned lanes' tokens in one batched step and the host then
// commits the quanta in order (see glacier_hip_lane_weave_plan_wave).
#include <limits.h>
#include <string.h>

#include <atomic>
#include <functional>
#include <mutex>
#include <vector>

#include "../../include/glacier_hip.h"
#include "host_util.h"
#include "lane_weave.h"

namespace {

constexpr uint64_t kU64Max = ~0ull;
constexpr uint64_t kBankAbi = 0x4752424B00000001ull;        // resource_bank.zig:12
constexpr uint64_t kAbi = 0x474C575100000001ull;            // lane_weave_qos.zig:17
constexpr uint64_t kEventAbi = 0x474C574500000001ull;       // :18
constexpr uint64_t kPermitAbi = 0x474C575000000001ull;      // :19 service_permit_abi
constexpr uint64_t kReservationDomain = 0x7265736572766531ull;  // resource_bank.zig:4159
constexpr uint64_t kReceiptDomain = 0x7265636569707431ull;      // :4160

using Claim = glacier_hip_claim_t;
using Limits = glacier_hip_limits_t;
using Spec = glacier_hip_request_spec_t;
using Handle = glacier_hip_lane_handle_t;
using Receipt = glacier_hip_bank_receipt_t;
using Event = glacier_hip_lane_event_t;

constexpr int kClaimFields = 10;
const uint64_t *claim_fields(const Claim &c) { return &c.capsule_bytes; }
uint64_t *claim_fields(Claim &c) { return &c.capsule_bytes; }

bool claim_zero(const Claim &c) {
  for (int i = 0; i < kClaimFields; ++i)
    if (claim_fields(c)[i]) return false;
  return true;
}

// Claim.hostBytes (resource_bank.zig:73-91): the seven host byte classes.
bool host_bytes(const Claim &c, uint64_t *out) {
  uint64_t t = 0;
  for (int i = 0; i < 7; ++i) {
    if (t > kU64Max - claim_fields(c)[i]) return false;
    t += claim_fields(c)[i];
  }
  *out = t;
  return true;
}

bool add_claims(const Claim &a, const Claim &b, Claim *out) {
  for (int i = 0; i < kClaimFields; ++i) {
    const uint64_t x = claim_fields(a)[i], y = claim_fields(b)[i];
    if (x > kU64Max - y) return false;
    claim_fields(*out)[i] = x + y;
  }
  return true;
}

bool sub_claims(const Claim &a, const Claim &b, Claim *out) {
  for (int i = 0; i < kClaimFields; ++i) {
    const uint64_t x = claim_fields(a)[i], y = claim_fields(b)[i];
    if (x < y) return false;
    claim_fields(*out)[i] = x - y;
  }
  return true;
}

// Limits.fits (resource_bank.zig:115-133)
bool fits(const Limits &l, const Claim &c) {
  uint64_t h;
  if (!host_bytes(c, &h)) return false;
  const uint64_t *lf = &l.capsule_bytes;  // per-class limits, same order as Claim
  if (h > l.host_bytes) return false;
  for (int i = 0; i < kClaimFields; ++i)
    if (claim_fields(c)[i] > lf[i]) return false;
  return true;
}

// mix64 / tokenIntegrity (resource_bank.zig:4877-4903)
uint64_t mix64(uint64_t v) {
  v ^= v >> 30;
  v *= 0xbf58476d1ce4e5b9ull;
  v ^= v >> 27;
  v *= 0x94d049bb133111ebull;
  v ^= v >> 31;
  return v;
}

uint64_t token_integrity(uint64_t epoch, uint32_t slot, uint64_t gen, uint64_t owner, const Claim &c,
                         uint64_t domain) {
  uint64_t r = mix64(domain ^ epoch);
  r = mix64(r ^ (uint64_t)slot);
  r = mix64(r ^ gen);
  r = mix64(r ^ owner);
  for (int i = 0; i < kClaimFields; ++i) r = mix64(r ^ claim_fields(c)[i]);
  return r;
}

// ---- little-endian field hashing (lane_weave_qos.zig:4066-4146) ----------
void h_u8(gh::Sha256 &h, uint8_t v) { h.update(&v, 1); }
void h_u16(gh::Sha256 &h, uint16_t v) {
  const uint8_t b[2] = {(uint8_t)v, (uint8_t)(v >> 8)};
  h.update(b, 2);
}
void h_claim(gh::Sha256 &h, const Claim &c) {
  for (int i = 0; i < kClaimFields; ++i) h.u64(claim_fields(c)[i]);
}
void h_limits(gh::Sha256 &h, const Limits &l) {
  const uint64_t *f = &l.host_bytes;
  for (int i = 0; i < 11; ++i) h.u64(f[i]);
}
void h_spec(gh::Sha256 &h, const Spec &s) {
  h.u64(s.tenant_key);
  h.u64(s.request_key);
  h.u64(s.request_generation);
  h.u64(s.resource_owner_key);
  h_u16(h, (uint16_t)s.weight);
  h.u64(s.work_quanta);
  h.u64(s.deadline_tick);
  h_claim(h, s.claim);
}
void h_handle(gh::Sha256 &h, const Handle &x) {
  h.u64(x.scheduler_epoch);
  h.u32((uint32_t)x.slot_index);
  h.u64(x.slot_generation);
  h.u64(x.tenant_key);
  h.u64(x.request_key);
  h.u64(x.request_generation);
}
void h_receipt(gh::Sha256 &h, const Receipt &r) {
  h.u64(r.bank_epoch);
  h.u32((uint32_t)r.slot_index);
  h.u64(r.generation);
  h.u64(r.owner_key);
  h_claim(h, r.claim);
  h.u64(r.integrity);
}

void receipt_sha256(const Receipt &r, uint8_t out[32]) {
  // resourceReceiptSha256 (:3994-4002)
  static const char dom[] = "glacier-lane-weave-qos-resource-receipt-v1";
  gh::Sha256 h;
  h.update(dom, sizeof dom);  // includes the terminating NUL, as the domain does
  h_receipt(h, r);
  h.final(out);
}

using Permit = glacier_hip_service_permit_v1_t;

// servicePermitSha256 (:3557-3581)
void permit_sha256(const Permit &p, uint8_t out[32]) {
  static const char dom[] = "glacier-lane-weave-qos-service-permit-v1";
  gh::Sha256 h;
  h.update(dom, sizeof dom);
  h.u64(p.abi_version);
  h.u64(p.scheduler_epoch);
  h.u64(p.coordinator_id);
  h.u64(p.coordinator_address);
  h.u64(p.permit_generation);
  h.u64(p.event_sequence);
  h_handle(h, p.handle);
  h.u64(p.logical_tick_before);
  h.u32(p.cursor_before);
  h_u16(h, (uint16_t)p.level_before);
  h.u32(p.cursor_after);
  h_u16(h, (uint16_t)p.level_after);
  h.u64(p.remaining_before);
  h.u64(p.wait_quanta);
  h.u64(p.maximum_service_gap);
  h.update(p.state_before_sha256, 32);
  h.update(p.chain_head_before_sha256, 32);
  h_receipt(h, p.resource_receipt);
  h.update(p.resource_receipt_sha256, 32);
  h.final(out);
}

// Scheduler lifetimes (nextServiceCoordinatorId :556-566): a permit of an
// earlier scheduler at the same address is refused.
std::atomic<uint64_t> g_next_coordinator{1};

void event_sha256(const Event &e, uint8_t out[32]) {
  // eventSha256 (:4004-4038)
  static const char dom[] = "glacier-lane-weave-qos-event-v1";
  gh::Sha256 h;
  h.update(dom, sizeof dom);
  h.u64(e.abi_version);
  h.u64(e.scheduler_epoch);
  h.u64(e.event_sequence);
  h_u8(h, (uint8_t)e.kind);
  h_u8(h, (uint8_t)e.rejection_reason);
  h.update(e.previous_sha256, 32);
  h.update(e.state_before_sha256, 32);
  h.update(e.state_after_sha256, 32);
  h.u64(e.logical_tick_before);
  h.u64(e.logical_tick_after);
  h.u32(e.cursor_before);
  h.u32(e.cursor_after);
  h_u16(h, (uint16_t)e.level_before);
  h_u16(h, (uint16_t)e.level_after);
  h_handle(h, e.handle);
  h_spec(h, e.spec);
  h_receipt(h, e.resource_receipt);
  h.update(e.resource_receipt_sha256, 32);
  h.u64(e.remaining_before);
  h.u64(e.remaining_after);
  h.u64(e.wait_quanta);
  h.u64(e.maximum_service_gap);
  h.u32(e.active_before);
  h.u32(e.active_after);
  h.u32(e.finished_before);
  h.u32(e.finished_after);
  h_claim(h, e.bank_used_before);
  h_claim(h, e.bank_used_after);
  h.final(out);
}

enum SlotState : uint8_t { kFree = 0, kActive = 1, kFinished = 2 };

struct Slot {
  uint8_t state = kFree;
  uint64_t generation = 0;
  Spec spec{};
  uint64_t remaining = 0, admitted_tick = 0, last_service_tick = 0, service_count = 0;
  Receipt receipt{};
  uint8_t receipt_sha256[32] = {};
};

// One flat Bank slot (resource_bank.zig:146-158, the fields LaneWeave uses).
struct BankSlot {
  uint8_t state = 0;  // 0 free, 1 reserved, 2 committed
  uint64_t generation = 0, owner = 0, integrity = 0;
  Claim claim{};
};

// Projection scratch entry (ProjectionSlot :347-352).
struct Proj {
  bool active = false;
  uint16_t weight = 0;
  uint64_t remaining = 0, deadline = 0;
};

struct Budget {
  uint64_t remaining;
  bool exhausted = false;
  bool spend(uint64_t n) {
    if (n > remaining) {
      exhausted = true;
      return false;
    }
    remaining -= n;
    return true;
  }
};

struct Selection {
  uint32_t index, cursor_after;
  uint16_t level_after;
};

// selectIWRRWithBudget (:3444-3496) over (active, weight) accessors.
template <class Active, class Weight>
bool select_iwrr(size_t n, Active active, Weight weight, uint32_t cursor0, uint16_t level0,
                 uint16_t max_weight, Budget *budget, Selection *out) {
  if (n == 0) return false;
  if (budget && !budget->spend(n)) return false;
  uint16_t max_active = 0;
  for (size_t i = 0; i < n; ++i)
    if (active(i)) max_active = std::max(max_active, weight(i));
  if (max_active == 0) return false;
  size_t cursor = std::min<size_t>(cursor0, n);
  uint16_t level = level0 == 0 ? 1 : level0;
  if (level > max_active || level > max_weight) {
    level = 1;
    cursor = 0;
  }
  const uint64_t scan_limit = (uint64_t)n * max_weight;
  for (uint64_t scanned = 0; scanned < scan_limit; ++scanned) {
    if (budget && !budget->spend(1)) return false;
    if (cursor >= n) {
      cursor = 0;
      level = level >= max_active ? 1 : (uint16_t)(level + 1);
    }
    const size_t idx = cursor++;
    if (active(idx) && weight(idx) >= level) {
      *out = {(uint32_t)idx, (uint32_t)cursor, level};
      return true;
    }
  }
  return false;
}

enum ProjOutcome { kFeasible, kProjectionLimit, kDeadlineInfeasible };

}  // namespace

struct glacier_hip_lane_weave {
  std::mutex mu;
  // config
  uint64_t epoch = 0;
  uint8_t challenge[32] = {};
  uint16_t max_weight = 64;
  uint64_t max_pq = 0, max_po = 0;
  // dedicated flat Bank
  std::vector<BankSlot> bank;
  Limits limits{};
  uint64_t bank_epoch = 0;
  Claim bank_used{};
  uint64_t bank_next_generation = 1;
  // scheduler state
  std::vector<Slot> slots;
  std::vector<Proj> proj;
  Claim used{};
  uint64_t tick = 0, next_seq = 0, next_slot_generation = 1;
  uint32_t cursor = 0;
  uint16_t level = 1;
  uint64_t max_gap = 0;
  uint8_t chain_head[32] = {};
  bool poisoned = false, closed = false;
  // prepared service (pending_service :676): one permit at most
  uint64_t coordinator_id = 0, next_permit_generation = 1;
  bool pending = false;
  Permit pending_permit{};

  void counts(uint32_t *active, uint32_t *finished) const {
    *active = *finished = 0;
    for (const Slot &s : slots) {
      if (s.state == kActive) ++*active;
      if (s.state == kFinished) ++*finished;
    }
  }

  // schedulerStateSha256 (:3399-3427)
  void state_sha(uint8_t out[32]) const {
    static const char dom[] = "glacier-lane-weave-qos-state-v1";
    gh::Sha256 h;
    h.update(dom, sizeof dom);
    h.u64(epoch);
    h.u64(tick);
    h.u64(next_seq);
    h.u64(next_slot_generation);
    h.u32(cursor);
    h_u16(h, level);
    h_u8(h, poisoned ? 1 : 0);
    h_u8(h, closed ? 1 : 0);
    h_claim(h, used);
    h.u32((uint32_t)slots.size());
    for (const Slot &s : slots) {  // hashSlot :4066-4076
      h_u8(h, s.state);
      h.u64(s.generation);
      h_spec(h, s.spec);
      h.u64(s.remaining);
      h.u64(s.admitted_tick);
      h.u64(s.last_service_tick);
      h.u64(s.service_count);
      h_receipt(h, s.receipt);
      h.update(s.receipt_sha256, 32);
    }
    h.final(out);
  }

  Handle handle_for(size_t i) const {
    const Slot &s = slots[i];
    return Handle{epoch, i, s.generation, s.spec.tenant_key, s.spec.request_key,
                  s.spec.request_generation};
  }

  // What every event captures before a transition (EventSeed :2108-2126).
  struct Before {
    uint8_t state[32];
    uint64_t tick;
    uint32_t cursor;
    uint16_t level;
    uint32_t active, finished;
    Claim used;
  };
  Before before(const uint8_t *state = nullptr) const {  // state: its digest, if known
    Before b;
    if (state)
      memcpy(b.state, state, 32);
    else
      state_sha(b.state);
    b.tick = tick;
    b.cursor = cursor;
    b.level = level;
    counts(&b.active, &b.finished);
    b.used = used;
    return b;
  }

  // emitCurrent (:2128-2164)
  void emit(Event &e, uint32_t kind, const Before &b) {
    e.abi_version = kEventAbi;
    e.scheduler_epoch = epoch;
    e.event_sequence = next_seq++;
    e.kind = kind;
    memcpy(e.previous_sha256, chain_head, 32);
    memcpy(e.state_before_sha256, b.state, 32);
    state_sha(e.state_after_sha256);
    e.logical_tick_before = b.tick;
    e.logical_tick_after = tick;
    e.cursor_before = b.cursor;
    e.cursor_after = cursor;
    e.level_before = b.level;
    e.level_after = level;
    e.maximum_service_gap = max_gap;
    e.active_before = b.active;
    e.finished_before = b.finished;
    counts(&e.active_after, &e.finished_after);
    e.bank_used_before = b.used;
    e.bank_used_after = used;
    event_sha256(e, e.event_sha256);
    memcpy(chain_head, e.event_sha256, 32);
  }

  ProjOutcome project_prepared(size_t deadline_count, Budget &budget) {
    // projectPreparedState (:3239-3289)
    if (deadline_count == 0) return kFeasible;
    uint64_t t = tick, pq = 0;
    uint32_t cur = cursor;
    uint16_t lvl = level;
    while (deadline_count != 0) {
      if (pq >= max_pq) return kProjectionLimit;
      if (!budget.spend(proj.size())) return kProjectionLimit;
      for (const Proj &p : proj)
        if (p.active && p.deadline != 0 && t >= p.deadline) return kDeadlineInfeasible;
      Selection sel;
      if (!select_iwrr(
              proj.size(), [&](size_t i) { return proj[i].active; },
              [&](size_t i) { return proj[i].weight; }, cur, lvl, max_weight, &budget, &sel))
        return budget.exhausted ? kProjectionLimit : kDeadlineInfeasible;
      Proj &p = proj[sel.index];
      p.remaining -= 1;
      if (t == kU64Max) return kDeadlineInfeasible;
      t += 1;
      pq += 1;
      if (p.remaining == 0) {
        if (p.deadline != 0 && t > p.deadline) return kDeadlineInfeasible;
        if (p.deadline != 0) deadline_count -= 1;
        p.active = false;
      }
      cur = sel.cursor_after;
      lvl = sel.level_after;
    }
    return kFeasible;
  }

  ProjOutcome project_admission(size_t cand, const Spec &sp) {
    // projectAdmissionState (:3160-3237)
    Budget budget{max_po};
    if (sp.deadline_tick != 0 && sp.work_quanta > max_pq) return kProjectionLimit;
    if (sp.deadline_tick == 0) {
      if (!budget.spend(slots.size())) return kProjectionLimit;
      bool existing = false;
      for (const Slot &s : slots)
        if (s.state == kActive && s.spec.deadline_tick != 0) {
          existing = true;
          break;
        }
      if (!existing) return kFeasible;
    }
    if (!budget.spend(slots.size())) return kProjectionLimit;
    size_t dc = 0;
    uint64_t mq = 0;
    for (size_t i = 0; i < slots.size(); ++i) {
      const Slot &s = slots[i];
      if (s.state == kActive) {
        proj[i] = Proj{true, (uint16_t)s.spec.weight, s.remaining, s.spec.deadline_tick};
        if (s.spec.deadline_tick != 0) {
          ++dc;
          if (mq > kU64Max - s.remaining) return kProjectionLimit;
          mq += s.remaining;
        }
      } else {
        proj[i] = Proj{};
      }
    }
    proj[cand] = Proj{true, (uint16_t)sp.weight, sp.work_quanta, sp.deadline_tick};
    if (sp.deadline_tick != 0) {
      ++dc;
      if (mq > kU64Max - sp.work_quanta) return kProjectionLimit;
      mq += sp.work_quanta;
    }
    if (mq > max_pq) return kProjectionLimit;
    return project_prepared(dc, budget);
  }

  bool next_selection(uint32_t cur, uint16_t lvl, const std::vector<uint8_t> &active,
                      Selection *sel) const {
    return select_iwrr(
        slots.size(), [&](size_t i) { return active[i] != 0; },
        [&](size_t i) { return (uint16_t)slots[i].spec.weight; }, cur, lvl, max_weight, nullptr,
        sel);
  }
};

namespace {

int finish_handle(glacier_hip_lane_weave *lw, const Handle *h, uint32_t kind, uint8_t required,
                  Event *out) {
  // finishHandleLocked (:1964-2014)
  if (!lw || !h || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lk(lw->mu);
  if (lw->poisoned) return GLACIER_HIP_SCHEDULER_POISONED;
  if (lw->closed) return GLACIER_HIP_SCHEDULER_CLOSED;
  if (lw->pending) return GLACIER_HIP_SERVICE_IN_FLIGHT;
  if (h->scheduler_epoch != lw->epoch || h->slot_index >= lw->slots.size())
    return GLACIER_HIP_STALE_HANDLE;
  const size_t i = (size_t)h->slot_index;
  Slot &s = lw->slots[i];
  if (s.state != required || s.generation != h->slot_generation ||
      s.spec.tenant_key != h->tenant_key || s.spec.request_key != h->request_key ||
      s.spec.request_generation != h->request_generation)
    return GLACIER_HIP_STALE_HANDLE;
  const auto b = lw->before();
  Event e{};
  e.handle = *h;
  e.spec = s.spec;
  e.resource_receipt = s.receipt;
  memcpy(e.resource_receipt_sha256, s.receipt_sha256, 32);
  e.remaining_before = s.remaining;
  // Bank.release (resource_bank.zig:3166): the receipt's slot becomes free
  BankSlot &bs = lw->bank[(size_t)s.receipt.slot_index];
  Claim bank_after{}, used_after{};
  if (bs.state != 2 || bs.generation != s.receipt.generation ||
      !sub_claims(lw->bank_used, s.receipt.claim, &bank_after) ||
      !sub_claims(lw->used, s.spec.claim, &used_after)) {
    lw->poisoned = true;
    return GLACIER_HIP_SCHEDULER_POISONED;
  }
  bs = BankSlot{};
  lw->bank_used = bank_after;
  lw->used = used_after;
  s = Slot{};
  lw->emit(e, kind, b);
  *out = e;
  return GLACIER_HIP_OK;
}

}  // namespace

extern "C" {

glacier_hip_lane_weave *glacier_hip_lane_weave_create(
    uint32_t capacity, const glacier_hip_limits_t *bank_limits, uint64_t bank_epoch,
    uint64_t scheduler_epoch, const uint8_t challenge[32], uint32_t max_weight,
    uint64_t max_projection_quanta, uint64_t max_projection_operations) {
  // Scheduler.initWithBankStorage (:634-735)
  static const uint8_t zero[32] = {};
  if (capacity == 0 || !bank_limits || !challenge || scheduler_epoch == 0 || max_weight == 0 ||
      max_weight > 0xFFFF || max_projection_quanta == 0 || max_projection_operations == 0 ||
      memcmp(challenge, zero, 32) == 0)
    return nullptr;
  const unsigned __int128 gap = (unsigned __int128)(capacity - 1) * max_weight + 1;
  if (gap > kU64Max) return nullptr;
  auto *lw = new glacier_hip_lane_weave();
  lw->epoch = scheduler_epoch;
  memcpy(lw->challenge, challenge, 32);
  lw->max_weight = (uint16_t)max_weight;
  lw->max_pq = max_projection_quanta;
  lw->max_po = max_projection_operations;
  lw->bank.assign(capacity, BankSlot{});
  lw->limits = *bank_limits;
  lw->bank_epoch = bank_epoch;
  lw->slots.assign(capacity, Slot{});
  lw->proj.assign(capacity, Proj{});
  lw->max_gap = (uint64_t)gap;
  // initialRoot (:4040-4064)
  static const char dom[] = "glacier-lane-weave-qos-root-v1";
  gh::Sha256 h;
  h.update(dom, sizeof dom);
  h.u64(kAbi);
  h.u64(kEventAbi);
  h.u64(kBankAbi);
  h.u64(scheduler_epoch);
  h.update(challenge, 32);
  h_u16(h, (uint16_t)max_weight);
  h.u64(max_projection_quanta);
  h.u64(max_projection_operations);
  h.u32(capacity);
  h.u64(bank_epoch);
  h_limits(h, *bank_limits);
  h.u64(lw->max_gap);
  h.final(lw->chain_head);
  lw->coordinator_id = g_next_coordinator.fetch_add(1);
  return lw;
}

void glacier_hip_lane_weave_destroy(glacier_hip_lane_weave *lw) { delete lw; }

int glacier_hip_lane_weave_admit(glacier_hip_lane_weave *lw, const glacier_hip_request_spec_t *spec,
                                 int *admitted, glacier_hip_lane_handle_t *handle_out,
                                 glacier_hip_lane_event_t *event_out) {
  // admitLocked (:748-900)
  if (!lw || !spec || !admitted || !event_out) return GLACIER_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lk(lw->mu);
  if (lw->poisoned) return GLACIER_HIP_SCHEDULER_POISONED;
  if (lw->closed) return GLACIER_HIP_SCHEDULER_CLOSED;
  if (lw->pending) return GLACIER_HIP_SERVICE_IN_FLIGHT;
  const Spec &sp = *spec;
  uint64_t hb;
  // validateRequestSpec (:3145-3158)
  if (sp.tenant_key == 0 || sp.request_key == 0 || sp.request_generation == 0 ||
      sp.resource_owner_key == 0 || sp.weight == 0 || sp.weight > lw->max_weight ||
      sp.work_quanta == 0 || claim_zero(sp.claim) || sp.claim.queue_slots != 1 ||
      (sp.deadline_tick != 0 && sp.deadline_tick <= lw->tick) || !host_bytes(sp.claim, &hb))
    return GLACIER_HIP_INVALID_ARGUMENT;
  const auto b = lw->before();
  Event e{};
  auto reject = [&](uint32_t reason) {
    e.spec = sp;
    e.rejection_reason = reason;
    lw->emit(e, GLACIER_HIP_EVENT_ADMISSION_REJECTED, b);
    *admitted = 0;
    *event_out = e;
    return GLACIER_HIP_OK;
  };
  int free_index = -1;
  for (size_t i = 0; i < lw->slots.size(); ++i) {
    const Slot &s = lw->slots[i];
    if (s.state != kFree && s.spec.tenant_key == sp.tenant_key)
      return reject(GLACIER_HIP_REJECT_DUPLICATE_TENANT);
    if (s.state == kFree && free_index < 0) free_index = (int)i;
  }
  if (free_index < 0) return reject(GLACIER_HIP_REJECT_NO_SLOT);
  Claim next{};
  if (!add_claims(lw->used, sp.claim, &next) || !fits(lw->limits, next))
    return reject(GLACIER_HIP_REJECT_RESOURCE_LIMIT);
  switch (lw->project_admission((size_t)free_index, sp)) {
    case kProjectionLimit: return reject(GLACIER_HIP_REJECT_PROJECTION_LIMIT);
    case kDeadlineInfeasible: return reject(GLACIER_HIP_REJECT_DEADLINE_INFEASIBLE);
    case kFeasible: break;
  }
  // Bank.reserve + Bank.commit (resource_bank.zig:976-1070): the first free
  // Bank slot, which is the scheduler's free slot (both are kept one-to-one)
  int bi = -1;
  for (size_t i = 0; i < lw->bank.size(); ++i)
    if (lw->bank[i].state == 0) {
      bi = (int)i;
      break;
    }
  Claim bank_next{};
  if (bi != free_index || !add_claims(lw->bank_used, sp.claim, &bank_next) ||
      lw->bank_next_generation != lw->next_slot_generation) {
    lw->poisoned = true;
    return GLACIER_HIP_SCHEDULER_POISONED;
  }
  const uint64_t gen = lw->bank_next_generation++;
  Receipt r{};
  r.bank_epoch = lw->bank_epoch;
  r.slot_index = (uint64_t)bi;
  r.generation = gen;
  r.owner_key = sp.resource_owner_key;
  r.claim = sp.claim;
  r.integrity = token_integrity(lw->bank_epoch, (uint32_t)bi, gen, sp.resource_owner_key, sp.claim,
                                kReceiptDomain);
  BankSlot &bs = lw->bank[(size_t)bi];
  bs.state = 2;
  bs.generation = gen;
  bs.owner = sp.resource_owner_key;
  bs.claim = sp.claim;
  bs.integrity = r.integrity;
  (void)kReservationDomain;  // the reserve-time integrity is replaced at commit
  lw->bank_used = bank_next;
  lw->next_slot_generation += 1;
  Slot &s = lw->slots[(size_t)free_index];
  s.state = kActive;
  s.generation = gen;
  s.spec = sp;
  s.remaining = sp.work_quanta;
  s.admitted_tick = lw->tick;
  s.last_service_tick = lw->tick;
  s.service_count = 0;
  s.receipt = r;
  receipt_sha256(r, s.receipt_sha256);
  lw->used = next;
  e.handle = lw->handle_for((size_t)free_index);
  e.spec = sp;
  e.resource_receipt = r;
  memcpy(e.resource_receipt_sha256, s.receipt_sha256, 32);
  e.remaining_after = sp.work_quanta;
  lw->emit(e, GLACIER_HIP_EVENT_ADMISSION_ACCEPTED, b);
  *admitted = 1;
  if (handle_out) *handle_out = e.handle;
  *event_out = e;
  return GLACIER_HIP_OK;
}

}  // extern "C"

namespace {

// serveOne (:1196-1270) with lw->mu held.
// The selection serveOne / prepareService make (lw->mu held): the next IWRR
// slot, its wait, and the checks that poison the scheduler (a deadline the
// selection breaks :3340-3355, a service gap over the bound).
int select_service_locked(glacier_hip_lane_weave *lw, Selection *sel, uint64_t *wait) {
  if (lw->tick == kU64Max) return GLACIER_HIP_SCHEDULER_POISONED;
  std::vector<uint8_t> active(lw->slots.size());
  for (size_t i = 0; i < active.size(); ++i) active[i] = lw->slots[i].state == kActive;
  if (!lw->next_selection(lw->cursor, lw->level, active, sel)) return GLACIER_HIP_NO_RUNNABLE;
  const Slot &s = lw->slots[sel->index];
  const uint64_t after_tick = lw->tick + 1;
  for (size_t j = 0; j < lw->slots.size(); ++j) {
    const Slot &o = lw->slots[j];
    if (o.state != kActive || o.spec.deadline_tick == 0) continue;
    const bool completes = j == sel->index && o.remaining == 1;
    if ((completes && after_tick > o.spec.deadline_tick) ||
        (!completes && after_tick >= o.spec.deadline_tick)) {
      lw->poisoned = true;
      return GLACIER_HIP_SCHEDULER_POISONED;
    }
  }
  *wait = after_tick - s.last_service_tick;
  if (*wait > lw->max_gap) {
    lw->poisoned = true;
    return GLACIER_HIP_SCHEDULER_POISONED;
  }
  return GLACIER_HIP_OK;
}

// serveOne (:1196-1270) with lw->mu held.
int serve_one_locked(glacier_hip_lane_weave *lw, glacier_hip_lane_event_t *out,
                     const Selection *pre = nullptr, uint64_t pre_wait = 0,
                     const uint8_t *pre_state = nullptr) {
  // (pre: the selection, wait and state digest a permit's commit has just
  // validated against the current state)
  if (lw->poisoned) return GLACIER_HIP_SCHEDULER_POISONED;
  if (lw->closed) return GLACIER_HIP_SCHEDULER_CLOSED;
  Selection sel;
  uint64_t wait = 0;
  if (pre) {
    sel = *pre;
    wait = pre_wait;
  } else if (int rc = select_service_locked(lw, &sel, &wait)) {
    return rc;
  }
  Slot &s = lw->slots[sel.index];
  const uint64_t after_tick = lw->tick + 1;
  const auto b = lw->before(pre_state);
  Event e{};
  e.handle = lw->handle_for(sel.index);
  e.spec = s.spec;
  e.resource_receipt = s.receipt;
  memcpy(e.resource_receipt_sha256, s.receipt_sha256, 32);
  e.remaining_before = s.remaining;
  e.wait_quanta = wait;
  s.remaining -= 1;
  s.last_service_tick = after_tick;
  s.service_count += 1;
  if (s.remaining == 0) s.state = kFinished;
  lw->tick = after_tick;
  lw->cursor = sel.cursor_after;
  lw->level = sel.level_after;
  e.remaining_after = s.remaining;
  lw->emit(e, GLACIER_HIP_EVENT_SERVICE, b);
  *out = e;
  return GLACIER_HIP_OK;
}

// prepareService (:1127-1192) with lw->mu held: the next selection frozen
// into a permit; nothing logical changes.
int prepare_service_locked(glacier_hip_lane_weave *lw, Permit *out) {
  if (lw->poisoned) return GLACIER_HIP_SCHEDULER_POISONED;
  if (lw->closed) return GLACIER_HIP_SCHEDULER_CLOSED;
  if (lw->pending) return GLACIER_HIP_SERVICE_IN_FLIGHT;
  if (lw->next_permit_generation == 0 || lw->next_permit_generation == kU64Max)
    return GLACIER_HIP_INVALID_TRANSACTION;  // GenerationOverflow
  Selection sel;
  uint64_t wait = 0;
  if (int rc = select_service_locked(lw, &sel, &wait)) return rc;
  const Slot &s = lw->slots[sel.index];
  if (s.service_count == kU64Max) return GLACIER_HIP_INVALID_TRANSACTION;  // ServiceOverflow
  Permit p;
  memset(&p, 0, sizeof p);
  p.abi_version = kPermitAbi;
  p.scheduler_epoch = lw->epoch;
  p.coordinator_id = lw->coordinator_id;
  p.coordinator_address = (uint64_t)(uintptr_t)lw;
  p.permit_generation = lw->next_permit_generation;
  p.event_sequence = lw->next_seq;
  p.handle = lw->handle_for(sel.index);
  p.logical_tick_before = lw->tick;
  p.cursor_before = lw->cursor;
  p.level_before = lw->level;
  p.cursor_after = sel.cursor_after;
  p.level_after = sel.level_after;
  p.remaining_before = s.remaining;
  p.wait_quanta = wait;
  p.maximum_service_gap = lw->max_gap;
  lw->state_sha(p.state_before_sha256);
  memcpy(p.chain_head_before_sha256, lw->chain_head, 32);
  p.resource_receipt = s.receipt;
  memcpy(p.resource_receipt_sha256, s.receipt_sha256, 32);
  permit_sha256(p, p.permit_sha256);
  lw->next_permit_generation += 1;
  lw->pending = true;
  lw->pending_permit = p;
  *out = p;
  return GLACIER_HIP_OK;
}

// validatePendingService (:2461-2487): exactly the pending permit, its digest
// recomputing; a pending permit whose own digest no longer does poisons.
int validate_pending_locked(glacier_hip_lane_weave *lw, const Permit &p) {
  if (!lw->pending) return GLACIER_HIP_STALE_SERVICE_PERMIT;
  uint8_t d[32];
  permit_sha256(lw->pending_permit, d);
  if (memcmp(d, lw->pending_permit.permit_sha256, 32) != 0) {
    lw->poisoned = true;
    return GLACIER_HIP_SCHEDULER_POISONED;
  }
  permit_sha256(p, d);
  if (p.abi_version != kPermitAbi || p.scheduler_epoch != lw->epoch ||
      p.coordinator_id != lw->coordinator_id ||
      p.coordinator_address != (uint64_t)(uintptr_t)lw || p.permit_generation == 0 ||
      memcmp(d, p.permit_sha256, 32) != 0 || memcmp(&p, &lw->pending_permit, sizeof p) != 0)
    return GLACIER_HIP_STALE_SERVICE_PERMIT;
  return GLACIER_HIP_OK;
}

// validateServiceBeforeState (:2512-2531): nothing logical moved since prepare.
int validate_before_state_locked(glacier_hip_lane_weave *lw, const Permit &p,
                                 uint8_t *state_out = nullptr) {
  uint8_t st[32];
  lw->state_sha(st);
  if (state_out) memcpy(state_out, st, 32);
  if (memcmp(st, p.state_before_sha256, 32) != 0 || p.event_sequence != lw->next_seq ||
      p.logical_tick_before != lw->tick || memcmp(p.chain_head_before_sha256, lw->chain_head, 32) != 0) {
    lw->poisoned = true;
    return GLACIER_HIP_SCHEDULER_POISONED;
  }
  return GLACIER_HIP_OK;
}

// commitService (:1272-1286 with validateServiceCommitLocked :2542-2600 and
// commitServiceLocked :2617-2663): the serveOne transition of the permit's
// selection, emitting the same Event-v1.
int commit_service_locked(glacier_hip_lane_weave *lw, const Permit &p, Event *out) {
  if (lw->poisoned) return GLACIER_HIP_SCHEDULER_POISONED;
  if (lw->closed) return GLACIER_HIP_SCHEDULER_CLOSED;
  if (int rc = validate_pending_locked(lw, p)) return rc;
  uint8_t state[32];
  if (int rc = validate_before_state_locked(lw, p, state)) return rc;
  Selection sel;
  uint64_t wait = 0;
  int rc = select_service_locked(lw, &sel, &wait);
  const Slot &s = lw->slots[p.handle.slot_index < lw->slots.size() ? p.handle.slot_index : 0];
  if (rc || sel.index != p.handle.slot_index || sel.cursor_after != p.cursor_after ||
      sel.level_after != p.level_after || wait != p.wait_quanta || s.state != kActive ||
      s.generation != p.handle.slot_generation || s.remaining != p.remaining_before ||
      memcmp(&s.receipt, &p.resource_receipt, sizeof s.receipt) != 0 ||
      memcmp(s.receipt_sha256, p.resource_receipt_sha256, 32) != 0) {
    lw->poisoned = true;
    return GLACIER_HIP_SCHEDULER_POISONED;
  }
  lw->pending = false;
  return serve_one_locked(lw, out, &sel, wait, state);
}

// abortService (:1438-1452): the pending permit consumed, nothing logical changes.
int abort_service_locked(glacier_hip_lane_weave *lw, const Permit &p) {
  if (lw->poisoned) return GLACIER_HIP_SCHEDULER_POISONED;
  if (lw->closed) return GLACIER_HIP_SCHEDULER_CLOSED;
  if (int rc = validate_pending_locked(lw, p)) return rc;
  if (int rc = validate_before_state_locked(lw, p)) return rc;
  lw->pending = false;
  return GLACIER_HIP_OK;
}

// The slots the next serve_one calls select (lw->mu held): replays the
// serve_one transitions on copies of the mutable selection state (cursor,
// level, tick, remaining quanta, last service) and stops before a slot would
// repeat or before a quantum whose serve_one would poison the scheduler
// (a deadline it cannot keep, a service gap over the budget), so every
// planned quantum commits.
int plan_wave_locked(glacier_hip_lane_weave *lw, uint32_t max_count, uint32_t *slots_out,
                     uint32_t *count_out) {
  *count_out = 0;
  if (lw->poisoned) return GLACIER_HIP_SCHEDULER_POISONED;
  if (lw->closed) return GLACIER_HIP_SCHEDULER_CLOSED;
  if (lw->pending) return GLACIER_HIP_SERVICE_IN_FLIGHT;
  const size_t n = lw->slots.size();
  std::vector<uint8_t> active(n), taken(n, 0);
  std::vector<uint64_t> remaining(n), last(n);
  for (size_t i = 0; i < n; ++i) {
    active[i] = lw->slots[i].state == kActive;
    remaining[i] = lw->slots[i].remaining;
    last[i] = lw->slots[i].last_service_tick;
  }
  uint32_t cur = lw->cursor;
  uint16_t lvl = lw->level;
  uint64_t tick = lw->tick;
  while (*count_out < max_count && tick != kU64Max) {
    Selection sel;
    if (!lw->next_selection(cur, lvl, active, &sel)) break;
    if (taken[sel.index]) break;
    const uint64_t after_tick = tick + 1;
    bool keeps = after_tick - last[sel.index] <= lw->max_gap;
    for (size_t j = 0; j < n && keeps; ++j) {
      const uint64_t dl = lw->slots[j].spec.deadline_tick;
      if (!active[j] || dl == 0) continue;
      const bool completes = j == sel.index && remaining[j] == 1;
      if ((completes && after_tick > dl) || (!completes && after_tick >= dl)) keeps = false;
    }
    if (!keeps) break;
    taken[sel.index] = 1;
    slots_out[(*count_out)++] = sel.index;
    if (--remaining[sel.index] == 0) active[sel.index] = 0;
    last[sel.index] = after_tick;
    tick = after_tick;
    cur = sel.cursor_after;
    lvl = sel.level_after;
  }
  return GLACIER_HIP_OK;
}

}  // namespace

namespace gh {

int lane_weave_run_wave(glacier_hip_lane_weave *lw, uint32_t max_count, const WaveOps &ops,
                        uint32_t *slots_out, glacier_hip_lane_event_t *events_out,
                        uint32_t *count_out) {
  std::lock_guard<std::mutex> lk(lw->mu);
  *count_out = 0;
  std::vector<uint32_t> plan(max_count);
  uint32_t n = 0;
  int rc = plan_wave_locked(lw, max_count, plan.data(), &n);
  if (rc) return rc;
  if (n == 0) return GLACIER_HIP_NO_RUNNABLE;
  rc = ops.run(plan.data(), n);
  if (rc) return rc;  // nothing published, the scheduler unchanged
  if (ops.sink && (rc = ops.sink())) {
    ops.abort(0);
    return rc;
  }
  for (uint32_t i = 0; i < n; ++i) {
    Permit p;
    rc = prepare_service_locked(lw, &p);
    if (rc || p.handle.slot_index != plan[i]) {
      if (!rc) (void)abort_service_locked(lw, p);
      ops.abort(i);
      lw->poisoned = true;
      return GLACIER_HIP_SCHEDULER_POISONED;
    }
    rc = ops.publish(i);
    if (rc) {
      (void)abort_service_locked(lw, p);
      ops.abort(i);
      if (i > 0) {  // earlier quanta are published: the wave cannot be undone
        lw->poisoned = true;
        return GLACIER_HIP_SCHEDULER_POISONED;
      }
      return rc;
    }
    glacier_hip_lane_event_t ev;
    rc = commit_service_locked(lw, p, &ev);
    if (rc) {  // published but not served
      ops.abort(i + 1);
      lw->poisoned = true;
      return GLACIER_HIP_SCHEDULER_POISONED;
    }
    if (slots_out) slots_out[i] = plan[i];
    if (events_out) events_out[i] = ev;
    *count_out = i + 1;
  }
  return GLACIER_HIP_OK;
}

}  // namespace gh

extern "C" {

int glacier_hip_lane_weave_serve_one(glacier_hip_lane_weave *lw, glacier_hip_lane_event_t *out) {
  if (!lw || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lk(lw->mu);
  if (!lw->poisoned && !lw->closed && lw->pending) return GLACIER_HIP_SERVICE_IN_FLIGHT;
  return serve_one_locked(lw, out);
}

int glacier_hip_lane_weave_prepare_service(glacier_hip_lane_weave *lw,
                                           glacier_hip_service_permit_v1_t *out) {
  if (!lw || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lk(lw->mu);
  return prepare_service_locked(lw, out);
}

int glacier_hip_lane_weave_commit_service(glacier_hip_lane_weave *lw,
                                          const glacier_hip_service_permit_v1_t *p,
                                          glacier_hip_lane_event_t *out) {
  if (!lw || !p || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lk(lw->mu);
  return commit_service_locked(lw, *p, out);
}

int glacier_hip_lane_weave_abort_service(glacier_hip_lane_weave *lw,
                                         const glacier_hip_service_permit_v1_t *p) {
  if (!lw || !p) return GLACIER_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lk(lw->mu);
  return abort_service_locked(lw, *p);
}

int glacier_hip_service_permit_sha256(const glacier_hip_service_permit_v1_t *p, uint8_t out[32]) {
  if (!p || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  permit_sha256(*p, out);
  return GLACIER_HIP_OK;
}

int glacier_hip_lane_weave_plan_wave(glacier_hip_lane_weave *lw, uint32_t max_count,
                                     uint32_t *slots_out, uint32_t *count_out) {
  if (!lw || !slots_out || !count_out) return GLACIER_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lk(lw->mu);
  return plan_wave_locked(lw, max_count, slots_out, count_out);
}

int glacier_hip_lane_weave_retire(glacier_hip_lane_weave *lw, const glacier_hip_lane_handle_t *h,
                                  glacier_hip_lane_event_t *out) {
  return finish_handle(lw, h, GLACIER_HIP_EVENT_RETIRE, kFinished, out);
}

int glacier_hip_lane_weave_cancel(glacier_hip_lane_weave *lw, const glacier_hip_lane_handle_t *h,
                                  glacier_hip_lane_event_t *out) {
  return finish_handle(lw, h, GLACIER_HIP_EVENT_CANCEL, kActive, out);
}

int glacier_hip_lane_weave_close(glacier_hip_lane_weave *lw, glacier_hip_lane_event_t *out) {
  // close (:1923-1952)
  if (!lw || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lk(lw->mu);
  if (lw->poisoned) return GLACIER_HIP_SCHEDULER_POISONED;
  if (lw->closed) return GLACIER_HIP_SCHEDULER_CLOSED;
  if (lw->pending) return GLACIER_HIP_SERVICE_IN_FLIGHT;
  uint32_t a, f;
  lw->counts(&a, &f);
  if (a || f || !claim_zero(lw->used)) return GLACIER_HIP_INCOMPLETE_DRAIN;
  auto b = lw->before();
  b.active = b.finished = 0;
  lw->closed = true;
  Event e{};
  lw->emit(e, GLACIER_HIP_EVENT_CLOSE, b);
  *out = e;
  return GLACIER_HIP_OK;
}

int glacier_hip_lane_weave_slot(glacier_hip_lane_weave *lw, uint32_t slot,
                                glacier_hip_lane_handle_t *handle_out, uint32_t *state_out,
                                uint64_t *remaining_out) {
  if (!lw) return GLACIER_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lk(lw->mu);
  if (slot >= lw->slots.size()) return GLACIER_HIP_SHAPE_MISMATCH;
  if (handle_out) *handle_out = lw->handle_for(slot);
  if (state_out) *state_out = lw->slots[slot].state;
  if (remaining_out) *remaining_out = lw->slots[slot].remaining;
  return GLACIER_HIP_OK;
}

int glacier_hip_lane_weave_chain_head(glacier_hip_lane_weave *lw, uint8_t out[32]) {
  if (!lw || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lk(lw->mu);
  memcpy(out, lw->chain_head, 32);
  return GLACIER_HIP_OK;
}

int glacier_hip_lane_weave_state_sha256(glacier_hip_lane_weave *lw, uint8_t out[32]) {
  if (!lw || !out) return GLACIER_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lk(lw->mu);
  lw->state_sha(out);
  return GLACIER_HIP_OK;
}

}  // extern "C"
