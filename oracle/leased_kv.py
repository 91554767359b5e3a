"""Restatement of the reference's LeaseTree page ownership for paged KV.

TEST INFRASTRUCTURE ONLY: the checker for glacier-engine_amd/csrc/lease_bank.cpp
and leased_kv.cpp (through the C ABI). Only tests/ use it.

Follows /root/reference/src/core/resource_bank.zig:
  reserve / commit / release            :976-1076, :3166-3184
  openLeaseTree / openLeaseScope        :1404-1514
  reserveAllocationsForSession          :1575-1783 (additive funding)
  commitAllocationsAfterAllocate        :1785-1823
  abortAllocationsAfterFree             :1909-1956
  beginRetireSubtreeForSession          :2227-2343
  cancelRetire / authorizeFree          :2345-2452
  commitFreeAfterAllocatorFree          :2454-2502
  closeLeaseTree                        :2582-2622
  publication sessions                  :2731-2750, :2938-3124
and /root/reference/src/leased_paged_kv_cache.zig:
  init :311-357, bindingSummaryForState :1178-1250, planNextRow :453-480,
  beginRowPlanned :482-565, commitRowTxn/abortRowTxn :666-689,
  sealTerminalForPublication :691-757, beginTerminalReclaim :852-867,
  beginReclaimExact :918-1036, commitReclaimAfterFree :1040-1080,
  reclaimForTeardown :894-916,
over oracle.paged_kv.PagedKVCache with the retirement plan of
paged_kv_cache.zig:1187-1250.

Tokens here are frozen snapshots of the state they name and are validated by
comparing every field with the current state (the reference additionally
carries integrity words; the product carries its own). Generations come from
one bank-wide counter in the reference's reservation order, so the generation
fields of trees, nodes and decisions are comparable with the product's.
"""
import copy
import hashlib
import struct

from oracle import paged_kv as pk

CLASSES = ("capsule_bytes", "kv_bytes", "activation_bytes", "partial_bytes", "logits_bytes",
           "output_journal_bytes", "staging_bytes", "device_bytes", "io_bytes", "queue_slots")
HOST_CLASSES = CLASSES[:7]
U64 = 2**64 - 1
NO_NODE = 0xFFFFFFFF


class LeaseFailure(Exception):
    """An error of the reference, by name (e.g. 'InvalidBinding')."""

    def __init__(self, reason):
        self.reason = reason
        super().__init__(reason)


def fail(reason):
    raise LeaseFailure(reason)


class Claim:
    __slots__ = CLASSES

    def __init__(self, **kw):
        for c in CLASSES:
            setattr(self, c, kw.get(c, 0))

    def t(self):
        return tuple(getattr(self, c) for c in CLASSES)

    def zero(self):
        return not any(self.t())

    def __add__(self, o):
        v = [a + b for a, b in zip(self.t(), o.t())]
        if any(x > U64 for x in v):
            fail("ClaimOverflow")
        return Claim(**dict(zip(CLASSES, v)))

    def __sub__(self, o):
        v = [a - b for a, b in zip(self.t(), o.t())]
        if any(x < 0 for x in v):
            fail("ClaimOverflow")
        return Claim(**dict(zip(CLASSES, v)))

    def within(self, ceiling):
        return all(a <= b for a, b in zip(self.t(), ceiling.t()))

    def __eq__(self, o):
        return self.t() == o.t()

    def host(self):
        return sum(getattr(self, c) for c in HOST_CLASSES)


class Tree:
    """LeaseTreeV1 as a mutable cell (the cohort shares one)."""

    def __init__(self, **kw):
        self.__dict__.update(kw)

    def key(self):
        return (self.slot, self.receipt_gen, self.tree_key, self.identity_generation,
                self.generation, self.structural_revision, self.current.t(), self.active_nodes,
                self.state)

    def assign(self, other):
        self.__dict__.update(other.__dict__)


class Node:
    def __init__(self, **kw):
        self.__dict__.update(kw)

    def key(self):
        return (self.slot, self.tree_identity_generation, self.node_index, self.generation,
                self.parent_index, self.parent_generation, self.node_key, self.tenant_key,
                self.binding_key, self.kind, self.claim.t())


class Bank:
    def __init__(self, slots, nodes, epoch, **limits):
        self.epoch = epoch
        self.limits = {k: limits.get(k, U64) for k in ("host_bytes",) + CLASSES}
        self.slots = [None] * slots          # dicts
        self.roots = [None] * slots
        self.nodes = [None] * nodes
        self.used = Claim()
        self.next_generation = 1
        self.next_lease_generation = 1
        self.counters = {k: 0 for k in (
            "successful_reservations", "successful_commits", "cancellations", "releases",
            "rejected_capacity", "rejected_slots", "lease_tree_opens", "lease_scope_opens",
            "lease_allocation_reserves", "lease_allocation_materializations",
            "lease_allocation_aborts", "lease_reclaim_prepares", "lease_reclaim_authorizations",
            "lease_reclaim_cancels", "lease_reclaim_commits", "lease_tree_closes",
            "rejected_lease_capacity", "rejected_lease_nodes")}

    # -- receipts ----------------------------------------------------------------
    def _fits(self, c):
        return c.host() <= self.limits["host_bytes"] and all(
            getattr(c, k) <= self.limits[k] for k in CLASSES)

    def reserve(self, owner_key, **claim):
        c = Claim(**claim)
        if owner_key == 0 or c.zero():
            fail("InvalidClaim")
        nxt = self.used + c
        if not self._fits(nxt):
            self.counters["rejected_capacity"] += 1
            fail("CapacityExceeded")
        idx = next((i for i, s in enumerate(self.slots) if s is None), None)
        if idx is None:
            self.counters["rejected_slots"] += 1
            fail("ReservationSlotsExhausted")
        gen = self.next_generation
        self.next_generation += 1
        self.slots[idx] = dict(state="reserved", gen=gen, owner=owner_key, claim=c, pub_epoch=0,
                               pub_session=0, pub_next=0, pub_active=False, pub_gen=0)
        self.used = nxt
        self.counters["successful_reservations"] += 1
        return ("reserved", idx, gen, owner_key, c.t())

    def _slot(self, r, state):
        kind, idx, gen, owner, claim = r
        s = self.slots[idx] if idx < len(self.slots) else None
        if s is None or s["state"] != kind or s["gen"] != gen or s["owner"] != owner or \
                s["claim"].t() != claim:
            fail("StaleReservation")
        if state and s["state"] != state:
            fail("InvalidTransition")
        return s

    def commit(self, r):
        s = self._slot(r, "reserved")
        s["state"] = "committed"
        self.counters["successful_commits"] += 1
        return ("committed",) + r[1:]

    def release(self, r):
        s = self._slot(r, "committed")
        if s["pub_session"] or s["pub_active"] or self.roots[r[1]] is not None:
            fail("InvalidTransition")
        self.used = self.used - s["claim"]
        self.slots[r[1]] = None
        self.counters["releases"] += 1

    def _gens(self, n):
        g = self.next_lease_generation
        self.next_lease_generation += n
        return g

    # -- trees -------------------------------------------------------------------
    def _tree_token(self, slot):
        root = self.roots[slot]
        s = self.slots[slot]
        return Tree(slot=slot, receipt_gen=s["gen"], tree_key=root["tree_key"],
                    identity_generation=root["ident"], generation=root["gen"],
                    structural_revision=root["rev"], current=copy.copy(root["current"]),
                    ceiling=root["ceiling"], active_nodes=root["active"],
                    state=self._state(slot))

    def _state(self, slot):
        # everything the tree token must pin: pending decision and every node
        root = self.roots[slot]
        nodes = tuple((i, n["gen"], n["state"], n["pending"], n["subtree"].t())
                      for i, n in enumerate(self.nodes)
                      if n is not None and n["slot"] == slot and n["ident"] == root["ident"])
        return (root["pending"], root["pending_gen"], root["pending_count"],
                root["pending_claim"].t(), root["pending_scope"], nodes)

    def _tree(self, t):
        s = self.slots[t.slot] if t.slot < len(self.slots) else None
        if s is None or s["gen"] != t.receipt_gen:
            fail("StaleReservation")
        if s["state"] != "committed":
            fail("InvalidTransition")
        root = self.roots[t.slot]
        if root is None or t.key() != self._tree_token(t.slot).key():
            fail("StaleReservation")
        return root

    def _node(self, t, n):
        self._tree(t)
        if n.slot != t.slot or n.tree_identity_generation != t.identity_generation or \
                n.node_index >= len(self.nodes):
            fail("StaleReservation")
        slot = self.nodes[n.node_index]
        if slot is None or self._node_token(t.slot, n.node_index).key() != n.key():
            fail("StaleReservation")
        return slot

    def _node_token(self, slot, i):
        n = self.nodes[i]
        return Node(slot=slot, tree_identity_generation=n["ident"], node_index=i,
                    generation=n["gen"], parent_index=n["parent"], parent_generation=n["parent_gen"],
                    node_key=n["key"], tenant_key=n["tenant"], binding_key=n["binding"],
                    kind=n["kind"], claim=n["claim"])

    def open_tree(self, r, tree_key, authority_key, **ceiling):
        c = Claim(**ceiling)
        if tree_key == 0 or authority_key == 0 or c.zero():
            fail("InvalidClaim")
        s = self._slot(r, None)
        if s["state"] != "committed" or self.roots[r[1]] is not None or s["pub_epoch"] or \
                s["pub_session"] or s["pub_active"]:
            fail("InvalidTransition")
        g = self._gens(2)
        self.roots[r[1]] = dict(tree_key=tree_key, auth=authority_key, ident=g, gen=g + 1, rev=1,
                                ceiling=c, current=Claim(), active=0, pending="none",
                                pending_gen=0, pending_completion=0, pending_free_permit=0,
                                pending_free_completion=0, pending_scope=NO_NODE,
                                pending_count=0, pending_claim=Claim())
        self.counters["lease_tree_opens"] += 1
        return self._tree_token(r[1])

    def open_scope(self, tree, scope_key, tenant_key, **ceiling):
        c = Claim(**ceiling)
        if scope_key == 0 or tenant_key == 0 or c.zero():
            fail("InvalidClaim")
        root = self._tree(tree)
        s = self.slots[tree.slot]
        if root["pending"] != "none" or s["pub_active"] or s["pub_epoch"] or s["pub_session"] or \
                not c.within(root["ceiling"]):
            fail("InvalidTransition")
        free = None
        for i, n in enumerate(self.nodes):
            if n is not None and n["slot"] == tree.slot and n["ident"] == root["ident"] and \
                    n["kind"] == 0 and n["key"] == scope_key:
                fail("InvalidTransition")
            if n is None and free is None:
                free = i
        if free is None:
            self.counters["rejected_lease_nodes"] += 1
            fail("LeaseNodesExhausted")
        g = self._gens(2)
        self.nodes[free] = dict(slot=tree.slot, ident=root["ident"], gen=g, parent=NO_NODE,
                                parent_gen=root["ident"], key=scope_key, tenant=tenant_key,
                                binding=0, kind=0, state="live", ceiling=c, claim=Claim(),
                                subtree=Claim(), pending=0)
        root["active"] += 1
        root["gen"] = g + 1
        root["rev"] += 1
        self.counters["lease_scope_opens"] += 1
        tree.assign(self._tree_token(tree.slot))
        return self._node_token(tree.slot, free)

    def close_tree(self, tree):
        root = self._tree(tree)
        s = self.slots[tree.slot]
        if root["pending"] != "none" or not root["current"].zero() or s["pub_active"] or \
                s["pub_session"]:
            fail("InvalidTransition")
        mine = [i for i, n in enumerate(self.nodes)
                if n is not None and n["slot"] == tree.slot and n["ident"] == root["ident"]]
        for i in mine:
            n = self.nodes[i]
            if n["kind"] != 0 or not n["claim"].zero() or not n["subtree"].zero():
                fail("InvalidTransition")
        if len(mine) != root["active"]:
            fail("InvalidTransition")
        for i in mine:
            self.nodes[i] = None
        self.roots[tree.slot] = None
        self.counters["lease_tree_closes"] += 1

    # -- publication -----------------------------------------------------------------
    def bind_session(self, tree, request_epoch, session_id):
        if request_epoch == 0 or session_id == 0:
            fail("InvalidConfiguration")
        root = self._tree(tree)
        if root["pending"] != "none":
            fail("InvalidTransition")
        s = self.slots[tree.slot]
        if s["pub_session"] or s["pub_epoch"]:
            fail("InvalidTransition")
        s.update(pub_epoch=request_epoch, pub_session=session_id, pub_next=0, pub_active=False)

    def close_session(self, r, request_epoch, session_id, expected_next):
        s = self._slot(r, None)
        root = self.roots[r[1]]
        if root is not None and (root["pending"] != "none" or not root["current"].zero()):
            fail("InvalidTransition")
        if s["state"] != "committed" or s["pub_epoch"] != request_epoch or \
                s["pub_session"] != session_id or s["pub_active"] or s["pub_next"] != expected_next:
            fail("InvalidTransition")
        s["pub_session"] = 0

    def publish(self, tree, request_epoch, session_id, sequence):
        """beginPublicationWithLeaseTree + commitPublicationAssumeValid."""
        root = self._tree(tree)
        s = self.slots[tree.slot]
        if root["pending"] != "none" or s["pub_epoch"] != request_epoch or \
                s["pub_session"] != session_id or s["pub_active"] or s["pub_next"] != sequence:
            fail("InvalidTransition")
        s["pub_gen"] += 1
        s["pub_next"] = sequence + 1

    def _session_ok(self, slot, request_epoch, session_id, sequence):
        s = self.slots[slot]
        return not s["pub_active"] and s["pub_epoch"] == request_epoch and \
            s["pub_session"] == session_id and s["pub_next"] == sequence

    # -- allocation leaves ---------------------------------------------------------------
    def reserve_allocations(self, tree, request_epoch, session_id, sequence, specs):
        """specs: [(scope Node, node_key, binding_key, Claim)] -> (batch, leaves)."""
        if request_epoch == 0 or session_id == 0 or not specs:
            fail("InvalidConfiguration")
        root = self._tree(tree)
        if root["pending"] != "none" or not self._session_ok(tree.slot, request_epoch, session_id,
                                                              sequence):
            fail("InvalidTransition")
        if sum(n is None for n in self.nodes) < len(specs):
            self.counters["rejected_lease_nodes"] += 1
            fail("LeaseNodesExhausted")
        agg = Claim()
        for k, (scope, node_key, binding_key, claim) in enumerate(specs):
            if node_key == 0 or binding_key == 0 or claim.zero():
                fail("InvalidClaim")
            sc = self._node(tree, scope)
            if sc["kind"] != 0 or sc["state"] != "live":
                fail("InvalidTransition")
            agg = agg + claim
            for n in self.nodes:
                if n is None or n["slot"] != tree.slot or n["ident"] != root["ident"] or n["kind"] != 1:
                    continue
                if (n["parent"] == scope.node_index and n["key"] == node_key) or \
                        n["binding"] == binding_key:
                    fail("InvalidTransition")
            for prior in specs[:k]:
                if (prior[0].node_index == scope.node_index and prior[1] == node_key) or \
                        prior[2] == binding_key:
                    fail("InvalidTransition")
            addition = Claim()
            for cand in specs:
                if cand[0].node_index == scope.node_index:
                    addition = addition + cand[3]
            if not (sc["subtree"] + addition).within(sc["ceiling"]):
                fail("InvalidClaim")
        nxt_tree = root["current"] + agg
        if not nxt_tree.within(root["ceiling"]):
            fail("InvalidClaim")
        nxt_used = self.used + agg
        if not self._fits(nxt_used):
            self.counters["rejected_lease_capacity"] += 1
            fail("CapacityExceeded")
        start = self._gens(len(specs) + 3)
        batch_gen, reserve_gen = start, start + 1 + len(specs)
        leaves = []
        for k, (scope, node_key, binding_key, claim) in enumerate(specs):
            i = next(j for j, n in enumerate(self.nodes) if n is None)
            self.nodes[i] = dict(slot=tree.slot, ident=root["ident"], gen=start + 1 + k,
                                 parent=scope.node_index, parent_gen=scope.generation,
                                 key=node_key, tenant=scope.tenant_key, binding=binding_key,
                                 kind=1, state="reserved", ceiling=claim, claim=claim,
                                 subtree=claim, pending=batch_gen)
            sc = self.nodes[scope.node_index]
            sc["subtree"] = sc["subtree"] + claim
            leaves.append(self._node_token(tree.slot, i))
        root.update(current=nxt_tree, active=root["active"] + len(specs), pending="allocation",
                    pending_gen=batch_gen, pending_completion=reserve_gen + 1,
                    pending_count=len(specs), pending_claim=agg, gen=reserve_gen,
                    rev=root["rev"] + 1)
        self.used = nxt_used
        self.counters["lease_allocation_reserves"] += 1
        batch = dict(slot=tree.slot, gen=batch_gen, tree_gen=reserve_gen, completion=reserve_gen + 1,
                     claim=agg, count=len(specs), epoch=request_epoch, session=session_id,
                     sequence=sequence)
        tree.assign(self._tree_token(tree.slot))
        return batch, leaves

    def _pending(self, batch, kind):
        # a decision token is the exact pending decision it names: a token
        # whose fields were altered is a forgery (the reference's integrity
        # word, validateLeaseAllocationBatchLocked :3816-3857), a consumed
        # one no longer matches the tree's state
        root = self.roots[batch["slot"]]
        if root is not None and root["pending"] == kind and root["pending_gen"] == batch["gen"] and \
                (root["pending_claim"] != batch["claim"] or root["pending_count"] != batch["count"]):
            fail("StaleReservation")
        if root is None or root["pending"] != kind or root["pending_gen"] != batch["gen"] or \
                root["gen"] != batch["tree_gen"] or \
                not self._session_ok(batch["slot"], batch["epoch"], batch["session"],
                                     batch["sequence"]):
            fail("InvalidTransition")
        return root

    def commit_allocations(self, batch, tree):
        root = self._pending(batch, "allocation")
        for n in self.nodes:
            if n is not None and n["slot"] == batch["slot"] and n["pending"] == batch["gen"]:
                n.update(state="live", pending=0)
        root.update(pending="none", pending_gen=0, pending_count=0, pending_claim=Claim(),
                    gen=batch["completion"], rev=root["rev"] + 1)
        self.counters["lease_allocation_materializations"] += 1
        tree.assign(self._tree_token(batch["slot"]))

    def abort_allocations(self, batch, tree):
        root = self._pending(batch, "allocation")
        for i, n in enumerate(self.nodes):
            if n is not None and n["slot"] == batch["slot"] and n["pending"] == batch["gen"]:
                sc = self.nodes[n["parent"]]
                sc["subtree"] = sc["subtree"] - n["claim"]
                self.nodes[i] = None
        root.update(current=root["current"] - batch["claim"], active=root["active"] - batch["count"],
                    pending="none", pending_gen=0, pending_count=0, pending_claim=Claim(),
                    gen=batch["completion"], rev=root["rev"] + 1)
        self.used = self.used - batch["claim"]
        self.counters["lease_allocation_aborts"] += 1
        tree.assign(self._tree_token(batch["slot"]))

    # -- retirement --------------------------------------------------------------------------
    def begin_retire(self, tree, scope, request_epoch, session_id, sequence):
        if request_epoch == 0 or session_id == 0:
            fail("InvalidConfiguration")
        root = self._tree(tree)
        sc = self._node(tree, scope)
        if sc["kind"] != 0 or sc["state"] != "live" or root["pending"] != "none" or \
                not self._session_ok(tree.slot, request_epoch, session_id, sequence):
            fail("InvalidTransition")
        mine = [n for n in self.nodes if n is not None and n["slot"] == tree.slot and
                n["ident"] == root["ident"] and n["kind"] == 1 and n["parent"] == scope.node_index]
        claim = Claim()
        for n in mine:
            if n["state"] != "live":
                fail("InvalidTransition")
            claim = claim + n["claim"]
        if not mine or claim.zero() or claim != sc["subtree"]:
            fail("InvalidTransition")
        g = self._gens(5)
        for n in mine:
            n.update(state="quiescing", pending=g)
        root.update(pending="retire", pending_gen=g, pending_completion=g + 2,
                    pending_free_permit=g + 3, pending_free_completion=g + 4,
                    pending_scope=scope.node_index, pending_count=len(mine), pending_claim=claim,
                    gen=g + 1, rev=root["rev"] + 1)
        self.counters["lease_reclaim_prepares"] += 1
        tree.assign(self._tree_token(tree.slot))
        return dict(slot=tree.slot, gen=g, tree_gen=g + 1, decision=g + 2, permit=g + 3,
                    completion=g + 4, scope=scope.node_index, count=len(mine), claim=claim,
                    epoch=request_epoch, session=session_id, sequence=sequence)

    def cancel_retire(self, ticket, tree):
        root = self._pending(ticket, "retire")
        for n in self.nodes:
            if n is not None and n["slot"] == ticket["slot"] and n["pending"] == ticket["gen"]:
                n.update(state="live", pending=0)
        root.update(pending="none", pending_gen=0, pending_count=0, pending_claim=Claim(),
                    pending_scope=NO_NODE, gen=ticket["decision"], rev=root["rev"] + 1)
        self.counters["lease_reclaim_cancels"] += 1
        tree.assign(self._tree_token(ticket["slot"]))

    def authorize_free(self, ticket, tree):
        root = self._pending(ticket, "retire")
        for n in self.nodes:
            if n is not None and n["slot"] == ticket["slot"] and n["pending"] == ticket["gen"]:
                n.update(state="free_authorized", pending=ticket["permit"])
        root.update(pending="free", pending_gen=ticket["permit"],
                    pending_completion=ticket["completion"], gen=ticket["decision"],
                    rev=root["rev"] + 1)
        self.counters["lease_reclaim_authorizations"] += 1
        tree.assign(self._tree_token(ticket["slot"]))
        return dict(ticket, gen=ticket["permit"], tree_gen=ticket["decision"])

    def commit_free(self, permit, tree):
        root = self._pending(permit, "free")
        for i, n in enumerate(self.nodes):
            if n is not None and n["slot"] == permit["slot"] and n["pending"] == permit["gen"]:
                self.nodes[i] = None
        sc = self.nodes[permit["scope"]]
        sc["subtree"] = sc["subtree"] - permit["claim"]
        root.update(current=root["current"] - permit["claim"],
                    active=root["active"] - permit["count"], pending="none", pending_gen=0,
                    pending_count=0, pending_claim=Claim(), pending_scope=NO_NODE,
                    gen=permit["completion"], rev=root["rev"] + 1)
        self.used = self.used - permit["claim"]
        self.counters["lease_reclaim_commits"] += 1
        tree.assign(self._tree_token(permit["slot"]))

    def snapshot(self):
        out = dict(self.counters)
        out["used"] = {c: getattr(self.used, c) for c in CLASSES}
        out["active_reservations"] = sum(s is not None and s["state"] == "reserved"
                                         for s in self.slots)
        out["committed_receipts"] = sum(s is not None and s["state"] == "committed"
                                        for s in self.slots)
        out["active_lease_trees"] = sum(r is not None for r in self.roots)
        live = [n for n in self.nodes if n is not None]
        out["active_lease_nodes"] = len(live)
        out["active_lease_scopes"] = sum(n["kind"] == 0 for n in live)
        for st, name in (("reserved", "reserved_unmaterialized_allocations"),
                         ("live", "live_allocations"), ("quiescing", "quiescing_allocations"),
                         ("free_authorized", "free_authorized_allocations")):
            out[name] = sum(n["kind"] == 1 and n["state"] == st for n in live)
        return out


# -- the page map with a pool, rows and retirement ----------------------------------------
class Pages:
    """oracle.paged_kv.PagedKVCache plus a payload pool of `pool_pages`
    (an allocator with a limit), f32 rows, logicalKvSha256 (hashLogicalPrefix,
    paged_kv_cache.zig:1532-1555) and retirement (:1187-1250)."""

    def __init__(self, layers, dim, max_seq, pool_pages):
        self.cache = pk.PagedKVCache(layers, dim, max_seq)
        self.capacity = pool_pages
        self.rows = {}            # (logical page, layer, kv, row) -> list of floats
        self.retired = False
        self.leased = None

    def page_count(self):
        return len(self.cache.payload)

    def page_bytes(self):
        return self.cache.page_payload_bytes()

    def set_pool_capacity(self, pages):
        self.capacity = pages

    def plan_next_row(self):
        if self.retired:
            fail("CacheRetired")
        c = self.cache
        try:
            page, row, installs = c._validate_next_row()
        except pk.PagedError as e:
            fail(str(e))
        present = c.payload[page] is not None
        return dict(cache_instance=c.instance_id, base_len=c.len, logical_page=page, row_in_page=row,
                    root_generation=c.committed_root.generation,
                    row_txn_generation=c.next_row_txn_generation,
                    root_after_generation=c.next_root_generation,
                    page_ownership_generation=c.ownership[page],
                    next_page_ownership_generation=c.next_page_generation,
                    allocated_pages=c.allocated_pages, page_payload_present=present,
                    allocation_bytes=self.page_bytes() if installs and not present else 0)

    def begin_row(self):
        c = self.cache
        page, row, installs = c._validate_next_row()
        if installs and c.payload[page] is None and c.allocated_pages >= self.capacity:
            fail("OutOfMemory")
        return c.begin_row()

    def append_row(self, mark, layer, k, v):
        self.rows[(mark.logical_page, layer, 0, mark.base_len % pk.PAGE)] = list(k)
        self.rows[(mark.logical_page, layer, 1, mark.base_len % pk.PAGE)] = list(v)

    def kv_sha256(self):
        if self.retired:
            fail("CacheRetired")
        c = self.cache
        h = hashlib.sha256(b"glacier-logical-kv-state-v1\x00" +
                           struct.pack("<3Q", c.num_layers, c.dim, c.len))
        for layer in range(c.num_layers):
            for kv in (0, 1):
                for pos in range(c.len):
                    vals = self.rows.get((pos // pk.PAGE, layer, kv, pos % pk.PAGE), [0.0] * c.dim)
                    h.update(struct.pack(f"<{c.dim}f", *vals))
        return h.digest()

    def plan_retirement(self):
        if self.retired:
            fail("CacheRetired")
        c = self.cache
        if c.active is not None:
            fail("TransactionActive")
        return (c.committed_root, c.len, c.allocated_pages, c.allocated_pages * self.page_bytes(),
                c.next_root_generation)

    def reclaim_retired(self, plan):
        if plan != self.plan_retirement():
            fail("InvalidTransaction")
        c = self.cache
        c.payload = [None] * len(c.payload)
        c.ownership = [0] * len(c.ownership)
        c.allocated_pages = 0
        c.committed_root = pk.Root(c.instance_id, c.next_root_generation, 0, 0,
                                   pk.empty_ownership_digest(c.instance_id, c.num_layers, c.dim,
                                                             c.max_seq))
        c.next_root_generation += 1
        c.len = 0
        self.retired = True
        return plan[3]


def page_binding_key(cache_instance, logical_page):
    # pageBindingKey (leased_paged_kv_cache.zig:1353-1357) over SplitMix64's finaliser
    def mix(v):
        v &= U64
        v ^= v >> 30
        v = (v * 0xBF58476D1CE4E5B9) & U64
        v ^= v >> 27
        v = (v * 0x94D049BB133111EB) & U64
        return v ^ (v >> 31)
    v = mix(0x706167656C656166 ^ cache_instance ^ mix(logical_page + 1))
    return v or 1


class Leased:
    """LeasedPagedKVCache over a Pages map. Bindings are (state, leaf) per page."""

    _next_instance = [1]

    def __init__(self, bank, tree, scope, pages, request_epoch, session_id, sequence):
        if request_epoch == 0 or session_id == 0 or scope.kind != 0 or scope.binding_key != 0:
            fail("InvalidCoordinator")
        c = pages.cache
        if pages.retired or c.allocated_pages or c.committed_root.committed_len or \
                c.committed_root.committed_pages or pages.leased is not None:
            fail("InvalidCoordinator")
        bank._node(tree, scope)
        self.bank, self.tree, self.scope, self.pages = bank, tree, scope, pages
        self.epoch, self.session, self.sequence = request_epoch, session_id, sequence
        self.instance = Leased._next_instance[0]
        Leased._next_instance[0] += 1
        pages.leased = self
        self.bindings = [None] * pages.page_count()   # None or [state, leaf, bytes]
        self.row = None
        self.seal = None
        self.pending = None
        self.reclaimed = False

    def _mutable(self):
        if self.reclaimed:
            fail("ReclaimComplete")
        if self.pending is not None:
            fail("ReclaimPending")
        if self.seal is not None:
            fail("AlreadyTerminal")
        self.bank._node(self.tree, self.scope)

    def binding_summary(self, state="live"):
        self.bank._node(self.tree, self.scope)
        count = nbytes = 0
        for i, b in enumerate(self.bindings):
            if b is None:
                continue
            if b[0] != state:
                fail("InvalidBinding")
            leaf = b[1]
            if leaf.kind != 1 or leaf.parent_index != self.scope.node_index or \
                    leaf.node_key != i + 1 or \
                    leaf.binding_key != page_binding_key(self.pages.cache.instance_id, i) or \
                    leaf.claim != Claim(kv_bytes=b[2]):
                fail("InvalidBinding")
            self.bank._node(self.tree, leaf)
            count += 1
            nbytes += b[2]
        c = self.pages.cache
        if state == "live" and (c.allocated_pages != count or
                                c.allocated_pages * self.pages.page_bytes() != nbytes):
            fail("InvalidBinding")
        return count, nbytes

    def kv_sha256(self):
        return self.pages.kv_sha256()

    def lifecycle(self):
        return ("reclaimed" if self.reclaimed else "freed_pending_uncharge" if self.pending
                else "terminal_retained" if self.seal else "live")

    def plan_next_row(self):
        self._mutable()
        if self.row is not None:
            fail("InvalidLeasedTransaction")
        summary = self.binding_summary()
        plan = self.pages.plan_next_row()
        b = self.bindings[plan["logical_page"]]
        if (plan["allocation_bytes"] == 0 and plan["page_payload_present"] and b is None) or \
                (plan["allocation_bytes"] and (plan["page_payload_present"] or b is not None)):
            fail("InvalidBinding")
        return dict(plan, tree=self.tree.key(), sequence=self.sequence.value, bindings=summary)

    def begin_row(self, plan):
        expected = self.plan_next_row()
        if plan != expected:
            fail("InvalidLeasedPlan")
        page = plan["logical_page"]
        if plan["allocation_bytes"]:
            spec = (self.scope, page + 1, page_binding_key(plan["cache_instance"], page),
                    Claim(kv_bytes=plan["allocation_bytes"]))
            batch, leaves = self.bank.reserve_allocations(self.tree, self.epoch, self.session,
                                                          plan["sequence"], [spec])
            try:
                mark = self.pages.begin_row()
            except LeaseFailure:
                self.bank.abort_allocations(batch, self.tree)
                raise
            self.bank.commit_allocations(batch, self.tree)
            self.bindings[page] = ["live", leaves[0], plan["allocation_bytes"]]
        else:
            mark = self.pages.begin_row()
        self.row = mark
        return mark

    def append_row(self, mark, layer, k, v):
        self.pages.append_row(mark, layer, k, v)

    def commit_row(self, mark):
        if self.row is None or self.row != mark:
            fail("InvalidLeasedTransaction")
        self.pages.cache.commit_row(mark)
        self.row = None
        return self.pages.cache.root()

    def abort_row(self, mark):
        if self.row is None or self.row != mark:
            fail("InvalidLeasedTransaction")
        self.pages.cache.abort_row(mark)
        self.row = None

    def seal_terminal(self, root, kv_sha256, sequence, reason, token):
        self._mutable()
        if self.row is not None:
            fail("InvalidLeasedTransaction")
        if sequence == U64 or sequence != self.sequence.value:
            fail("InvalidTerminalSeal")
        if self.pages.retired:
            fail("CacheRetired")
        if root != self.pages.cache.committed_root:
            fail("InvalidRoot")
        if self.pages.kv_sha256() != bytes(kv_sha256):
            fail("InvalidTerminalSeal")
        summary = self.binding_summary()
        self.bank.publish(self.tree, self.epoch, self.session, sequence)
        self.sequence.value = sequence + 1
        self.seal = dict(root=root, kv=bytes(kv_sha256), bindings=summary, sequence=sequence,
                         reason=reason, token=token, scope=self.scope.node_index)
        return self.seal

    def begin_reclaim(self, seal, expected_sequence):
        if self.seal is None:
            fail("TerminalRequired")
        if seal != self.seal:
            fail("InvalidTerminalSeal")
        return self._reclaim_exact(seal["root"], seal["kv"], seal["bindings"], seal["sequence"],
                                   expected_sequence)

    def _reclaim_exact(self, root, kv, bindings, terminal_sequence, expected_sequence):
        if self.pending is not None:
            fail("ReclaimPending")
        if self.reclaimed:
            fail("ReclaimComplete")
        if expected_sequence != self.sequence.value or \
                (terminal_sequence is not None and expected_sequence <= terminal_sequence):
            fail("InvalidTerminalSeal")
        if self.pages.retired:
            fail("CacheRetired")
        if root != self.pages.cache.committed_root:
            fail("InvalidRoot")
        if self.pages.kv_sha256() != kv:
            fail("InvalidTerminalSeal")
        summary = self.binding_summary()
        if summary != bindings:
            fail("InvalidBinding")
        plan = self.pages.plan_retirement()
        if plan[0] != root or plan[2] != summary[0] or plan[3] != summary[1]:
            fail("InvalidBinding")
        ticket = self.bank.begin_retire(self.tree, self.scope, self.epoch, self.session,
                                        expected_sequence)
        permit = self.bank.authorize_free(ticket, self.tree)
        freed_bytes = self.pages.reclaim_retired(plan)
        for b in self.bindings:
            if b is not None:
                b[0] = "freed_pending_uncharge"
        self.pending = dict(permit=permit, count=summary[0], bytes=freed_bytes,
                            root_before=root, root_after=self.pages.cache.committed_root)
        return self.pending

    def commit_reclaim(self, freed):
        if self.pending is None:
            fail("ReclaimComplete" if self.reclaimed else "InvalidFreedPayload")
        if freed != self.pending:
            fail("InvalidFreedPayload")
        if self.binding_summary("freed_pending_uncharge") != (freed["count"], freed["bytes"]):
            fail("InvalidBinding")
        self.bank.commit_free(freed["permit"], self.tree)
        self.bindings = [None] * len(self.bindings)
        self.pending = None
        self.reclaimed = True

    def reclaim_for_teardown(self, expected_sequence):
        if self.reclaimed:
            return
        if self.pending is not None:
            return self.commit_reclaim(self.pending)
        if self.row is not None:
            self.abort_row(self.row)
        if expected_sequence != self.sequence.value:
            fail("InvalidTerminalSeal")
        root = self.pages.cache.committed_root
        kv = self.pages.kv_sha256()
        summary = self.binding_summary()
        if summary[0] == 0:
            plan = self.pages.plan_retirement()
            if plan[2] != 0:
                fail("InvalidBinding")
            self.pages.reclaim_retired(plan)
            self.reclaimed = True
            return
        freed = self._reclaim_exact(root, kv, summary, None, expected_sequence)
        self.commit_reclaim(freed)
