"""Restatement of the reference's PagedKVCache page map and row transaction.

TEST INFRASTRUCTURE ONLY: the checker for the product's page maps
(glacier-engine_amd/csrc/paged_kv.cpp and the session lanes built on it).
Only tests/, __graft_entry__.smoke() and bench.py's CPU leg use it.

Follows /root/reference/src/paged_kv_cache.zig:
  PagedKVCache.init            :530-568  (next_root_generation 2, next_page_generation 1,
                                          committed root generation 1, empty ownership digest)
  validateNextRowState         :1386-1419
  beginRowInternal             :1011-1072 (page and root generations are consumed at begin)
  prepareCommit / commit       :1105-1135
  abortRow                     :1146-1158 (clears the page's ownership generation only;
                                          the payload stays with the logical page)
  reset                        :1162-1182
  validateCommittedPageRef     :944-957
  validateCurrentRoot          :934-942
  allocationCommitmentLedger   :840-892
  emptyOwnershipDigest / appendOwnershipDigest :323-353
Payloads are modelled as opaque ids (the allocator address in the reference);
K/V contents are not part of the page map. Payload bytes are f32, as the
reference stores them.
"""
import hashlib
import struct

PAGE = 16
PAGE_REF_ABI = 0x4750524600000001
PAGE_MAP_ROOT_ABI = 0x47504D5200000001
ROW_TXN_ABI = 0x4750525400000001


class PagedError(Exception):
    """The reference's PagedKVCache.Error, by name (e.g. 'InvalidRoot')."""


def empty_ownership_digest(inst, layers, dim, max_seq):
    # paged_kv_cache.zig:323-338
    return hashlib.sha256(b"glacier-paged-kv-ownership-v1\x00" +
                          struct.pack("<5Q", inst, layers, dim, max_seq, PAGE)).digest()


def append_ownership_digest(before, inst, logical_page, generation):
    # paged_kv_cache.zig:341-353
    return hashlib.sha256(b"glacier-paged-kv-root-append-v1\x00" + bytes(before) +
                          struct.pack("<4Q", PAGE_REF_ABI, inst, logical_page, generation)).digest()


class Root:
    __slots__ = ("cache_instance", "generation", "committed_len", "committed_pages",
                 "ownership_sha256")

    def __init__(self, cache_instance, generation, committed_len, committed_pages, ownership):
        self.cache_instance = cache_instance
        self.generation = generation
        self.committed_len = committed_len
        self.committed_pages = committed_pages
        self.ownership_sha256 = bytes(ownership)

    def key(self):
        return (PAGE_MAP_ROOT_ABI, self.cache_instance, self.generation, self.committed_len,
                self.committed_pages, self.ownership_sha256)

    def __eq__(self, other):
        return self.key() == other.key()

    def __repr__(self):
        return (f"Root(inst={self.cache_instance}, gen={self.generation}, "
                f"len={self.committed_len}, pages={self.committed_pages}, "
                f"own={self.ownership_sha256.hex()[:16]})")


class Mark:
    """RowTxnMark (:255-265) with its PageRefV1 (:55-60)."""
    __slots__ = ("cache_instance", "generation", "base_len", "root_before_generation",
                 "root_after_generation", "logical_page", "ownership_generation")

    def __init__(self, **kw):
        for k, v in kw.items():
            setattr(self, k, v)

    def key(self):
        return tuple(getattr(self, k) for k in self.__slots__)

    def __eq__(self, other):
        return self.key() == other.key()


class PagedKVCache:
    _next_instance = [1]
    _next_payload = [1]

    def __init__(self, num_layers, dim, max_seq, instance=None):
        if num_layers == 0 or dim == 0 or max_seq == 0:
            raise PagedError("ShapeMismatch")
        self.num_layers, self.dim, self.max_seq = num_layers, dim, max_seq
        if instance is None:
            instance = PagedKVCache._next_instance[0]
            PagedKVCache._next_instance[0] += 1
        self.instance_id = instance
        pages = -(-max_seq // PAGE)
        self.payload = [None] * pages          # opaque payload id per logical page
        self.ownership = [0] * pages           # ownership generation per logical page
        self.allocated_pages = 0
        self.len = 0
        self.next_root_generation = 2
        self.next_page_generation = 1
        self.next_row_txn_generation = 1
        self.committed_root = Root(instance, 1, 0, 0,
                                   empty_ownership_digest(instance, num_layers, dim, max_seq))
        self.active = None

    # -- queries ---------------------------------------------------------------
    def root(self):
        return self.committed_root

    def page_payload_bytes(self):
        return self.num_layers * 2 * PAGE * self.dim * 4

    def validate_current_root(self, root):
        if root != self.committed_root:
            raise PagedError("InvalidRoot")

    def validate_committed_page_ref(self, instance, logical_page, generation):
        if (instance != self.instance_id or logical_page >= self.committed_root.committed_pages
                or logical_page >= len(self.payload)):
            raise PagedError("InvalidPageRef")
        if (self.payload[logical_page] is None or self.ownership[logical_page] == 0
                or self.ownership[logical_page] != generation):
            raise PagedError("InvalidPageRef")

    def resident_ledger(self):
        provisional = 1 if (self.active is not None and self.active["installs"]) else 0
        committed = self.committed_root.committed_pages
        if committed + provisional > self.allocated_pages:
            raise PagedError("InvalidRoot")
        map_bytes = len(self.payload) * 16
        resident = self.allocated_pages * self.page_payload_bytes()
        return dict(page_count_capacity=len(self.payload), allocated_pages=self.allocated_pages,
                    committed_pages=committed, provisional_pages=provisional,
                    reusable_pages=self.allocated_pages - committed - provisional,
                    page_map_bytes=map_bytes, resident_tensor_payload_bytes=resident,
                    resident_allocation_bytes=map_bytes + resident,
                    committed_tensor_payload_bytes=self.num_layers * 2 * self.len * self.dim * 4)

    # -- row transaction -----------------------------------------------------------
    def _validate_next_row(self):
        if self.active is not None:
            raise PagedError("TransactionActive")
        if self.len >= self.max_seq:
            raise PagedError("CacheFull")
        r = self.committed_root
        if r.committed_len != self.len or r.cache_instance != self.instance_id:
            raise PagedError("InvalidRoot")
        page, row = divmod(self.len, PAGE)
        installs = row == 0
        if page >= len(self.payload):
            raise PagedError("CacheFull")
        if r.committed_pages != page + (1 if row != 0 else 0):
            raise PagedError("InvalidRoot")
        if installs:
            if self.ownership[page] != 0:
                raise PagedError("InvalidRoot")
        elif self.payload[page] is None or self.ownership[page] == 0:
            raise PagedError("InvalidRoot")
        return page, row, installs

    def begin_row(self):
        page, row, installs = self._validate_next_row()
        if installs and self.payload[page] is None:
            self.payload[page] = PagedKVCache._next_payload[0]
            PagedKVCache._next_payload[0] += 1
            self.allocated_pages += 1
        if installs:
            self.ownership[page] = self.next_page_generation
            self.next_page_generation += 1
        before = self.committed_root
        own = (append_ownership_digest(before.ownership_sha256, self.instance_id, page,
                                       self.ownership[page])
               if installs else before.ownership_sha256)
        after = Root(self.instance_id, self.next_root_generation, self.len + 1,
                     before.committed_pages + (1 if installs else 0), own)
        self.next_root_generation += 1
        mark = Mark(cache_instance=self.instance_id, generation=self.next_row_txn_generation,
                    base_len=self.len, root_before_generation=before.generation,
                    root_after_generation=after.generation, logical_page=page,
                    ownership_generation=self.ownership[page])
        self.next_row_txn_generation += 1
        self.active = dict(mark=mark, before=before, after=after, page=page, installs=installs)
        return mark

    def _validate_txn(self, mark):
        if self.active is None or self.active["mark"] != mark:
            raise PagedError("InvalidTransaction")
        return self.active

    def prepare_commit(self, mark):
        a = self._validate_txn(mark)
        return a["before"], a["after"], a["installs"]

    def commit_row(self, mark):
        a = self._validate_txn(mark)
        if a["before"] != self.committed_root or a["after"].committed_len != self.len + 1:
            raise PagedError("InvalidTransaction")
        self.committed_root = a["after"]
        self.len += 1
        self.active = None

    def abort_row(self, mark):
        a = self._validate_txn(mark)
        if a["installs"]:
            if self.ownership[a["page"]] != mark.ownership_generation:
                raise PagedError("InvalidPageRef")
            self.ownership[a["page"]] = 0
        self.active = None

    def reset(self):
        if self.active is not None:
            raise PagedError("TransactionActive")
        self.ownership = [0] * len(self.ownership)
        self.committed_root = Root(self.instance_id, self.next_root_generation, 0, 0,
                                   empty_ownership_digest(self.instance_id, self.num_layers,
                                                          self.dim, self.max_seq))
        self.next_root_generation += 1
        self.len = 0
