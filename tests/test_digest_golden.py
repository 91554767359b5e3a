"""Digests pinned by vectors the reference's own Python restatements wrote
(tests/golden/make_digest_golden.py imports bench/lane4_event_evidence.py,
bench/prepared_text_checkpoint.py and bench/device_capability_contract.py in
the build container; tests/golden/digests.json holds inputs and digests):

* tokenSequenceSha256 (generate.zig:3193-3203): the C oracle and the
  product's host function (the digest a lane's state reports);
* logicalKvPrefixSha256 (generate.zig:3150-3172): the C oracle over
  [L][max_seq][kv_dim] K/V arrays, and the product's host page map
  (glacier_hip_kv_pages_*) filled row by row through its row transactions,
  including -0.0, NaN and infinity bit patterns;
* capabilityRootV1: the oracle's capability_root_v1, which the GPU boundary
  test compares with the product's record digest.
"""
import ctypes as C
import json
import os
import types

import numpy as np
import pytest

from oracle import device_contract as dc

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "digests.json")))


def _kv_arrays(case):
    L, d, p = case["num_layers"], case["kv_dim"], case["positions"]
    words = np.frombuffer(bytes.fromhex(case["payload_hex"]), dtype="<u4").reshape(L, 2, p, d)
    return words[:, 0].view(np.float32), words[:, 1].view(np.float32)


@pytest.mark.parametrize("i", range(len(GOLDEN["token_sequence"])))
def test_token_sequence_digest(ora, gh, i):
    case = GOLDEN["token_sequence"][i]
    want = bytes.fromhex(case["sha256"])
    assert ora.token_sequence_sha256(case["tokens"]) == want
    toks = np.asarray(case["tokens"], dtype=np.uint32)
    out = (C.c_uint8 * 32)()
    assert gh.lib().glacier_hip_token_sequence_sha256(toks.ctypes.data if toks.size else None,
                                                      toks.size, out) == gh.OK
    assert bytes(out) == want


@pytest.mark.parametrize("i", range(len(GOLDEN["logical_kv"])))
def test_logical_kv_digest(ora, gh, i):
    case = GOLDEN["logical_kv"][i]
    want = bytes.fromhex(case["sha256"])
    k, v = _kv_arrays(case)
    L, d, p = case["num_layers"], case["kv_dim"], case["positions"]
    # the oracle over a cache longer than the prefix (only [0, p) is hashed)
    kc = np.full((L, p + 5, d), 7.0, np.float32)
    vc = np.full((L, p + 5, d), -7.0, np.float32)
    kc[:, :p], vc[:, :p] = k, v
    assert ora.logical_kv_sha256(kc, vc, p) == want
    # the product's host page map, row transactions in position order
    pages = gh.KvPages(L, d, 64, 8)
    try:
        for pos in range(p):
            rc, mark = pages.begin_row()
            assert rc == gh.OK
            for layer in range(L):
                kk = np.ascontiguousarray(k[layer, pos])
                vv = np.ascontiguousarray(v[layer, pos])
                fp = C.POINTER(C.c_float)
                assert gh.lib().glacier_hip_kv_pages_append_row(
                    pages.h, C.byref(mark), layer, kk.ctypes.data_as(fp),
                    vv.ctypes.data_as(fp)) == gh.OK
            assert pages.commit_row(mark) == gh.OK
        assert pages.kv_sha256() == want
    finally:
        pages.close()


def test_logical_kv_digest_sees_every_bit(ora):
    # a one-bit change anywhere in the payload, or a different shape split of
    # the same bytes, changes the digest
    case = GOLDEN["logical_kv"][1]
    k, v = _kv_arrays(case)
    base = ora.logical_kv_sha256(k, v, case["positions"])
    for arr in (k, v):
        flipped = arr.view(np.uint32).copy()
        flipped.reshape(-1)[-1] ^= 1
        f = flipped.view(np.float32)
        got = ora.logical_kv_sha256(f, v, case["positions"]) if arr is k else \
            ora.logical_kv_sha256(k, f, case["positions"])
        assert got != base
    assert ora.logical_kv_sha256(k[:, :-1], v[:, :-1], case["positions"] - 1) != base


@pytest.mark.parametrize("i", range(len(GOLDEN["capability"])))
def test_capability_root(i):
    case = GOLDEN["capability"][i]
    rec = dict(case["record"])
    for f in ("backend_sha256", "device_sha256", "driver_sha256", "placement_sha256"):
        rec[f] = bytes.fromhex(rec[f])
    assert dc.capability_root_v1(types.SimpleNamespace(**rec)) == bytes.fromhex(case["sha256"])
