"""Paged-KV checkpoint page images on the CPU: the oracle's restatement
(oracle/page_image.py) pinned by the reference's golden image root, and the
product's codec (glacier_hip_page_image_encode_canonical / _decode,
csrc/page_image.cpp) giving byte-identical images and the reference's
verdict on every corruption. Reference tests restated:
src/continuation_paged_kv_restore.zig:659-747 ("paged KV page image is
canonical and mutation complete")."""
import ctypes as C
import random
import struct

import pytest

from oracle import page_image as pi
from oracle.paged_kv import PAGE_MAP_ROOT_ABI, PAGE_REF_ABI, Root, append_ownership_digest, \
    empty_ownership_digest

GOLDEN = "e052306f36ef24b9b92f7f0ef505045ea25fddf7bdf8f4c9e81b96733437d1e4"
CHALLENGE = bytes([0x61]) * 32


def _reference_case():
    # continuation_paged_kv_restore.zig:659-700
    own = append_ownership_digest(empty_ownership_digest(501, 2, 2, 32), 501, 0, 9)
    root = Root(501, 8, 16, 1, own)
    payload = b"".join(struct.pack("<f", float(i)) for i in range(128))
    return root, payload


def _c_root(gh, r):
    c = gh.PageMapRoot()
    c.abi_version = PAGE_MAP_ROOT_ABI
    c.cache_instance, c.generation = r.cache_instance, r.generation
    c.committed_len, c.committed_pages = r.committed_len, r.committed_pages
    c.ownership_sha256[:] = list(r.ownership_sha256)
    return c


def _c_ref(gh, inst, lp, gen):
    c = gh.PageRef()
    c.abi_version, c.cache_instance, c.logical_page, c.ownership_generation = \
        PAGE_REF_ABI, inst, lp, gen
    return c


def test_oracle_reproduces_the_reference_golden_root():
    root, payload = _reference_case()
    img = pi.encode_canonical(root, 2, 2, 32, (501, 0, 9), 16, payload, CHALLENGE)
    assert len(img) == 752
    d = pi.decode(img, CHALLENGE)
    assert d["image_sha256"].hex() == GOLDEN
    assert d["payload"] == payload


def test_product_encodes_the_same_bytes_and_decodes_them(gh):
    root, payload = _reference_case()
    want = pi.encode_canonical(root, 2, 2, 32, (501, 0, 9), 16, payload, CHALLENGE)
    got = gh.page_image_encode_canonical(_c_root(gh, root), 2, 2, 32, _c_ref(gh, 501, 0, 9), 16,
                                         payload, CHALLENGE)
    assert got == want
    assert gh.lib().glacier_hip_page_image_bytes(2, 2, 16) == 752
    info = gh.page_image_decode(got, CHALLENGE)
    assert bytes(info.image_sha256).hex() == GOLDEN
    assert (info.num_layers, info.dim, info.max_seq, info.committed_rows,
            info.payload_element_count, info.payload_offset) == (2, 2, 32, 16, 128, 208)
    assert info.source_ref.ownership_generation == 9 and info.source_root.generation == 8


def _verdict_product(gh, data, challenge=CHALLENGE):
    try:
        gh.page_image_decode(data, challenge)
    except gh.PageImageError as e:
        return e.reason
    return "Ok"


def _verdict_oracle(data, challenge=CHALLENGE):
    try:
        pi.decode(data, challenge)
    except pi.ImageError as e:
        return str(e)
    return "Ok"


def test_every_single_byte_corruption_is_rejected_with_the_references_reason(gh):
    # mutation completeness (:722-734): flipping the low bit of any byte fails
    root, payload = _reference_case()
    img = pi.encode_canonical(root, 2, 2, 32, (501, 0, 9), 16, payload, CHALLENGE)
    for i in range(len(img)):
        bad = bytearray(img)
        bad[i] ^= 1
        want = _verdict_oracle(bytes(bad))
        assert want != "Ok"
        assert _verdict_product(gh, bytes(bad)) == want, i
    # random bits with the footer recomputed, so the field checks decide
    rng = random.Random(7)
    names = set()
    for _ in range(400):
        bad = bytearray(img)
        bad[rng.randrange(len(img) - 32)] ^= 1 << rng.randrange(8)
        bad[-32:] = pi.image_root(bytes(bad[:-32]))
        want = _verdict_oracle(bytes(bad))
        assert _verdict_product(gh, bytes(bad)) == want
        names.add(want)
    assert {"InvalidFlags", "InvalidMagic", "InvalidAbi", "InvalidLength",
            "InvalidPageImage"} <= names


def test_reserved_word_is_invalid_flags(gh):
    # :735-746
    root, payload = _reference_case()
    img = bytearray(pi.encode_canonical(root, 2, 2, 32, (501, 0, 9), 16, payload, CHALLENGE))
    struct.pack_into("<I", img, 28, 1)
    img[-32:] = pi.image_root(bytes(img[:-32]))
    assert _verdict_oracle(bytes(img)) == "InvalidFlags"
    assert _verdict_product(gh, bytes(img)) == "InvalidFlags"


def test_wrong_or_zero_challenge_rejected(gh):
    root, payload = _reference_case()
    img = pi.encode_canonical(root, 2, 2, 32, (501, 0, 9), 16, payload, CHALLENGE)
    for ch in (bytes([0x62]) * 32, bytes(32)):
        assert _verdict_oracle(img, ch) == "InvalidPageImage"
        assert _verdict_product(gh, img, ch) == "InvalidPageImage"


def test_encode_rejects_bad_inputs_like_the_reference(gh):
    root, payload = _reference_case()
    croot, cref = _c_root(gh, root), _c_ref(gh, 501, 0, 9)
    L = gh.lib()

    def enc(**kw):
        a = dict(root=croot, layers=2, dim=2, max_seq=32, ref=cref, rows=16, payload=payload,
                 challenge=CHALLENGE, cap=752)
        a.update(kw)
        out = C.create_string_buffer(max(a["cap"], 1))
        n = C.c_uint64()
        info = gh.PageImageInfo()
        buf = C.create_string_buffer(a["payload"], len(a["payload"]))
        rc = L.glacier_hip_page_image_encode_canonical(
            C.byref(a["root"]), a["layers"], a["dim"], a["max_seq"], C.byref(a["ref"]), a["rows"],
            buf, len(a["payload"]), a["challenge"], out, a["cap"], C.byref(n), C.byref(info))
        return "Ok" if rc == 0 else gh.PAGE_IMAGE_ERRORS[info.error]

    assert enc() == "Ok"
    assert enc(cap=751) == "CapacityExceeded"
    assert enc(rows=15) == "InvalidPageImage"            # rows the root does not imply
    assert enc(rows=17) == "InvalidPageImage"            # more than a page
    assert enc(challenge=bytes(32)) == "InvalidPageImage"
    assert enc(payload=payload[:-4]) == "InvalidPageImage"
    assert enc(ref=_c_ref(gh, 502, 0, 9)) == "InvalidPageImage"
    assert enc(ref=_c_ref(gh, 501, 0, 0)) == "InvalidPageImage"
    assert enc(max_seq=8) == "InvalidPageImage"          # committed_len beyond max_seq
    # the destination overlapping the canonical rows
    buf = C.create_string_buffer(752 + 512)
    C.memmove(C.addressof(buf) + 208, payload, 512)
    n = C.c_uint64()
    info = gh.PageImageInfo()
    rc = L.glacier_hip_page_image_encode_canonical(
        C.byref(croot), 2, 2, 32, C.byref(cref), 16, C.addressof(buf) + 208, 512, CHALLENGE,
        C.addressof(buf), 752, C.byref(n), C.byref(info))
    assert rc == gh.INVALID_CHECKPOINT and gh.PAGE_IMAGE_ERRORS[info.error] == "UnsafeDestination"


def test_oracle_restore_remaps_onto_fresh_generations():
    """restoreCheckpointV1 (paged_kv_cache.zig:608-762) on a source chain of
    two pages with arbitrary generations: target refs get generations 1..n,
    the target root generation 2, and a broken source chain is refused."""
    L, dim, max_seq = 2, 2, 32
    own = empty_ownership_digest(77, L, dim, max_seq)
    own = append_ownership_digest(own, 77, 0, 5)
    own = append_ownership_digest(own, 77, 1, 11)
    root = Root(77, 14, 20, 2, own)
    p0 = b"\0" * (L * 2 * 16 * dim * 4)
    p1 = b"\0" * (L * 2 * 4 * dim * 4)
    imgs = [pi.encode_canonical(root, L, dim, max_seq, (77, 0, 5), 16, p0, CHALLENGE),
            pi.encode_canonical(root, L, dim, max_seq, (77, 1, 11), 4, p1, CHALLENGE)]
    troot, refs, _ = pi.restore(imgs, CHALLENGE, 78, L, dim, max_seq)
    tgt = append_ownership_digest(append_ownership_digest(
        empty_ownership_digest(78, L, dim, max_seq), 78, 0, 1), 78, 1, 2)
    assert troot == Root(78, 2, 20, 2, tgt) and refs == [(78, 0, 1), (78, 1, 2)]
    with pytest.raises(pi.ImageError, match="InvalidRestorePlan"):
        pi.restore(imgs[::-1], CHALLENGE, 78, L, dim, max_seq)
    bad = pi.encode_canonical(root, L, dim, max_seq, (77, 1, 12), 4, p1, CHALLENGE)
    with pytest.raises(pi.ImageError, match="InvalidCheckpoint"):
        pi.restore([imgs[0], bad], CHALLENGE, 78, L, dim, max_seq)
    with pytest.raises(pi.ImageError, match="InvalidCheckpoint"):
        pi.restore(imgs, CHALLENGE, 77, L, dim, max_seq)
