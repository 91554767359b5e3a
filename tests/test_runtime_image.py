"""Prepared runtime images (.glrt) on the CPU: the oracle's restatement of
the reference codec (oracle/runtime_image.py) pinned by the reference's own
constants and tests, and the product's reader (glacier_hip_glrt_open,
csrc/runtime_image.cpp) giving the reference's verdict on valid and broken
images. The reference tests restated here are in
src/model/runtime_image.zig:1560-2193."""
import hashlib
import random
import struct

import numpy as np
import pytest

from oracle import runtime_image as ri
from glrt_images import raw_record, int4_record, reference_test_config, repair_crcs

# runtime_image.zig:44-82, the fingerprints as the reference tables them
REF_ABI = {
    (1, "aarch64"): "dc5fe778a28150235c6f11c53bbf876e130dde0804c3b7a492f4de7e059bc7ad",
    (1, "portable"): "0c1f185ceff5e9d366a920c8b0046f1543290f85965fbd7cb13f21fe2eec42b6",
    (2, "aarch64"): "d0d7df06350af6b2d48e282f65ff873a3cf95bd6397b1d2d26cc6e679304e06f",
    (2, "portable"): "8f291472be36fab2d8e32bfbb87671ebbb18a982036a2d17dc06cbe2907ec890",
}


def test_oracle_abi_fingerprints_are_the_reference_constants():
    for key, hexd in REF_ABI.items():
        assert ri.abi_fingerprint(*key).hex() == hexd


def test_crc32_is_ieee():
    # the published CRC-32 check value
    assert ri.crc32(b"123456789") == 0xCBF43926


def _roundtrip_records():
    # runtime_image.zig:1588-1656
    raw_values = np.array([1.25, -2.5, 3.75, 4.0], np.float32)
    packed = bytes([0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE])
    return [raw_record(0, "final_norm", raw_values),
            int4_record(0, "attn_q", np.frombuffer(packed, np.uint8), 1, 16,
                        scales_f32=np.array([0.5], np.float32),
                        scales_f16=np.array([0.5], np.float16), group=16)]


def _open(gh, path, **kw):
    try:
        img = gh.GlrtImage(str(path), **kw)
    except gh.GlrtError as e:
        return e.reason, None
    return "Ok", img


def _oracle_verdict(data, **kw):
    try:
        ri.open_image(data, **kw)
    except ri.ImageError as e:
        return str(e)
    return "Ok"


def test_roundtrip_exposes_mapped_typed_views(gh, tmp_path):
    src = ri.fingerprint(b"source-model")
    p = tmp_path / "model.glrt"
    data = ri.write_image(str(p), reference_test_config(), src, _roundtrip_records())
    verdict, img = _open(gh, p, expected_source=src)
    assert verdict == "Ok"
    try:
        i = img.info
        assert i.version == 2 and i.record_count == 2 and i.file_size == len(data)
        assert i.file_size % 64 == 0 and bytes(i.source_fingerprint) == src
        assert bytes(i.abi_fingerprint) == ri.abi_fingerprint(2)
        assert (i.dim, i.hidden_dim, i.layers, i.vocab, i.heads, i.head_dim, i.kv_heads) == \
            (16, 32, 2, 64, 2, 8, 1)
        assert i.tie_embeddings == 1 and i.rope_theta == 10000.0
        sha, n = img.identity()
        assert n == len(data) and sha == hashlib.sha256(data).digest()
        raw = img.find(0, ri.KIND["final_norm"])
        assert raw.role == ri.ROLE_TENSOR and raw.pair_nibble_layout == ri.PAIR_NONE
        assert any(raw.payload_digest) and raw.offset[4] % 64 == 0
        assert np.array_equal(np.frombuffer(img.stream(raw, 4), np.float32),
                              np.array([1.25, -2.5, 3.75, 4.0], np.float32))
        q = img.find(0, ri.KIND["attn_q"])
        assert img.stream(q, 0) == bytes([0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE])
        assert np.frombuffer(img.stream(q, 1), np.float32).tolist() == [0.5]
        assert np.frombuffer(img.stream(q, 2), np.float16).tolist() == [0.5]
        assert img.stream(q, 3) == b""
        assert img.find(1, ri.KIND["attn_q"]) is None
        # every decoded field equals the oracle's decode of the same bytes
        _, orecs = ri.open_image(data)
        for r, o in zip(img.records(), orecs):
            assert (r.layer_idx, r.kind, r.role, r.encoding, r.packed_layout,
                    r.pair_nibble_layout, r.group_size, r.out_f, r.in_f, r.flags,
                    r.payload_crc32, r.num_elements, bytes(r.payload_digest)) == \
                (o.layer, o.kind, o.role, o.encoding, o.layout, o.pair_layout, o.group_size,
                 o.out_f, o.in_f, o.flags, o.crc, o.num_elements, o.digest)
            for s, name in enumerate(ri.STREAMS):
                assert (r.offset[s], r.length[s]) == o.rng(name)
    finally:
        img.close()


def test_reader_keeps_read_only_v1_compatibility(gh, tmp_path):
    # runtime_image.zig:1810-1842
    src = ri.fingerprint(b"legacy-source")
    p = tmp_path / "legacy.glrt"
    ri.write_image_v1(str(p), reference_test_config(), src,
                      [(0, ri.KIND["final_norm"], [1.5, -2.0, 3.25, 4.5])])
    verdict, img = _open(gh, p, expected_source=src)
    assert verdict == "Ok"
    r = img.find(0, ri.KIND["final_norm"])
    assert img.info.version == 1 and r.role == 0 and r.pair_nibble_layout == 0xFFFF
    assert not any(r.payload_digest)
    assert np.frombuffer(img.stream(r, 4), np.float32).tolist() == [1.5, -2.0, 3.25, 4.5]
    img.close()
    assert _open(gh, p, allow_v1=False)[0] == "LegacyVersionDisabled"


def test_open_rejects_payload_corruption_and_fingerprint_mismatch(gh, tmp_path):
    # runtime_image.zig:1968-2025
    p = tmp_path / "model.glrt"
    src = ri.fingerprint(b"source-a")
    data = ri.write_image(str(p), reference_test_config(), src,
                          [raw_record(0, "final_norm", [1, 2, 3, 4])])
    assert _open(gh, p, expected_source=ri.fingerprint(b"source-b"))[0] == \
        "SourceFingerprintMismatch"
    # an image written for another execution layout
    q = tmp_path / "arm.glrt"
    ri.write_image(str(q), reference_test_config(), src, [raw_record(0, "final_norm", [1, 2, 3, 4])],
                   abi_fp=ri.abi_fingerprint(2, "aarch64"))
    assert _open(gh, q)[0] == "AbiFingerprintMismatch"
    _, recs = ri.open_image(data)
    off = recs[0].rng("raw")[0]
    bad = bytearray(data)
    bad[off] = 0xFF
    p.write_bytes(bytes(bad))
    assert _open(gh, p, verify_payload_crc=False)[0] == "DigestMismatch"
    assert _open(gh, p)[0] == "CrcMismatch"
    assert _open(gh, p, verify_payload_crc=False, verify_payload_digest=False)[0] == "Ok"


def test_v2_digest_binds_descriptor(gh, tmp_path):
    # runtime_image.zig:2027-2082
    data = ri.write_image(None, reference_test_config(), ri.fingerprint(b"digest-source"),
                          [raw_record(0, "final_norm", [1, 2, 3, 4])])
    d = bytearray(data)
    struct.pack_into("<I", d, ri.HEADER_SIZE + 4, ri.KIND["input_norm"])
    p = tmp_path / "descriptor.glrt"
    p.write_bytes(repair_crcs(bytes(d)))
    assert _open(gh, p)[0] == "DigestMismatch"
    d = bytearray(data)
    d[ri.HEADER_SIZE + ri.V2_DIGEST_OFFSET] ^= 0xFF
    p = tmp_path / "digest.glrt"
    p.write_bytes(repair_crcs(bytes(d)))
    assert _open(gh, p)[0] == "DigestMismatch"


def _two_record_image():
    return ri.write_image(None, reference_test_config(), ri.fingerprint(b"x"),
                          [raw_record(0, "final_norm", np.arange(4)),
                           int4_record(0, "attn_q", np.arange(8, dtype=np.uint8), 1, 16,
                                       scales_f32=np.array([0.25], np.float32), group=16)])


def _patch_index(data, rec, offset, fmt, value):
    d = bytearray(data)
    struct.pack_into(fmt, d, ri.HEADER_SIZE + rec * ri.RECORD_SIZE + offset, value)
    return repair_crcs(bytes(d))


@pytest.mark.parametrize("case, want", [
    # record validation (runtime_image.zig:2084-2117, 2131-2192)
    (("raw_off", 1), "BadAlignment"),          # raw offset + 1: misaligned
    (("raw_len_only",), "BadBounds"),          # offset 0 with a length
    (("raw_beyond",), "BadBounds"),            # past the end of the file
    (("overlap_streams",), "OverlappingPayload"),
    (("overlap_records",), "OverlappingPayload"),
    (("flags",), "BadFlags"),
    (("reserved_124",), "BadReservedField"),
    (("role",), "BadRole"),
    (("pair_layout",), "BadPairNibbleLayout"),
    (("kind",), "BadTensorKind"),
    (("encoding",), "BadEncoding"),
    (("layout",), "BadPackedLayout"),
    (("duplicate",), "DuplicateRecord"),
    (("shape",), "BadTensorShape"),
    (("no_scales",), "MissingScales"),
    (("zero_digest",), "MissingDigest"),
    # header (Header.decode / validateHeaderBytes)
    (("header_reserved",), "BadReservedField"),
    (("version",), "BadVersion"),
    (("record_size",), "BadRecordSize"),
    (("magic",), "BadMagic"),
    (("header_crc",), "HeaderCrcMismatch"),
    (("index_crc",), "IndexCrcMismatch"),
    (("config",), "BadConfig"),
    (("tie_byte",), "BadConfig"),
    (("truncated",), "BadBounds"),
])
def test_broken_images_fail_like_the_reference(gh, tmp_path, case, want):
    data = _two_record_image()
    _, recs = ri.open_image(data)
    raw_off = recs[0].rng("raw")[0]
    q_packed, q_scales = recs[1].rng("packed"), recs[1].rng("scales_f32")
    kind = case[0]
    if kind == "raw_off":
        data = _patch_index(data, 0, 40 + 16 * 4, "<Q", raw_off + case[1])
    elif kind == "raw_len_only":
        data = _patch_index(data, 0, 40 + 16 * 4, "<Q", 0)
    elif kind == "raw_beyond":
        data = _patch_index(data, 0, 40 + 16 * 4, "<Q", len(data))
    elif kind == "overlap_streams":
        data = _patch_index(data, 1, 40 + 16 * 1, "<Q", q_packed[0])
    elif kind == "overlap_records":
        data = _patch_index(data, 1, 40 + 16 * 1, "<Q", raw_off)
    elif kind == "flags":
        data = _patch_index(data, 0, 24, "<I", 1)
    elif kind == "reserved_124":
        data = _patch_index(data, 0, 124, "<B", 1)
    elif kind == "role":
        data = _patch_index(data, 0, ri.V2_ROLE_OFFSET, "<H", 0x7FFF)
    elif kind == "pair_layout":
        data = _patch_index(data, 0, ri.V2_PAIR_LAYOUT_OFFSET, "<H", 0x7FFF)
    elif kind == "kind":
        data = _patch_index(data, 0, 4, "<I", 77)
    elif kind == "encoding":
        data = _patch_index(data, 0, 8, "<H", 9)
    elif kind == "layout":
        data = _patch_index(data, 0, 10, "<H", 5)
    elif kind == "duplicate":
        data = _patch_index(data, 1, 4, "<I", ri.KIND["final_norm"])
    elif kind == "shape":
        data = _patch_index(data, 0, 20, "<I", 5)
    elif kind == "no_scales":
        d = _patch_index(data, 1, 40 + 16 * 1, "<Q", 0)
        data = _patch_index(d, 1, 48 + 16 * 1, "<Q", 0)
    elif kind == "zero_digest":
        d = bytearray(data)
        off = ri.HEADER_SIZE + ri.V2_DIGEST_OFFSET
        d[off:off + 32] = bytes(32)
        data = repair_crcs(bytes(d))
    elif kind == "header_reserved":
        d = bytearray(data)
        d[ri.HEADER_SIZE - 1] = 1
        data = bytes(d)
    elif kind == "version":
        d = bytearray(data)
        struct.pack_into("<H", d, 4, 3)
        data = bytes(d)
    elif kind == "record_size":
        d = bytearray(data)
        struct.pack_into("<H", d, 8, ri.V1_RECORD_SIZE)
        data = bytes(d)
    elif kind == "magic":
        data = b"GLRX" + data[4:]
    elif kind == "header_crc":
        d = bytearray(data)
        d[ri.HEADER_CRC_OFFSET] ^= 1
        data = bytes(d)
    elif kind == "index_crc":
        d = bytearray(data)
        d[ri.HEADER_SIZE + 33] ^= 1
        data = bytes(d)
    elif kind == "config":
        d = bytearray(data)
        struct.pack_into("<f", d, 144, -1.0)
        data = bytes(d)
    elif kind == "tie_byte":
        d = bytearray(data)
        d[140] = 2
        data = bytes(d)
    elif kind == "truncated":
        data = data[:-64]
    assert _oracle_verdict(data) == want
    p = tmp_path / "bad.glrt"
    p.write_bytes(data)
    verdict, img = _open(gh, p)
    if img:
        img.close()
    assert verdict == want


def test_random_byte_corruption_verdicts_match_the_oracle(gh, tmp_path):
    """Single-byte corruptions anywhere in a valid multi-record image: the
    product and the restated reference reject (or accept) each one with the
    same error, with and without CRC repair of the header and index."""
    base = ri.write_image(None, reference_test_config(), ri.fingerprint(b"fuzz"),
                          [raw_record(0, "input_norm", np.arange(16)),
                           int4_record(0, "attn_q", np.arange(128, dtype=np.uint8), 16, 16,
                                       scales_f32=np.full(8, 0.5, np.float32),
                                       scales_f16=np.full(8, 0.5, np.float16), group=32),
                           raw_record(ri.GLOBAL_LAYER, "final_norm", np.ones(16))])
    rng = random.Random(0x474C5254)
    p = tmp_path / "fuzz.glrt"
    seen = set()
    for trial in range(240):
        d = bytearray(base)
        pos = rng.randrange(len(d)) if trial % 2 else rng.randrange(ri.HEADER_SIZE + 3 * ri.RECORD_SIZE)
        d[pos] ^= 1 << rng.randrange(8)
        data = bytes(d)
        if trial % 3 == 0 and pos >= ri.HEADER_SIZE:
            data = repair_crcs(data)
        want = _oracle_verdict(data)
        p.write_bytes(data)
        got, img = _open(gh, p)
        if img:
            img.close()
        assert got == want, (trial, pos)
        seen.add(want)
    assert len(seen) >= 8, seen
