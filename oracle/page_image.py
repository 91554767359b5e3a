"""Restatement of the reference's portable paged-KV checkpoint page images.

TEST INFRASTRUCTURE ONLY: the checker for the product's page-image codec
and checkpoint restore (glacier-engine_amd/csrc/page_image.cpp and the
session entry points over it). Only tests/ use it.

Follows /root/reference/src/continuation_paged_kv_restore.zig:
  constants (ABI, magic, header 208 / footer 32 bytes)   :18-29
  encodedPageImageBytesV1                                 :68-97
  encodeCanonicalPageImageV1                              :101-170
  decodePageImageV1 (checks in this order)                :263-360
  pageImageRootV1 = SHA-256(domain ++ body)               :488-495
  expectedRowsV1                                          :510-517
and /root/reference/src/paged_kv_cache.zig:
  restoreCheckpointV1 (validation, target refs with generations 1..n,
  target root generation 2, next root generation 3)       :608-762
  checkpointEmptyOwnershipDigestV1 / AppendOwnershipDigest :356-380
The canonical payload is the committed rows only, in (layer, K/V, row, dim)
order, as little-endian f32 bit patterns.
"""
import hashlib
import struct

from oracle.paged_kv import (PAGE, PAGE_MAP_ROOT_ABI, PAGE_REF_ABI, Root,
                             append_ownership_digest, empty_ownership_digest)

PAGE_IMAGE_ABI = 0x4743_4B50_0000_0001
MAGIC = b"GCKVPG01"
HEADER = 208
FOOTER = 32
DOMAIN = b"glacier-continuation-paged-kv-page-image-v1\x00"
CHECKPOINT_RESTORE_ABI = 0x4750_4352_0000_0001


class ImageError(Exception):
    """The reference's error, by name (e.g. 'InvalidPageImage')."""


def image_root(body):
    return hashlib.sha256(DOMAIN + body).digest()


U64 = (1 << 64) - 1


def _mul(a, b):
    if a * b > U64:
        raise ImageError("ArithmeticOverflow")
    return a * b


def encoded_bytes(num_layers, dim, committed_rows):
    # usize arithmetic with overflow checks, in the reference's order
    if num_layers == 0 or dim == 0 or committed_rows == 0 or committed_rows > PAGE:
        raise ImageError("InvalidPageImage")
    elements = _mul(_mul(_mul(num_layers, 2), committed_rows), dim)
    total = _mul(elements, 4) + HEADER + FOOTER
    if total > U64:
        raise ImageError("ArithmeticOverflow")
    return total


def expected_rows(root, logical_page):
    return min(root.committed_len - logical_page * PAGE, PAGE)


def _pack_root(r):
    return struct.pack("<5Q", PAGE_MAP_ROOT_ABI, r.cache_instance, r.generation, r.committed_len,
                       r.committed_pages) + r.ownership_sha256


def _pack_ref(inst, logical_page, gen):
    return struct.pack("<4Q", PAGE_REF_ABI, inst, logical_page, gen)


def encode_canonical(source_root, num_layers, dim, max_seq, ref, committed_rows, payload,
                     challenge):
    """encodeCanonicalPageImageV1; ref = (cache_instance, logical_page, generation)."""
    need = encoded_bytes(num_layers, dim, committed_rows)
    count = (need - HEADER - FOOTER) // 4
    inst, lp, gen = ref
    r = source_root
    if (len(payload) != count * 4 or r.cache_instance == 0 or r.generation == 0
            or r.committed_len == 0 or r.committed_len > max_seq or r.committed_pages == 0
            or inst != r.cache_instance or lp >= r.committed_pages or gen == 0
            or committed_rows != expected_rows(r, lp) or not any(r.ownership_sha256)
            or not any(challenge)):
        raise ImageError("InvalidPageImage")
    if r.committed_pages != -(-r.committed_len // PAGE):
        raise ImageError("InvalidPageImage")
    body = (MAGIC + struct.pack("<QQII", PAGE_IMAGE_ABI, need, 0, 0) + _pack_root(r) +
            struct.pack("<3Q", num_layers, dim, max_seq) + _pack_ref(inst, lp, gen) +
            struct.pack("<2Q", committed_rows, count) + bytes(challenge))
    assert len(body) == HEADER
    body += bytes(payload)
    return body + image_root(body)


def decode(data, expected_challenge):
    """decodePageImageV1: a dict of the image's fields, or ImageError."""
    if len(data) < HEADER + FOOTER:
        raise ImageError("InvalidLength")
    if data[0:8] != MAGIC:
        raise ImageError("InvalidMagic")
    abi, ln, flags, res = struct.unpack_from("<QQII", data, 8)
    if abi != PAGE_IMAGE_ABI:
        raise ImageError("InvalidAbi")
    if ln != len(data):
        raise ImageError("InvalidLength")
    if flags != 0 or res != 0:
        raise ImageError("InvalidFlags")
    rabi, rinst, rgen, rlen, rpages = struct.unpack_from("<5Q", data, 32)
    rown = bytes(data[72:104])
    num_layers, dim, max_seq = struct.unpack_from("<3Q", data, 104)
    fabi, finst, flp, fgen = struct.unpack_from("<4Q", data, 128)
    rows, count = struct.unpack_from("<2Q", data, 160)
    challenge = bytes(data[176:208])
    need = encoded_bytes(num_layers, dim, rows)
    if len(data) != need:
        raise ImageError("InvalidLength")
    if _mul(count, 4) != len(data) - HEADER - FOOTER:
        raise ImageError("InvalidPageImage")
    payload = bytes(data[HEADER:HEADER + count * 4])
    root_digest = bytes(data[HEADER + count * 4:])
    if root_digest != image_root(bytes(data[:len(data) - FOOTER])):
        raise ImageError("InvalidPageImage")
    root = Root(rinst, rgen, rlen, rpages, rown)
    exp_pages = -(-rlen // PAGE)
    if (rabi != PAGE_MAP_ROOT_ABI or rinst == 0 or rgen == 0 or rlen == 0 or rlen > max_seq
            or rpages == 0 or rpages != exp_pages or not any(rown) or fabi != PAGE_REF_ABI
            or finst != rinst or flp >= rpages or fgen == 0 or num_layers == 0 or dim == 0
            or max_seq == 0 or rows != expected_rows(root, flp) or not any(expected_challenge)
            or challenge != bytes(expected_challenge)):
        raise ImageError("InvalidPageImage")
    if count != _mul(_mul(_mul(num_layers, 2), rows), dim):
        raise ImageError("InvalidPageImage")
    return dict(source_root=root, num_layers=num_layers, dim=dim, max_seq=max_seq,
                source_ref=(finst, flp, fgen), committed_rows=rows, payload=payload,
                challenge=challenge, image_sha256=root_digest)


def restore(images, challenge, target_instance, num_layers, dim, max_seq):
    """Decode every page image (restoreAndCommitV1's decode loop,
    continuation_paged_kv_restore.zig:405-447) and remap them onto a fresh
    cache (restoreCheckpointV1): returns (target root, target refs, pages'
    canonical payloads)."""
    decoded = []
    for i, wire in enumerate(images):
        d = decode(wire, challenge)
        if d["source_ref"][1] != i:
            raise ImageError("InvalidRestorePlan")
        if decoded and (d["source_root"] != decoded[0]["source_root"]
                        or (d["num_layers"], d["dim"], d["max_seq"]) !=
                        (decoded[0]["num_layers"], decoded[0]["dim"], decoded[0]["max_seq"])):
            raise ImageError("ForeignCheckpoint")
        decoded.append(d)
    src = decoded[0]["source_root"]
    if (decoded[0]["num_layers"], decoded[0]["dim"], decoded[0]["max_seq"]) != \
            (num_layers, dim, max_seq):
        raise ImageError("InvalidCheckpoint")
    if (src.cache_instance == target_instance or src.committed_len > max_seq
            or src.committed_pages != len(images)):
        raise ImageError("InvalidCheckpoint")
    own = empty_ownership_digest(src.cache_instance, num_layers, dim, max_seq)
    for i, d in enumerate(decoded):
        inst, lp, gen = d["source_ref"]
        own = append_ownership_digest(own, inst, lp, gen)
    if own != src.ownership_sha256:
        raise ImageError("InvalidCheckpoint")
    tgt = empty_ownership_digest(target_instance, num_layers, dim, max_seq)
    refs = []
    for i in range(len(images)):
        refs.append((target_instance, i, i + 1))
        tgt = append_ownership_digest(tgt, target_instance, i, i + 1)
    root = Root(target_instance, 2, src.committed_len, src.committed_pages, tgt)
    return root, refs, [d["payload"] for d in decoded]
