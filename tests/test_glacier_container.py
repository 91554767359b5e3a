"""Portable .glacier containers (src/model/format.zig), the qio page codec
(src/model/qio.zig over src/core/quant.zig) and the loader's host assembly
(src/loader.zig), product (glacier_hip_glacier_* / glacier_hip_qio_*)
against the oracle (oracle/glacier_container.py).

The oracle is pinned by the reference's own tests, restated case for case:
format.zig:783-1309 (header / entry round trips, CRC-32, lying page
geometry, numerical little-endian raw decoding, the quant payload schema,
strict admission, reserved domains, exact layout, metadata and index
bounds), qio.zig:172-224 (round trip, layout detection, bad magic, zero
group size, truncated packed bytes) and quant.zig:209-313 (INT8 integers,
two INT4 codes per byte, the spare +8 code from group 16, round-trip bound,
zero tensors, independent group scales). The product must then give the
oracle's verdict and bytes on random containers, random edits of them and
JSON metadata cases; the std.json edge cases (duplicate keys, lone
surrogates, UTF-8) follow RFC 8259 and the Zig parser's documented defaults
and are not pinned by a reference vector.
"""
import hashlib
import json
import random
import struct
import zlib

import numpy as np
import pytest

from oracle import glacier_container as gc
import glacier_build as gb

HS = gc.HEADER_SIZE
META = b'{"format":"portable-test"}'
PAYLOADS = [b"abcdefgh", b"ijklmnop"]
INDEX = HS + len(META)
DATA = INDEX + gc.ENTRY_SIZE * 2
TOTAL = DATA + 16


def _test_container():
    """writeTestContainerV1 (format.zig:729-781)."""
    return gc.build_container(META, [
        dict(layer=i, kind=0 if i == 0 else 255, row_start=4 * i, row_end=4 * i + 4,
             precision=gc.FP16, quant_group=0, payload=p) for i, p in enumerate(PAYLOADS)])


def _both(gh, tmp_path, data, name="c.glacier"):
    """(oracle verdict, product verdict, product container or None)."""
    try:
        gc.open_container(data)
        want = "Ok"
    except gc.GlacError as e:
        want = e.name
    p = tmp_path / name
    p.write_bytes(bytes(data))
    try:
        c = gh.Glacier(str(p))
        got = "Ok"
    except gh.GlacierError as e:
        c, got = None, e.reason
    return want, got, c


def _u64(data, off, v):
    b = bytearray(data)
    b[off:off + 8] = struct.pack("<Q", v)
    return bytes(b)


def _byte(data, off, v):
    b = bytearray(data)
    b[off] = v
    return bytes(b)


# ---- format.zig tests --------------------------------------------------------
def test_header_and_entry_round_trip(gh, tmp_path):
    h = gc.header_bytes(256, 16, 3, 272, 464)
    assert len(h) == HS
    back = gc._read_header(h)
    assert (back["num_pages"], back["meta_offset"], back["page_data_offset"]) == (3, 256, 464)
    e = gc.entry_bytes(42, 7, 5, 0, 128, gc.INT4, 32, 1024, 512, 0xDEADBEEF)
    assert len(e) == gc.ENTRY_SIZE
    r = gc._read_entry(e)
    assert (r["page_id"], r["layer_idx"], r["tensor_kind"], r["precision"], r["crc32"]) == \
        (42, 7, 5, gc.INT4, 0xDEADBEEF)
    # the product reads what the writer wrote
    data = _test_container()
    want, got, c = _both(gh, tmp_path, data)
    assert want == got == "Ok"
    x = c.header()
    assert (x.version, x.header_size, x.meta_offset, x.meta_len, x.num_pages,
            x.page_index_offset, x.page_data_offset, x.page_size_log2, x.container_bytes) == \
        (1, HS, HS, len(META), 2, INDEX, DATA, 18, TOTAL)
    p = c.page(1)
    assert (p.page_id, p.layer_idx, p.tensor_kind, p.row_start, p.row_end, p.precision,
            p.quant_group, p.data_offset, p.data_len, p.crc32) == \
        (1, 1, 255, 4, 8, gc.FP16, 0, DATA + 8, 8, zlib.crc32(PAYLOADS[1]))
    assert c.metadata() == META
    c.close()


def test_crc32_matches_std():
    assert gc.crc32(b"hello glacier") == zlib.crc32(b"hello glacier")


def test_strict_admission_crcs_and_identity(gh, tmp_path):
    """format.zig:988-1090."""
    data = _test_container()
    want, got, c = _both(gh, tmp_path, data)
    assert want == got == "Ok"
    assert c.header().container_bytes == TOTAL and len(c.pages()) == 2
    assert c.page(1).tensor_kind == 255
    c.validate_crcs(3)
    c.validate_crcs()
    ident, n = c.identity()
    assert n == TOTAL and ident == hashlib.sha256(data).digest()
    for bad in (0,):
        with pytest.raises(gh.GlacierError) as e:
            c.validate_crcs(bad)
        assert e.value.reason == "EmptyStreamBuffer"
    assert c.read_page(0) == PAYLOADS[0]
    with pytest.raises(gh.GlacierError) as e:
        c.read_page(0, capacity=7)
    assert e.value.reason == "BufferTooSmall"
    h, pages = gc.open_container(data)
    assert c.source_fingerprint() == gc.source_fingerprint(data, h, pages)
    c.close()
    # one payload byte changed: admission passes, the CRCs and identity move
    x = _byte(data, DATA, ord("X"))
    want, got, c = _both(gh, tmp_path, x, "x.glacier")
    assert want == got == "Ok"
    with pytest.raises(gh.GlacierError) as e:
        c.validate_crcs()
    assert e.value.reason == "CrcMismatch"
    with pytest.raises(gc.GlacError):
        gc.validate_all_crcs(x, gc.open_container(x)[1])
    assert c.identity()[0] != ident
    with pytest.raises(gh.GlacierError) as e:
        c.read_page(0)
    assert e.value.reason == "CrcMismatch"
    # the fingerprint covers the typed entries, not the payload bytes
    assert c.source_fingerprint() == gc.source_fingerprint(data, h, pages)
    c.close()


@pytest.mark.parametrize("off, val, want", [
    (4, 2, "BadVersion"), (6, 1, "BadHeaderSize"), (48, 19, "BadPageSize"),
    (52, 1, "BadReservedField"), (HS - 1, 1, "BadReservedField"), (0, ord("g"), "BadMagic"),
    (INDEX + 12, 16, "BadTensorKind"), (INDEX + 32, 0xFF, "BadPrecision"),
    (INDEX + 34, 1, "BadReservedField"), (INDEX + 56, 1, "BadReservedField"),
    (INDEX + 60, 1, "BadReservedField"),
])
def test_header_and_entry_reserved_domains(gh, tmp_path, off, val, want):
    """format.zig:1092-1185."""
    data = _byte(_test_container(), off, val)
    w, g, _ = _both(gh, tmp_path, data)
    assert w == g == want


def _edit_rows(data, page, field_off, v):
    return _u64(data, INDEX + page * gc.ENTRY_SIZE + field_off, v)


@pytest.mark.parametrize("case, want", [
    ("bad_metadata", "BadMetadata"), ("meta_offset", "BadLayout"),
    ("num_pages_max", "IndexTooLarge"), ("page_id", "BadPageId"), ("row_range", "BadRowRange"),
    ("empty_page", "EmptyPage"), ("gap", "NonContiguousPayload"),
    ("trailing", "TrailingBytes"), ("truncated", "TruncatedPage"),
    ("short_header", "TruncatedHeader"), ("truncated_meta", "TruncatedMeta"),
])
def test_exact_layout_rejections(gh, tmp_path, case, want):
    """format.zig:1187-1267 (plus the truncation checks of openFile)."""
    d = _test_container()
    if case == "bad_metadata":
        d = _byte(d, HS, ord("!"))
    elif case == "meta_offset":
        d = _u64(d, 8, HS + 1)
    elif case == "num_pages_max":
        d = _u64(d, 24, (1 << 64) - 1)
    elif case == "page_id":
        d = _u64(d, INDEX, 1)
    elif case == "row_range":
        d = _u64(d, INDEX + 24, 0)
    elif case == "empty_page":
        d = _u64(d, INDEX + 44, 0)
    elif case == "gap":
        d = _u64(d, INDEX + gc.ENTRY_SIZE + 36, DATA + 8 + 1)
    elif case == "trailing":
        d = d + b"\0"
    elif case == "truncated":
        d = d[:-1]
    elif case == "short_header":
        d = d[:HS - 1]
    elif case == "truncated_meta":
        d = d[:HS + 4]
    w, g, _ = _both(gh, tmp_path, d)
    assert w == g == want


@pytest.mark.parametrize("field, want", [("meta_len", "MetadataTooLarge"),
                                         ("num_pages", "IndexTooLarge")])
def test_metadata_and_index_bounds(gh, tmp_path, field, want):
    """format.zig:1269-1309."""
    if field == "meta_len":
        ml = gc.MAX_METADATA + 1
        h = gc.header_bytes(HS, ml, 0, HS + ml, HS + ml)
    else:
        n = gc.MAX_PAGES + 1
        h = gc.header_bytes(HS, 0, n, HS, HS + n * gc.ENTRY_SIZE)
    w, g, _ = _both(gh, tmp_path, h)
    assert w == g == want


@pytest.mark.parametrize("edit, want", [
    (None, "Ok"), (("data_len", 7), "BadPageGeometry"), (("quant_group", 4), "BadQuantGroup"),
    (("precision", gc.INT2), "UnsupportedPrecision"), (("precision", 5), "UnsupportedPrecision"),
    (("huge", None), "PageGeometryTooLarge"), (("int4_no_group", None), "BadQuantGroup"),
    (("int4_window", None), "PageGeometryTooLarge"),
])
def test_page_geometry_rejects_lying_descriptors(gh, tmp_path, edit, want):
    """format.zig:835-876 on a one-page container."""
    d = gc.build_container(b"{}", [dict(layer=0, kind=255, row_start=0, row_end=4,
                                        precision=gc.FP16, quant_group=0, payload=bytes(8))])
    e0 = HS + 2
    if edit is not None:
        k, v = edit
        if k == "data_len":
            d = _u64(d, e0 + 44, v)
        elif k == "quant_group":
            d = _byte(d, e0 + 33, v)
        elif k == "precision":
            d = _byte(d, e0 + 32, v)
        elif k == "huge":
            n = gc.PAGE_SIZE_BYTES // 2 + 1
            d = _u64(_u64(d, e0 + 24, n), e0 + 44, 2 * n)
        elif k == "int4_no_group":
            d = _byte(d, e0 + 32, gc.INT4)
        elif k == "int4_window":
            n = gc.PAGE_SIZE_BYTES // 4 + 1
            d = _byte(_byte(_u64(d, e0 + 24, n), e0 + 32, gc.INT4), e0 + 33, 32)
    w, g, _ = _both(gh, tmp_path, d)
    assert w == g == want


@pytest.mark.parametrize("prec, raw", [
    (gc.FP32, bytes([0x00, 0x00, 0x80, 0x3F, 0x00, 0x00, 0x20, 0xC0])),
    (gc.FP16, bytes([0x00, 0x3C, 0x00, 0xC1])),
    (gc.BF16, bytes([0x80, 0x3F, 0x20, 0xC0])),
])
def test_raw_page_decoding_is_numerical_and_little_endian(gh, tmp_path, prec, raw):
    """format.zig:878-943."""
    d = gc.build_container(b"{}", [dict(layer=0, kind=255, row_start=0, row_end=2,
                                        precision=prec, quant_group=0, payload=raw)])
    w, g, c = _both(gh, tmp_path, d)
    assert w == g == "Ok"
    assert c.read_page_f32(0).tolist() == [1.0, -2.5]
    assert gc.read_page_f32(d, gc.open_container(d)[1][0]).tolist() == [1.0, -2.5]
    c.close()


def test_quant_payload_schema_binds_entry_geometry(gh, tmp_path):
    """format.zig:945-986."""
    src = np.arange(64, dtype=np.float32)
    payload = gc.encode_page(src, gc.Q_INT4, 32)
    assert gh.qio_encode_f32(src, gc.Q_INT4, 32) == payload
    page = dict(layer=0, kind=255, row_start=0, row_end=64, precision=gc.INT4, quant_group=32,
                payload=payload)
    d = gc.build_container(b"{}", [page])
    w, g, c = _both(gh, tmp_path, d)
    assert w == g == "Ok"
    c.validate_crcs()
    c.close()
    data_off = HS + 2 + gc.ENTRY_SIZE
    for off, v in ((13, 1), (14, 1), (15, 1), (12, 0), (4, 63), (8, 16), (0, 0)):
        bad = _byte(d, data_off + off, v)
        w, g, c = _both(gh, tmp_path, bad, "bad.glacier")
        assert w == g == "Ok"  # admission does not read payloads
        with pytest.raises(gh.GlacierError) as e:
            c.validate_crcs()
        with pytest.raises(gc.GlacError) as o:
            gc.validate_all_crcs(bad, gc.open_container(bad)[1])
        assert e.value.reason == o.value.name == "BadQuantPayload", (off, v)
        c.close()


# ---- qio.zig / quant.zig tests -------------------------------------------------
def test_qio_round_trip_int4():
    """qio.zig:172-196 (a seeded source of the same range)."""
    rng = np.random.default_rng(7)
    src = ((rng.random(128, dtype=np.float32) * 2 - 1) * 0.5).astype(np.float32)
    import glacier_hip as gh
    payload = gh.qio_encode_f32(src, gc.Q_INT4, 32)
    assert payload == gc.encode_page(src, gc.Q_INT4, 32)
    assert gc.read_quant_header(payload) == (128, 32, gc.Q_INT4)
    back = gh.qio_decode_f32(payload)
    assert np.array_equal(back, gc.decode_page(payload))
    assert float(np.max(np.abs(src - back))) < 0.06


def test_qio_layout_and_header_rejections(gh):
    """qio.zig:198-224."""
    with pytest.raises(gh.GlacierError) as e:
        gh.qio_decode_f32(bytes(16))
    assert e.value.reason == "BadMagic"
    h = bytearray(16)
    h[0:4] = struct.pack("<I", gc.QIO_MAGIC)
    h[4:8] = struct.pack("<I", 8)
    h[12] = gc.Q_INT4
    with pytest.raises(gh.GlacierError) as e:
        gh.qio_decode_f32(bytes(h))
    assert e.value.reason == "BadGroupSize"
    enc = gh.qio_encode_f32(np.ones(8, np.float32), gc.Q_INT4, 4)
    for cut, want in ((1, "TruncatedPacked"), (len(enc) - 17, "TruncatedScales"),
                      (len(enc) - 15, "TruncatedHeader")):
        with pytest.raises(gh.GlacierError) as e:
            gh.qio_decode_f32(enc[:len(enc) - cut])
        with pytest.raises(gc.GlacError) as o:
            gc.decode_page(enc[:len(enc) - cut])
        assert e.value.reason == o.value.name == want
    bad = bytearray(enc)
    bad[12] = 2
    with pytest.raises(gh.GlacierError) as e:
        gh.qio_decode_f32(bytes(bad))
    assert e.value.reason == "BadPrecision"
    with pytest.raises(gh.GlacierError) as e:
        gh.qio_encode_f32(np.array([1.0, np.nan], np.float32), gc.Q_INT4, 32)
    assert e.value.reason == "InvalidValue"


def _codes(payload, n):
    groups = -(-n // struct.unpack_from("<I", payload, 8)[0])
    return payload[16 + 4 * groups:], np.frombuffer(payload, "<f4", groups, 16)


def test_quant_known_answers(gh):
    """quant.zig:209-313."""
    p = gh.qio_encode_f32(np.zeros(4, np.float32), gc.Q_INT4, 4)
    packed, scales = _codes(p, 4)
    assert packed == b"\x77\x77" and scales.tolist() == [0.0, 0.0][:1]
    src = np.zeros(16, np.float32)
    src[0] = 1
    packed, scales = _codes(gh.qio_encode_f32(src, gc.Q_INT4, 16), 16)
    assert packed[0] == 0x7F and scales[0] == np.float32(0.125)
    packed, _ = _codes(gh.qio_encode_f32(src[:8], gc.Q_INT4, 8), 8)
    assert packed[0] == 0x7E
    ints = np.array([0, 1, -1, 2, -2, 64, -64, 127, -127], np.float32)
    back = gh.qio_decode_f32(gh.qio_encode_f32(ints, gc.Q_INT8, 16))
    assert float(np.max(np.abs(back - ints))) <= 1.0
    rng = np.random.default_rng(42)
    w = ((rng.random(256, dtype=np.float32) * 2 - 1) * 0.1).astype(np.float32)
    assert float(np.max(np.abs(gh.qio_decode_f32(gh.qio_encode_f32(w, gc.Q_INT4, 64)) - w))) < 0.02
    z = gh.qio_encode_f32(np.zeros(8, np.float32), gc.Q_INT4, 4)
    _, zs = _codes(z, 8)
    assert zs.tolist() == [0.0, 0.0] and not np.signbit(zs).any()
    assert gh.qio_decode_f32(z).tolist() == [0.0] * 8
    two = np.concatenate([np.arange(8) * 0.001, np.arange(8) * 10.0]).astype(np.float32)
    _, s2 = _codes(gh.qio_encode_f32(two, gc.Q_INT4, 8), 16)
    assert s2[0] < s2[1] / 1000
    assert gh.qio_encode_f32(np.zeros(0, np.float32), gc.Q_INT4, 32) == \
        gc.encode_page(np.zeros(0, np.float32), gc.Q_INT4, 32)


@pytest.mark.parametrize("seed", range(6))
def test_product_codec_equals_oracle_on_random_sources(gh, seed):
    rng = np.random.default_rng(seed)
    for _ in range(6):
        n = int(rng.integers(1, 700))
        g = int(rng.choice([4, 8, 16, 32, 64, 33]))
        prec = int(rng.integers(0, 2))
        src = (rng.standard_normal(n) * rng.choice([1e-3, 1.0, 300.0])).astype(np.float32)
        src[rng.random(n) < 0.1] = 0.0
        src[rng.random(n) < 0.05] = -0.0
        a = gh.qio_encode_f32(src, prec, g)
        assert a == gc.encode_page(src, prec, g), (n, g, prec)
        assert np.array_equal(gh.qio_decode_f32(a).view(np.uint32),
                              gc.decode_page(a).view(np.uint32))


# ---- metadata --------------------------------------------------------------------
@pytest.mark.parametrize("meta, ok", [
    (b"{}", True), (b' {"x": -0.5e+3 , "y":[true,false,null,{}]} ', True),
    ('{"a":"\\u00e9\\ud83d\\ude00","b":"é"}'.encode(), True), (b'{"a":{"a":1}}', True),
    (b"", False), (b"[]", False), (b'"s"', False), (b'{"a":1,}', False), (b'{"a":01}', False),
    (b"{'a':1}", False), (b'{"a":NaN}', False), (b'{"a":"\\ud800"}', False),
    (b'{"a":"\\udc00x"}', False), (b'{"a":1,"a":2}', False), (b'{"a":"\x01"}', False),
    (b'{"a":"\xff"}', False), (b'{"a":"\xed\xa0\x80"}', False), (b'{"a":"\xc0\xaf"}', False),
    (b'{"a":1} x', False), (b'{"a" 1}', False), (b'{"a":tru}', False), (b'{"a":1.}', False),
    (b'{"a":-}', False), (b'{"a":[1 2]}', False), (b'{"a":"\\x"}', False), (b"{\"a\":1}\x00", False),
])
def test_metadata_json(gh, tmp_path, meta, ok):
    assert gc.json_object(meta) == ok
    d = gc.build_container(meta, [])
    w, g, c = _both(gh, tmp_path, d)
    assert w == g == ("Ok" if ok else "BadMetadata")
    if c:
        assert c.metadata() == meta
        c.close()


# ---- random containers and edits ----------------------------------------------
def _random_pages(rng):
    pages = []
    for i in range(int(rng.integers(1, 7))):
        prec = int(rng.choice([gc.FP32, gc.FP16, gc.BF16, gc.INT8, gc.INT4]))
        kind = int(rng.choice(sorted(gc.KINDS)))
        n = int(rng.integers(1, 300))
        start = int(rng.integers(0, 1000))
        if prec in (gc.INT8, gc.INT4):
            g = int(rng.choice([8, 16, 32, 64]))
            payload = gc.encode_page(rng.standard_normal(n).astype(np.float32),
                                     gc.Q_INT8 if prec == gc.INT8 else gc.Q_INT4, g)
        else:
            g = 0
            v = rng.standard_normal(n).astype(np.float32)
            payload = gb.raw_pages(0, "other", v, prec)[0]["payload"]
        pages.append(dict(layer=int(rng.integers(0, 3)), kind=kind, row_start=start,
                          row_end=start + n, precision=prec, quant_group=g, payload=payload))
    return pages


@pytest.mark.parametrize("seed", range(8))
def test_product_equals_oracle_on_random_containers_and_edits(gh, tmp_path, seed):
    rng = np.random.default_rng(1000 + seed)
    data = gc.build_container(json.dumps({"seed": seed}).encode(), _random_pages(rng))
    w, g, c = _both(gh, tmp_path, data)
    assert w == g == "Ok"
    h, pages = gc.open_container(data)
    assert c.source_fingerprint() == gc.source_fingerprint(data, h, pages)
    c.validate_crcs()
    for i, p in enumerate(pages):
        assert np.array_equal(c.read_page_f32(i).view(np.uint32),
                              gc.read_page_f32(data, p).view(np.uint32))
    c.close()
    verdicts = set()
    for k in range(40):
        d = bytearray(data)
        if k % 2:
            off = int(rng.integers(0, HS + len(json.dumps({"seed": seed})) +
                                   gc.ENTRY_SIZE * len(pages)))
        else:
            off = int(rng.integers(0, len(d)))
        d[off] ^= 1 << int(rng.integers(0, 8))
        w, g, c = _both(gh, tmp_path, bytes(d), f"e{k}.glacier")
        assert w == g, (k, off)
        verdicts.add(w)
        if c is not None:
            try:
                gc.validate_all_crcs(bytes(d), gc.open_container(bytes(d))[1])
                want = "Ok"
            except gc.GlacError as e:
                want = e.name
            try:
                c.validate_crcs()
                got = "Ok"
            except gh.GlacierError as e:
                got = e.reason
            assert want == got, (k, off)
            c.close()
    assert len(verdicts) >= 2


# ---- loader assembly --------------------------------------------------------------
TINY = dict(num_layers=2, dim=256, hidden_dim=512, num_heads=4, num_kv_heads=2, head_dim=64,
            vocab_size=4096, group_size=32, rms_eps=1e-6, rope_theta=1e6)


def _assembly(gh, tmp_path, data, name="m.glacier"):
    p = tmp_path / name
    p.write_bytes(data)
    c = gh.Glacier(str(p))
    try:
        return c.assemble()
    finally:
        c.close()


def _oracle_assembly(data):
    h, pages = gc.open_container(data)
    try:
        geo = gc.derive_geometry(pages)
        return "Ok", geo, gc.assembly_sha256(gc.materialize(data, pages))
    except gc.GlacError as e:
        return e.name, None, None


@pytest.mark.parametrize("variant", ["int4_embedding", "f32_embedding", "quantized_f32",
                                     "small_pages"])
def test_loader_assembly_equals_oracle(gh, tmp_path, variant):
    host = gh.random_model_host(TINY, 11)
    emb = None
    if variant == "int4_embedding":
        V, D = TINY["vocab_size"], TINY["dim"]
        emb = (gh.synth_int4(11, 0x454D4245, V * D // 2),
               gh.synth_scales_f16(11, 0x454D4246, V * D // 32).view(np.float16).astype(np.float32))
    pages = gb.model_pages(TINY, host, emb=emb,
                           page_elems=4096 if variant == "small_pages" else gb.PAGE_ELEMS)
    if variant == "quantized_f32":  # a converter-style tensor quantized from f32 page by page
        rng = np.random.default_rng(3)
        w = (rng.standard_normal(TINY["dim"] * TINY["dim"]) * 0.05).astype(np.float32)
        pages = [p for p in pages if (p["layer"], p["kind"]) != (1, gb.KIND["attn_o"])]
        pages += gb.quantized_pages(1, "attn_o", w)
        pages += gb.quantized_pages(0, "other", w[:1000], precision=gc.Q_INT8, group=64)
    data = gb.container(pages)
    err, a = _assembly(gh, tmp_path, data)
    want, geo, sha = _oracle_assembly(data)
    assert err == want == "Ok"
    assert (a.num_layers, a.dim, a.hidden_dim, a.vocab_size) == (
        geo["num_layers"], geo["dim"], geo["hidden_dim"], geo["vocab_size"]) == (
        2, 256, 512, 4096)
    assert bytes(a.sha256) == sha


@pytest.mark.parametrize("case", ["crc", "ragged_page", "mixed_groups", "qio_count",
                                  "raw_crc", "qio_precision", "no_pages"])
def test_loader_assembly_rejections_equal_oracle(gh, tmp_path, case):
    host = gh.random_model_host(TINY, 12)
    pages = gb.model_pages(TINY, host, page_elems=4096)
    idx = next(i for i, p in enumerate(pages) if p["kind"] == gb.KIND["mlp_down"])
    p = dict(pages[idx])
    if case == "crc":
        data = bytearray(gb.container(pages))
        h, ps = gc.open_container(bytes(data))
        data[ps[idx]["data_offset"] + 40] ^= 0x10
        data = bytes(data)
    else:
        if case == "ragged_page":  # a non-final page off the group boundary
            u = gb.unpack_codes(p["payload"][16 + 4 * 128:], 4096)
            s = np.frombuffer(p["payload"], "<f4", 128, 16)
            p.update(row_end=p["row_start"] + 3990, payload=gb.int4_payload(u[:3990], s[:125],
                                                                             3990, 32))
        elif case == "mixed_groups":
            u = gb.unpack_codes(p["payload"][16 + 4 * 128:], 4096)
            s = np.frombuffer(p["payload"], "<f4", 128, 16)
            p.update(quant_group=64, payload=gb.int4_payload(u, s[::2], 4096, 64))
        elif case == "qio_count":  # the sub-header disagrees with the entry
            b = bytearray(p["payload"])
            b[4:8] = struct.pack("<I", 4095)
            p["payload"] = bytes(b)
        elif case == "qio_precision":
            b = bytearray(p["payload"])
            b[12] = gc.Q_INT8
            p["payload"] = bytes(b)
        pages[idx] = p
        if case == "raw_crc":
            data = bytearray(gb.container(pages))
            h, ps = gc.open_container(bytes(data))
            j = next(i for i, q in enumerate(ps) if q["tensor_kind"] == gb.KIND["final_norm"])
            data[ps[j]["data_offset"]] ^= 1
            data = bytes(data)
        elif case == "no_pages":
            data = gb.container([])
        else:
            data = gb.container(pages)
    err, _ = _assembly(gh, tmp_path, data)
    want, _, _ = _oracle_assembly(data)
    assert err == want
    assert want == ("NoLayers" if case == "no_pages" else "BadPayload")
