"""Restatement of the portable `.glacier` container of the reference.

TEST INFRASTRUCTURE ONLY: the checker for the product's container reader,
qio codec and loader assembly (glacier_hip_glacier_*, glacier_hip_qio_*,
csrc/glacier_container.cpp). Only tests/ use it.

Follows /root/reference/src/model/format.zig:
  Header writeTo / readFrom            :67-137
  PageEntry writeTo / readFrom         :141-199
  validateHeaderLayoutV1               :211-247
  validatePagesV1                      :249-275
  validatePageGeometryV1               :277-341
  validatePayloadSchemaV1              :351-376
  FileReader.openFile                  :409-478 (metadata: std.json into a
                                        Value, then the object check)
  readPage / validateAllPageCrcs       :488-531
  containerIdentityV1                  :536-575
  readPageDequant / decodeRawPageV1    :638-717
src/model/qio.zig readQuantHeader :52-69, encodePage :72-112, decodePage
:115-162; src/core/quant.zig quantize :36-112, dequantize :114-163;
src/loader.zig sourceFingerprint :167-189, the geometry pass of
loadWithOptions :1226-1268, its (layer, kind) grouping :1270-1434,
concatInt4Pages :1636-1720 and decodePageF32 :1759-1822.

The metadata check restates std.json (Zig 0.15 standard library, absent
here): RFC 8259 JSON, strings UTF-8 without control characters, surrogate
escapes paired, duplicate keys an error (ParseOptions' default), the top
level an object. Containers here are bytes; errors are the reference's
error names.
"""
import hashlib
import json
import math
import struct
import zlib

import numpy as np

MAGIC = b"GLAC"
VERSION = 1
HEADER_SIZE = 256
PAGE_SIZE_LOG2 = 18
PAGE_SIZE_BYTES = 1 << 18
ENTRY_SIZE = 64
MAX_METADATA = 16 * 1024 * 1024
MAX_PAGES = 1024 * 1024
QIO_MAGIC = 0x514F4954
SUB_HEADER = 16

FP16, BF16, INT8, INT4, INT2, TRI, FP32 = 0, 1, 2, 3, 4, 5, 6
Q_INT8, Q_INT4 = 0, 1
KINDS = set(range(16)) | {255}
COMPACT_KINDS = {0, 1, 2, 3, 4, 5, 6, 7, 9}


class GlacError(Exception):
    def __init__(self, name):
        super().__init__(name)
        self.name = name


def crc32(b):
    return zlib.crc32(bytes(b)) & 0xFFFFFFFF


# ---- writers (Header.writeTo / PageEntry.writeTo) -------------------------
def header_bytes(meta_offset, meta_len, num_pages, page_index_offset, page_data_offset,
                 version=VERSION, header_size=HEADER_SIZE, page_size_log2=PAGE_SIZE_LOG2,
                 reserved=0):
    h = (MAGIC + struct.pack("<HHQQQQQII", version, header_size, meta_offset, meta_len,
                             num_pages, page_index_offset, page_data_offset, page_size_log2,
                             reserved))
    return h + bytes(HEADER_SIZE - len(h))


def entry_bytes(page_id, layer_idx, tensor_kind, row_start, row_end, precision, quant_group,
                data_offset, data_len, crc):
    return struct.pack("<QIIQQBBHQQIII", page_id, layer_idx, tensor_kind, row_start, row_end,
                       precision, quant_group, 0, data_offset, data_len, crc, 0, 0)


def build_container(meta, pages):
    """A container from metadata bytes and pages given as dicts with
    layer, kind, row_start, row_end, precision, quant_group and payload."""
    index_off = HEADER_SIZE + len(meta)
    data_off = index_off + ENTRY_SIZE * len(pages)
    out = bytearray(header_bytes(HEADER_SIZE, len(meta), len(pages), index_off, data_off))
    out += meta
    off = data_off
    for i, p in enumerate(pages):
        pl = p["payload"]
        out += entry_bytes(i, p["layer"], p["kind"], p["row_start"], p["row_end"],
                           p["precision"], p["quant_group"], off, len(pl), crc32(pl))
        off += len(pl)
    for p in pages:
        out += p["payload"]
    return bytes(out)


# ---- JSON ------------------------------------------------------------------
def _no_surrogates(v):
    if isinstance(v, str):
        return not any(0xD800 <= ord(ch) <= 0xDFFF for ch in v)
    if isinstance(v, list):
        return all(_no_surrogates(x) for x in v)
    if isinstance(v, dict):
        return all(_no_surrogates(k) and _no_surrogates(x) for k, x in v.items())
    return True


def json_object(b):
    def pairs(items):
        keys = [k for k, _ in items]
        if len(set(keys)) != len(keys):
            raise ValueError("duplicate key")
        return dict(items)

    def bad_constant(_):
        raise ValueError("not JSON")

    try:
        text = bytes(b).decode("utf-8")
        v = json.loads(text, object_pairs_hook=pairs, parse_constant=bad_constant)
    except (UnicodeDecodeError, ValueError, RecursionError):
        return False
    return isinstance(v, dict) and _no_surrogates(v)


# ---- admission -------------------------------------------------------------
def _read_header(b):
    if b[:4] != MAGIC:
        raise GlacError("BadMagic")
    version, header_size = struct.unpack_from("<HH", b, 4)
    if version != VERSION:
        raise GlacError("BadVersion")
    if header_size != HEADER_SIZE:
        raise GlacError("BadHeaderSize")
    mo, ml, npg, pio, pdo = struct.unpack_from("<QQQQQ", b, 8)
    psl, res = struct.unpack_from("<II", b, 48)
    if psl != PAGE_SIZE_LOG2:
        raise GlacError("BadPageSize")
    if res != 0 or any(b[56:HEADER_SIZE]):
        raise GlacError("BadReservedField")
    return dict(version=version, header_size=header_size, meta_offset=mo, meta_len=ml,
                num_pages=npg, page_index_offset=pio, page_data_offset=pdo, page_size_log2=psl,
                reserved=res)


U64 = (1 << 64) - 1


def validate_layout(h, file_size):
    if h["meta_offset"] != HEADER_SIZE:
        raise GlacError("BadLayout")
    if h["meta_len"] > MAX_METADATA:
        raise GlacError("MetadataTooLarge")
    if h["num_pages"] > MAX_PAGES:
        raise GlacError("IndexTooLarge")
    meta_end = h["meta_offset"] + h["meta_len"]
    if meta_end > U64:
        raise GlacError("LayoutOverflow")
    if h["page_index_offset"] != meta_end:
        raise GlacError("BadLayout")
    index_end = h["page_index_offset"] + h["num_pages"] * ENTRY_SIZE
    if index_end > U64:
        raise GlacError("LayoutOverflow")
    if h["page_data_offset"] != index_end:
        raise GlacError("BadLayout")
    if meta_end > file_size:
        raise GlacError("TruncatedMeta")
    if index_end > file_size:
        raise GlacError("TruncatedIndex")


def _read_entry(b):
    (page_id, layer, kind, rs, re_, prec, qg, r0, doff, dlen, crc, r2,
     r3) = struct.unpack("<QIIQQBBHQQIII", b)
    if r0 or r2 or r3:
        raise GlacError("BadReservedField")
    if kind not in KINDS:
        raise GlacError("BadTensorKind")
    if prec > FP32:
        raise GlacError("BadPrecision")
    return dict(page_id=page_id, layer_idx=layer, tensor_kind=kind, row_start=rs, row_end=re_,
                precision=prec, quant_group=qg, data_offset=doff, data_len=dlen, crc32=crc)


def validate_geometry(p):
    n = p["row_end"] - p["row_start"]
    prec = p["precision"]
    if prec in (FP32, FP16, BF16):
        if p["quant_group"] != 0:
            raise GlacError("BadQuantGroup")
        expected = n * (4 if prec == FP32 else 2)
        if expected > U64:
            raise GlacError("LayoutOverflow")
    elif prec in (INT8, INT4):
        if p["quant_group"] == 0:
            raise GlacError("BadQuantGroup")
        if n > PAGE_SIZE_BYTES // 4:
            raise GlacError("PageGeometryTooLarge")
        groups = -(-n // p["quant_group"])
        packed = n if prec == INT8 else -(-n // 2)
        expected = SUB_HEADER + groups * 4 + packed
    else:
        raise GlacError("UnsupportedPrecision")
    if expected != p["data_len"]:
        raise GlacError("BadPageGeometry")
    if prec in (FP32, FP16, BF16) and expected > PAGE_SIZE_BYTES:
        raise GlacError("PageGeometryTooLarge")


def validate_pages(pages, data_offset, file_size):
    expected = data_offset
    for i, p in enumerate(pages):
        if p["page_id"] != i:
            raise GlacError("BadPageId")
        if p["row_end"] <= p["row_start"]:
            raise GlacError("BadRowRange")
        if p["data_len"] == 0:
            raise GlacError("EmptyPage")
        validate_geometry(p)
        if p["data_offset"] != expected:
            raise GlacError("NonContiguousPayload")
        expected = p["data_offset"] + p["data_len"]
        if expected > U64:
            raise GlacError("LayoutOverflow")
        if expected > file_size:
            raise GlacError("TruncatedPage")
    if expected != file_size:
        raise GlacError("TrailingBytes")


def open_container(data):
    """FileReader.openFile over the bytes of a file: (header, pages)."""
    data = bytes(data)
    if len(data) < HEADER_SIZE:
        raise GlacError("TruncatedHeader")
    h = _read_header(data)
    validate_layout(h, len(data))
    if not json_object(data[h["meta_offset"]:h["meta_offset"] + h["meta_len"]]):
        raise GlacError("BadMetadata")
    pages = []
    for i in range(h["num_pages"]):
        o = h["page_index_offset"] + i * ENTRY_SIZE
        pages.append(_read_entry(data[o:o + ENTRY_SIZE]))
    validate_pages(pages, h["page_data_offset"], len(data))
    h["container_bytes"] = len(data)
    return h, pages


# ---- qio / quant -----------------------------------------------------------
def read_quant_header(b):
    if len(b) < SUB_HEADER:
        raise GlacError("TruncatedHeader")
    magic, n, g = struct.unpack_from("<III", b, 0)
    if magic != QIO_MAGIC:
        raise GlacError("BadMagic")
    if g == 0:
        raise GlacError("BadGroupSize")
    if b[12] > Q_INT4:
        raise GlacError("BadPrecision")
    return n, g, b[12]


def _f32(x):
    return float(np.float32(x))


def _min_number(a, b):
    if a < b:
        return a
    if b < a:
        return b
    return a if math.copysign(1.0, a) < 0 else b


def _max_number(a, b):
    if a > b:
        return a
    if b > a:
        return b
    return b if math.copysign(1.0, a) < 0 else a


def quantize(src, precision, group_size):
    """quant.quantize of f32 values: (packed bytes, f32 scales)."""
    src = np.asarray(src, dtype=np.float32)
    n = src.size
    if n == 0:
        return b"", np.zeros(0, np.float32)
    if group_size == 0:
        raise GlacError("BadGroupSize")
    bits = 8 if precision == Q_INT8 else 4
    qzero = (1 << (bits - 1)) - 1
    qmin = -qzero
    qmax = qzero + 1 if precision == Q_INT4 and group_size >= 16 else qzero
    groups = -(-n // group_size)
    scales = np.zeros(groups, np.float32)
    packed = bytearray(-(-n * bits // 8))
    for g in range(groups):
        i, end = g * group_size, min(n, (g + 1) * group_size)
        lo = hi = 0.0
        for v in src[i:end]:
            lo = _min_number(lo, float(v))
            hi = _max_number(hi, float(v))
        neg = np.float32(-lo) / np.float32(-qmin)
        pos = np.float32(hi) / np.float32(qmax)
        scale = np.float32(_max_number(float(neg), float(pos)))
        scales[g] = scale
        inv = np.float32(0.0) if scale == 0 else np.float32(1.0) / scale
        for j in range(i, end):
            y = float(np.float32(src[j]) * inv)
            q = int(math.floor(abs(y) + 0.5)) * (1 if y >= 0 else -1)  # half away from zero
            q = min(max(q, qmin), qmax)
            u = q + qzero
            if bits == 8:
                packed[j] = u
            elif j % 2 == 0:
                packed[j // 2] = (packed[j // 2] & 0xF0) | (u & 0x0F)
            else:
                packed[j // 2] = (packed[j // 2] & 0x0F) | ((u & 0x0F) << 4)
    return bytes(packed), scales


def encode_page(src, precision, group_size):
    """qio.encodePage for f32 source."""
    src = np.asarray(src, dtype=np.float32)
    if not np.all(np.isfinite(src)):
        raise GlacError("InvalidValue")
    packed, scales = quantize(src, precision, group_size)
    return (struct.pack("<IIIB3x", QIO_MAGIC, src.size, group_size, precision) +
            scales.astype("<f4").tobytes() + packed)


def decode_page(payload):
    """qio.decodePage to f32."""
    payload = bytes(payload)
    n, g, prec = read_quant_header(payload)
    groups = -(-n // g)
    off = SUB_HEADER + groups * 4
    if len(payload) < off:
        raise GlacError("TruncatedScales")
    bits = 8 if prec == Q_INT8 else 4
    plen = -(-n * bits // 8)
    if len(payload) - off < plen:
        raise GlacError("TruncatedPacked")
    qmax = (1 << (bits - 1)) - 1
    scales = np.frombuffer(payload, "<f4", groups, SUB_HEADER)
    raw = np.frombuffer(payload, np.uint8, plen, off)
    if bits == 8:
        u = raw[:n].astype(np.int32)
    else:
        u = np.empty(n, np.int32)
        u[0::2] = (raw & 0x0F)[: (n + 1) // 2]
        u[1::2] = (raw >> 4)[: n // 2]
    return ((u - qmax).astype(np.float32) * np.repeat(scales, g)[:n]).astype(np.float32)


# ---- pages -----------------------------------------------------------------
def payload(data, p):
    return bytes(data[p["data_offset"]:p["data_offset"] + p["data_len"]])


def validate_payload_schema(data, p):
    if p["precision"] in (FP32, FP16, BF16):
        return
    if p["precision"] not in (INT8, INT4):
        raise GlacError("UnsupportedPrecision")
    b = payload(data, p)[:SUB_HEADER]
    if len(b) != SUB_HEADER:
        raise GlacError("TruncatedPage")
    if any(b[13:16]):
        raise GlacError("BadQuantPayload")
    try:
        n, g, prec = read_quant_header(b)
    except GlacError:
        raise GlacError("BadQuantPayload")
    if n != p["row_end"] - p["row_start"] or g != p["quant_group"]:
        raise GlacError("BadQuantPayload")
    if prec != (Q_INT8 if p["precision"] == INT8 else Q_INT4):
        raise GlacError("BadQuantPayload")


def validate_all_crcs(data, pages, buffer_bytes=65536):
    if buffer_bytes == 0:
        raise GlacError("EmptyStreamBuffer")
    for p in pages:
        validate_payload_schema(data, p)
        if crc32(payload(data, p)) != p["crc32"]:
            raise GlacError("CrcMismatch")


def read_page(data, p):
    b = payload(data, p)
    if crc32(b) != p["crc32"]:
        raise GlacError("CrcMismatch")
    return b


def _raw_values(b, precision):
    if precision == FP32:
        return np.frombuffer(b, "<f4").astype(np.float32)
    h = np.frombuffer(b, "<u2")
    if precision == FP16:
        return h.view(np.float16).astype(np.float32)
    return (h.astype(np.uint32) << 16).view(np.float32)


def read_page_f32(data, p):
    """readPageDequant(f32)."""
    b = read_page(data, p)
    n = p["row_end"] - p["row_start"]
    if p["precision"] in (FP32, FP16, BF16):
        if n * (4 if p["precision"] == FP32 else 2) != len(b):
            raise GlacError("SizeMismatch")
        return _raw_values(b, p["precision"])
    if p["precision"] in (INT8, INT4):
        validate_payload_schema(data, p)
        return decode_page(b)
    raise GlacError("UnsupportedPrecision")


def identity(data):
    return hashlib.sha256(bytes(data)).digest(), len(data)


def source_fingerprint(data, h, pages):
    s = hashlib.sha256(b"glacier-source-fingerprint-v1\x00")
    s.update(struct.pack("<HQ", h["version"], h["meta_len"]))
    s.update(bytes(data[h["meta_offset"]:h["meta_offset"] + h["meta_len"]]))
    s.update(struct.pack("<Q", len(pages)))
    for p in pages:
        s.update(struct.pack("<QIIQQBBIQ", p["page_id"], p["layer_idx"], p["tensor_kind"],
                             p["row_start"], p["row_end"], p["precision"], p["quant_group"],
                             p["crc32"], p["data_len"]))
    return s.digest()


# ---- loader assembly -------------------------------------------------------
def derive_geometry(pages):
    if not pages:
        raise GlacError("NoLayers")
    layers = dim = hidden = vocab = 0
    for p in pages:
        layers = max(layers, p["layer_idx"] + 1)
        k = p["tensor_kind"]
        if k in (8, 11, 10):
            dim = max(dim, p["row_end"])
        elif k in (5, 7, 6):
            hidden = max(hidden, p["row_end"])
        elif k in (0, 9):
            vocab = max(vocab, p["row_end"])
    if dim > 0:
        if hidden > dim:
            hidden //= dim
        if vocab > dim:
            vocab //= dim
    else:
        dim = hidden // 4 if hidden > 0 else 16
        hidden = 4 * dim
    if layers == 0 or dim == 0:
        raise GlacError("MissingTensor")
    return dict(num_layers=layers, dim=dim, hidden_dim=hidden, vocab_size=vocab)


def _decode_page_loader(data, p):
    try:
        b = read_page(data, p)
    except GlacError:
        raise GlacError("BadPayload")
    if len(b) >= 4 and struct.unpack_from("<I", b)[0] == QIO_MAGIC:
        try:
            return decode_page(b)
        except GlacError:
            raise GlacError("BadPayload")
    if p["precision"] in (FP16, BF16):
        if len(b) % 2:
            raise GlacError("BadPayload")
        return _raw_values(b, p["precision"])
    if len(b) % 4:
        raise GlacError("BadPayload")
    return _raw_values(b, FP32)


def _concat_int4(data, pages):
    group = 0
    total = total_scales = 0
    for i, p in enumerate(pages):
        if p["precision"] != INT4 or p["quant_group"] == 0 or p["row_end"] < p["row_start"]:
            raise GlacError("BadPayload")
        group = group or p["quant_group"]
        if p["quant_group"] != group:
            raise GlacError("BadPayload")
        n = p["row_end"] - p["row_start"]
        if i + 1 < len(pages) and n % group:
            raise GlacError("BadPayload")
        ps = -(-n // group)
        if p["data_len"] != SUB_HEADER + ps * 4 + -(-n // 2):
            raise GlacError("BadPayload")
        total += n
        total_scales += ps
    if total_scales != -(-total // group):
        raise GlacError("BadPayload")
    codes, scales = [], []
    for p in pages:
        try:
            b = read_page(data, p)
            n, g, prec = read_quant_header(b)
        except GlacError:
            raise GlacError("BadPayload")
        if prec != Q_INT4 or g != group or n != p["row_end"] - p["row_start"]:
            raise GlacError("BadPayload")
        ps = -(-n // g)
        off = SUB_HEADER + ps * 4
        plen = (n + 1) // 2
        if len(b) < off or len(b) - off < plen:
            raise GlacError("BadPayload")
        scales.append(np.frombuffer(b, "<f4", ps, SUB_HEADER))
        raw = np.frombuffer(b, np.uint8, plen, off)
        u = np.empty(n, np.uint8)
        u[0::2] = (raw & 0x0F)[: (n + 1) // 2]
        u[1::2] = (raw >> 4)[: n // 2]
        codes.append(u)
    u = np.concatenate(codes)
    packed = np.zeros(-(-total // 2), np.uint8)
    packed[: (total + 1) // 2] |= u[0::2]
    packed[: total // 2] |= (u[1::2] << 4).astype(np.uint8)
    return dict(int4=True, group_size=group, elements=total, packed=packed.tobytes(),
                scales=np.concatenate(scales).astype(np.float32))


def materialize(data, pages):
    """The loader's (layer, kind) groups, visited in (layer, kind) order."""
    by = {}
    for p in pages:
        by.setdefault((p["layer_idx"], p["tensor_kind"]), []).append(p)
    out = {}
    for key in sorted(by):
        ps = sorted(by[key], key=lambda p: p["page_id"])
        if key[1] in COMPACT_KINDS and all(p["precision"] == INT4 for p in ps):
            out[key] = _concat_int4(data, ps)
            continue
        vals = []
        for p in ps:
            v = _decode_page_loader(data, p)
            if v.size != p["row_end"] - p["row_start"]:
                raise GlacError("BadPayload")
            vals.append(v)
        v = np.concatenate(vals).astype(np.float32)
        out[key] = dict(int4=False, group_size=0, elements=v.size, values=v)
    return out


def assembly_sha256(groups):
    """Digest of the materialised groups (the product's
    glacier_hip_glacier_assemble summary; not a reference digest)."""
    s = hashlib.sha256(b"glacier-hip-assembly-v1\x00")
    s.update(struct.pack("<Q", len(groups)))
    for (layer, kind), g in sorted(groups.items()):
        s.update(struct.pack("<IIIIQ", layer, kind, 1 if g["int4"] else 0, g["group_size"],
                             g["elements"]))
        if g["int4"]:
            s.update(g["packed"])
            s.update(g["scales"].astype("<f4").tobytes())
        else:
            s.update(g["values"].astype("<f4").tobytes())
    return s.digest()
