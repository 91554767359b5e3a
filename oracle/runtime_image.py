"""Restatement of the reference's GLRT prepared runtime-image codec.

TEST INFRASTRUCTURE ONLY: writes the `.glrt` images the tests load through
the product (glacier-engine_amd/csrc/runtime_image.cpp) and decides, as the
reference would, whether an image opens. Only tests/ use it.

Follows /root/reference/src/model/runtime_image.zig:
  constants, ABI fingerprints          :21-105  (the fingerprints are SHA-256
                                                 of the strings quoted there)
  Header.encode / decode               :200-276
  Record.encode / decode               :324-433
  Record.validateDescriptor            :435-541
  Record.validateBoundsForVersion      :543-573
  writeUnpublishedWithProviderV1       :1210-1327 (streams in all_streams order,
                                                  64-byte aligned; payload CRC32
                                                  over the streams; v2 digest =
                                                  SHA-256(descriptor[0:128] ++ streams))
  validateHeaderBytes                  :1335-1372
  MappedImage.validateIndexAndRecords  :1008-1049 and verifyRecord :990-1006
and /root/reference/src/loader.zig for the prepared-model record set:
  validatePreparedConfig :618-654, validatePreparedRecordSet :656-716,
  isExpectedPreparedRecord :731-768, preparedRaw :785-809, preparedInt4 :811-868.
Tensor kinds: src/model/format.zig:46-64. CRC32 is the IEEE polynomial
(std.hash.Crc32 = zlib.crc32).
"""
import hashlib
import struct
import zlib

MAGIC = b"GLRT"
HEADER_SIZE = 512
V1_RECORD_SIZE = 128
RECORD_SIZE = 160
DATA_ALIGNMENT = 64
GLOBAL_LAYER = 0xFFFFFFFF
HEADER_CRC_OFFSET = 156
V2_ROLE_OFFSET, V2_PAIR_LAYOUT_OFFSET, V2_DIGEST_OFFSET = 120, 122, 128

# runtime_image.zig:44-82: SHA-256 of these strings
ABI_STRINGS = {
    (1, "aarch64"): b"GLRT v1 header512 record128 rows4-k16 f16-v1",
    (1, "portable"): b"GLRT v1 header512 record128 row-major-f32-v1",
    (2, "aarch64"): b"GLRT v2 header512 record160 roles pair-nibble descriptor-payload-sha256 rows4-k16 f16-v2",
    (2, "portable"): b"GLRT v2 header512 record160 roles pair-nibble descriptor-payload-sha256 row-major-f32-v2",
}


def abi_fingerprint(version, arch="portable"):
    return hashlib.sha256(ABI_STRINGS[(version, arch)]).digest()


def fingerprint(b):
    return hashlib.sha256(b).digest()


# format.zig:46-64
KIND = dict(embedding=0, attn_q=1, attn_k=2, attn_v=3, attn_o=4, mlp_up=5, mlp_down=6,
            mlp_gate=7, input_norm=8, lm_head=9, final_norm=10, post_attn_norm=11,
            attn_q_bias=12, attn_k_bias=13, attn_v_bias=14, attn_o_bias=15, other=255)
ENC_RAW_F32, ENC_INT4, ENC_PAIR_NIBBLE = 0, 1, 2
LAYOUT_ROW_MAJOR, LAYOUT_ROWS4_K16, LAYOUT_NONE = 0, 1, 0xFFFF
ROLE_TENSOR, ROLE_MLP_GATE_UP_PAIR = 0, 1
PAIR_ROWS4_K16, PAIR_NONE = 0, 0xFFFF
STREAMS = ("packed", "scales_f32", "scales_f16", "scales_f16_rows4", "raw")


class ImageError(Exception):
    """The reference's error, by name (e.g. 'CrcMismatch')."""


def crc32(b):
    return zlib.crc32(b) & 0xFFFFFFFF


def align(v, a=DATA_ALIGNMENT):
    return (v + a - 1) & ~(a - 1)


class Config:
    def __init__(self, dim, hidden_dim, layers, vocab, heads, head_dim, kv_heads, rms_eps=1e-6,
                 rope_theta=1e6, tie_embeddings=False):
        self.dim, self.hidden_dim, self.layers, self.vocab = dim, hidden_dim, layers, vocab
        self.heads, self.head_dim, self.kv_heads = heads, head_dim, kv_heads
        self.rms_eps, self.rope_theta, self.tie_embeddings = rms_eps, rope_theta, tie_embeddings


def encode_header(version, record_count, data_offset, file_size, source_fp, abi_fp, cfg,
                  index_crc, header_crc, flags=0, index_offset=HEADER_SIZE):
    out = bytearray(HEADER_SIZE)
    out[0:4] = MAGIC
    struct.pack_into("<HHHHI", out, 4, version, HEADER_SIZE,
                     RECORD_SIZE if version == 2 else V1_RECORD_SIZE, DATA_ALIGNMENT, flags)
    struct.pack_into("<QQQQ", out, 16, record_count, index_offset, data_offset, file_size)
    out[48:80] = source_fp
    out[80:112] = abi_fp
    struct.pack_into("<7I", out, 112, cfg.dim, cfg.hidden_dim, cfg.layers, cfg.vocab, cfg.heads,
                     cfg.head_dim, cfg.kv_heads)
    out[140] = 1 if cfg.tie_embeddings else 0
    struct.pack_into("<ffII", out, 144, cfg.rms_eps, cfg.rope_theta, index_crc, header_crc)
    return bytes(out)


class Record:
    def __init__(self, layer, kind, encoding, layout, group_size, out_f, in_f, num_elements=None,
                 role=ROLE_TENSOR, pair_layout=PAIR_NONE, flags=0, ranges=None, crc=0,
                 digest=b"\0" * 32):
        self.layer, self.kind, self.encoding, self.layout = layer, kind, encoding, layout
        self.group_size, self.out_f, self.in_f = group_size, out_f, in_f
        self.num_elements = out_f * in_f if num_elements is None else num_elements
        self.role, self.pair_layout, self.flags = role, pair_layout, flags
        self.ranges = dict(ranges or {})  # stream -> (offset, len)
        self.crc, self.digest = crc, digest

    def rng(self, s):
        return self.ranges.get(s, (0, 0))

    def encode(self, version):
        out = bytearray(RECORD_SIZE)
        struct.pack_into("<IIHHIIIIIQ", out, 0, self.layer, self.kind, self.encoding, self.layout,
                         self.group_size, self.out_f, self.in_f, self.flags, self.crc,
                         self.num_elements)
        for i, s in enumerate(STREAMS):
            struct.pack_into("<QQ", out, 40 + 16 * i, *self.rng(s))
        if version == 2:
            struct.pack_into("<HH", out, V2_ROLE_OFFSET, self.role, self.pair_layout)
            out[V2_DIGEST_OFFSET:] = self.digest
            return bytes(out)
        return bytes(out[:V1_RECORD_SIZE])

    @staticmethod
    def decode(b, version):
        if version == 1 and any(b[120:128]):
            raise ImageError("BadReservedField")
        if version == 2 and any(b[124:128]):
            raise ImageError("BadReservedField")
        layer, kind, enc, lay, gs, of, inf, flags, crc, ne = struct.unpack_from("<IIHHIIIIIQ", b, 0)
        if kind not in KIND.values():
            raise ImageError("BadTensorKind")
        if enc not in (0, 1, 2):
            raise ImageError("BadEncoding")
        if lay not in (0, 1, 0xFFFF):
            raise ImageError("BadPackedLayout")
        role, pl, dg = ROLE_TENSOR, PAIR_NONE, b"\0" * 32
        if version == 2:
            role, pl = struct.unpack_from("<HH", b, V2_ROLE_OFFSET)
            if role not in (0, 1):
                raise ImageError("BadRole")
            if pl not in (0, 0xFFFF):
                raise ImageError("BadPairNibbleLayout")
            dg = bytes(b[V2_DIGEST_OFFSET:RECORD_SIZE])
        ranges = {s: struct.unpack_from("<QQ", b, 40 + 16 * i) for i, s in enumerate(STREAMS)}
        return Record(layer, kind, enc, lay, gs, of, inf, ne, role, pl, flags,
                      {s: r for s, r in ranges.items() if r != (0, 0)}, crc, dg)

    def validate_descriptor(self, version, require_digest):
        # runtime_image.zig:435-541
        if self.flags:
            raise ImageError("BadFlags")
        if version == 1:
            if self.role != ROLE_TENSOR or self.pair_layout != PAIR_NONE or any(self.digest):
                raise ImageError("BadVersionedRecord")
            if self.encoding == ENC_PAIR_NIBBLE:
                raise ImageError("BadEncoding")
        elif require_digest and not any(self.digest):
            raise ImageError("MissingDigest")
        if self.out_f == 0 or self.in_f == 0 or self.num_elements == 0:
            raise ImageError("BadTensorShape")
        if self.out_f * self.in_f != self.num_elements:
            raise ImageError("BadTensorShape")
        L = {s: self.rng(s)[1] for s in STREAMS}
        if self.encoding == ENC_RAW_F32:
            if (self.role != ROLE_TENSOR or self.layout != LAYOUT_NONE or self.pair_layout != PAIR_NONE
                    or self.group_size != 0):
                raise ImageError("BadEncoding")
            if L["raw"] == 0 or L["packed"] or L["scales_f32"] or L["scales_f16"] or L["scales_f16_rows4"]:
                raise ImageError("BadEncoding")
            if L["raw"] != self.num_elements * 4:
                raise ImageError("BadTensorShape")
        elif self.encoding == ENC_INT4:
            if (self.role != ROLE_TENSOR or self.pair_layout != PAIR_NONE or self.layout == LAYOUT_NONE
                    or self.group_size == 0 or L["packed"] == 0 or L["raw"]):
                raise ImageError("BadEncoding")
            if L["packed"] != self.num_elements // 2 + self.num_elements % 2:
                raise ImageError("BadTensorShape")
            groups = -(-self.num_elements // self.group_size)
            if L["scales_f32"] and L["scales_f32"] != groups * 4:
                raise ImageError("BadTensorShape")
            if L["scales_f16"] and L["scales_f16"] != groups * 2:
                raise ImageError("BadTensorShape")
            if L["scales_f16_rows4"] and L["scales_f16_rows4"] != groups * 2:
                raise ImageError("BadTensorShape")
            if not (L["scales_f32"] or L["scales_f16"] or L["scales_f16_rows4"]):
                raise ImageError("MissingScales")
            if self.layout == LAYOUT_ROWS4_K16 and (self.out_f % 4 or self.in_f % 16
                                                    or not L["scales_f16_rows4"]):
                raise ImageError("BadPackedLayout")
        else:
            if version != 2 or self.role != ROLE_MLP_GATE_UP_PAIR:
                raise ImageError("BadRole")
            if self.layout != LAYOUT_NONE or self.pair_layout != PAIR_ROWS4_K16:
                raise ImageError("BadPairNibbleLayout")
            if (self.group_size not in (8, 16) or self.out_f % 4 or self.in_f % 16
                    or self.in_f % self.group_size):
                raise ImageError("BadTensorShape")
            if L["raw"] or L["scales_f32"] or L["scales_f16"]:
                raise ImageError("BadEncoding")
            if L["packed"] != self.num_elements:
                raise ImageError("BadTensorShape")
            if L["scales_f16_rows4"] != self.out_f * (self.in_f // self.group_size) * 2 * 2:
                raise ImageError("BadTensorShape")

    def validate_bounds(self, data_offset, file_size, version=2, require_digest=True):
        # runtime_image.zig:543-573
        self.validate_descriptor(version, require_digest)
        for s in STREAMS:
            off, ln = self.rng(s)
            if (off == 0) != (ln == 0):
                raise ImageError("BadBounds")
            if ln == 0:
                continue
            if off < data_offset or off % DATA_ALIGNMENT:
                raise ImageError("BadAlignment")
            if off + ln > file_size:
                raise ImageError("BadBounds")
        live = [self.rng(s) for s in STREAMS if self.rng(s)[1]]
        for i, a in enumerate(live):
            for b in live[i + 1:]:
                if a[0] < b[0] + b[1] and b[0] < a[0] + a[1]:
                    raise ImageError("OverlappingPayload")


def write_image(path, cfg, source_fp, records, abi_fp=None):
    """writeUnpublishedWithProviderV1 (runtime_image.zig:1210-1327): records is
    a list of (Record without ranges, {stream: bytes}); writes a GLRT v2 file
    and returns its bytes."""
    abi_fp = abi_fingerprint(2) if abi_fp is None else abi_fp
    if not records:
        raise ImageError("NoRecords")
    for i, (r, _) in enumerate(records):
        for p, _ in records[:i]:
            if r.layer == p.layer and r.role == p.role and (r.role != ROLE_TENSOR or r.kind == p.kind):
                raise ImageError("DuplicateRecord")
    cursor = align(HEADER_SIZE + len(records) * RECORD_SIZE)
    data_offset = cursor
    plans = []
    for r, payload in records:
        rr = Record(r.layer, r.kind, r.encoding, r.layout, r.group_size, r.out_f, r.in_f,
                    r.num_elements, r.role, r.pair_layout, r.flags)
        for s in STREAMS:
            b = payload.get(s, b"")
            if not b:
                continue
            cursor = align(cursor)
            rr.ranges[s] = (cursor, len(b))
            cursor += len(b)
        plans.append(rr)
    file_size = align(cursor)
    body = bytearray(file_size)
    for rr, (_, payload) in zip(plans, records):
        rr.validate_bounds(data_offset, file_size, 2, False)
        cat = b"".join(payload.get(s, b"") for s in STREAMS)
        rr.crc = crc32(cat)
        rr.digest = hashlib.sha256(rr.encode(2)[:V2_DIGEST_OFFSET] + cat).digest()
        for s in STREAMS:
            if rr.rng(s)[1]:
                off, ln = rr.rng(s)
                body[off:off + ln] = payload[s]
        rr.validate_bounds(data_offset, file_size, 2, True)
    index = b"".join(rr.encode(2) for rr in plans)
    hdr = encode_header(2, len(plans), data_offset, file_size, source_fp, abi_fp, cfg, crc32(index), 0)
    hdr = encode_header(2, len(plans), data_offset, file_size, source_fp, abi_fp, cfg, crc32(index),
                        crc32(hdr))
    body[0:HEADER_SIZE] = hdr
    body[HEADER_SIZE:HEADER_SIZE + len(index)] = index
    data = bytes(body)
    if path is not None:
        with open(path, "wb") as f:
            f.write(data)
    return data


def write_image_v1(path, cfg, source_fp, raw_records):
    """A read-only GLRT v1 image of raw_f32 records (the reference's
    writeLegacyV1RawImage, runtime_image.zig:1496-1540, for any count)."""
    data_offset = align(HEADER_SIZE + len(raw_records) * V1_RECORD_SIZE)
    cursor = data_offset
    recs, body = [], []
    for layer, kind, values in raw_records:
        b = struct.pack(f"<{len(values)}f", *values)
        cursor = align(cursor)
        recs.append((Record(layer, kind, ENC_RAW_F32, LAYOUT_NONE, 0, 1, len(values),
                            ranges={"raw": (cursor, len(b))}, crc=crc32(b)), b))
        cursor += len(b)
    file_size = align(cursor)
    out = bytearray(file_size)
    index = b"".join(r.encode(1) for r, _ in recs)
    hdr = encode_header(1, len(recs), data_offset, file_size, source_fp, abi_fingerprint(1), cfg,
                        crc32(index), 0)
    hdr = encode_header(1, len(recs), data_offset, file_size, source_fp, abi_fingerprint(1), cfg,
                        crc32(index), crc32(hdr))
    out[0:HEADER_SIZE] = hdr
    out[HEADER_SIZE:HEADER_SIZE + len(index)] = index
    for r, b in recs:
        off = r.rng("raw")[0]
        out[off:off + len(b)] = b
    with open(path, "wb") as f:
        f.write(out)
    return bytes(out)


def open_image(data, verify_payload_crc=True, verify_payload_digest=True, allow_v1=True,
               expected_source_fp=None, expected_abi=None, expected_v1_abi=None):
    """MappedImage.openOwnedFileWithOptionsV1: returns (version, header
    fields, records) or raises ImageError with the reference's error name."""
    expected_abi = abi_fingerprint(2) if expected_abi is None else expected_abi
    expected_v1_abi = abi_fingerprint(1) if expected_v1_abi is None else expected_v1_abi
    if len(data) < HEADER_SIZE:
        raise ImageError("TruncatedHeader")
    h = data[:HEADER_SIZE]
    # Header.decode (runtime_image.zig:232-275)
    if h[0:4] != MAGIC:
        raise ImageError("BadMagic")
    version, hsz, rsz, dal, flags = struct.unpack_from("<HHHHI", h, 4)
    if version not in (1, 2):
        raise ImageError("BadVersion")
    if hsz != HEADER_SIZE:
        raise ImageError("BadHeaderSize")
    if rsz != (RECORD_SIZE if version == 2 else V1_RECORD_SIZE):
        raise ImageError("BadRecordSize")
    if dal != DATA_ALIGNMENT:
        raise ImageError("BadAlignment")
    if h[140] > 1:
        raise ImageError("BadConfig")
    if any(h[141:144]) or any(h[160:HEADER_SIZE]):
        raise ImageError("BadReservedField")
    count, index_offset, data_offset, file_size = struct.unpack_from("<QQQQ", h, 16)
    dims = struct.unpack_from("<7I", h, 112)
    eps, theta, index_crc, header_crc = struct.unpack_from("<ffII", h, 144)
    if 0 in dims or not (eps > 0 and eps != float("inf")) or not (theta > 0 and theta != float("inf")):
        raise ImageError("BadConfig")
    # validateHeaderBytes (:1335-1372)
    hb = bytearray(h)
    hb[HEADER_CRC_OFFSET:HEADER_CRC_OFFSET + 4] = b"\0\0\0\0"
    if crc32(bytes(hb)) != header_crc:
        raise ImageError("HeaderCrcMismatch")
    if version == 1 and not allow_v1:
        raise ImageError("LegacyVersionDisabled")
    if flags or count == 0:
        raise ImageError("BadHeader")
    if index_offset != HEADER_SIZE or file_size != len(data):
        raise ImageError("BadBounds")
    index_end = index_offset + count * rsz
    if data_offset < index_end or data_offset % DATA_ALIGNMENT or data_offset > file_size:
        raise ImageError("BadAlignment")
    if expected_source_fp is not None and expected_source_fp != h[48:80]:
        raise ImageError("SourceFingerprintMismatch")
    exp_abi = expected_v1_abi if version == 1 else expected_abi
    if exp_abi is not None and exp_abi != h[80:112]:
        raise ImageError("AbiFingerprintMismatch")
    # validateIndexAndRecords (:1008-1049)
    if index_end > len(data):
        raise ImageError("BadBounds")
    if crc32(data[index_offset:index_end]) != index_crc:
        raise ImageError("IndexCrcMismatch")
    recs = []
    for i in range(count):
        r = Record.decode(data[index_offset + i * rsz:index_offset + (i + 1) * rsz], version)
        r.validate_bounds(data_offset, file_size, version, True)
        for p in recs:
            if r.layer == p.layer and r.role == p.role and (r.role != ROLE_TENSOR or r.kind == p.kind):
                raise ImageError("DuplicateRecord")
            for s in STREAMS:
                a = r.rng(s)
                if not a[1]:
                    continue
                for t in STREAMS:
                    b = p.rng(t)
                    if b[1] and a[0] < b[0] + b[1] and b[0] < a[0] + a[1]:
                        raise ImageError("OverlappingPayload")
        cat = b"".join(data[r.rng(s)[0]:r.rng(s)[0] + r.rng(s)[1]] for s in STREAMS)
        if verify_payload_crc and crc32(cat) != r.crc:
            raise ImageError("CrcMismatch")
        if verify_payload_digest and version == 2:
            if hashlib.sha256(r.encode(2)[:V2_DIGEST_OFFSET] + cat).digest() != r.digest:
                raise ImageError("DigestMismatch")
        recs.append(r)
    return dict(version=version, count=count, data_offset=data_offset, file_size=file_size,
                source_fp=bytes(h[48:80]), abi_fp=bytes(h[80:112]), dims=dims, rms_eps=eps,
                rope_theta=theta, tie=bool(h[140])), recs


def stream(data, r, s):
    off, ln = r.rng(s)
    return data[off:off + ln]


def prepared_record_set(info, recs):
    """validatePreparedConfig + validatePreparedRecordSet (loader.zig:618-716,
    731-768) for the separate gate/up layout; raises the loader's error."""
    dim, hidden, layers, vocab, heads, hd, kvh = info["dims"]
    if heads * hd != dim or kvh > heads or heads % kvh:
        raise ImageError("BadPayload")
    raw_kinds = ("input_norm", "attn_q_bias", "attn_k_bias", "attn_v_bias", "attn_o_bias",
                 "post_attn_norm")
    mat_kinds = ("attn_q", "attn_k", "attn_v", "attn_o", "mlp_gate", "mlp_up", "mlp_down")
    ok_layer = {KIND[k] for k in raw_kinds + mat_kinds}
    for r in recs:
        if r.role == ROLE_MLP_GATE_UP_PAIR:
            if r.layer == GLOBAL_LAYER or r.layer >= layers:
                raise ImageError("BadPayload")
            continue
        if r.layer == GLOBAL_LAYER:
            allowed = {KIND["final_norm"], KIND["embedding"]}
            if not info["tie"]:
                allowed.add(KIND["lm_head"])
            if r.kind not in allowed:
                raise ImageError("BadPayload")
        elif r.layer >= layers or r.kind not in ok_layer:
            raise ImageError("BadPayload")
    return True
