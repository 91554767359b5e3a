"""Builders of prepared runtime images (.glrt) for the tests, written by the
oracle's restatement of the reference writer (oracle/runtime_image.py)."""
import struct

import numpy as np

from oracle import runtime_image as ri


def reference_test_config():
    # runtime_image.zig:1482-1494 (testConfig)
    return ri.Config(dim=16, hidden_dim=32, layers=2, vocab=64, heads=2, head_dim=8, kv_heads=1,
                     rms_eps=1e-6, rope_theta=10000.0, tie_embeddings=True)


def raw_record(layer, kind, values):
    v = np.ascontiguousarray(values, dtype=np.float32)
    return (ri.Record(layer, ri.KIND[kind], ri.ENC_RAW_F32, ri.LAYOUT_NONE, 0, 1, v.size),
            {"raw": v.tobytes()})


def int4_record(layer, kind, packed, out_f, in_f, scales_f32=None, scales_f16=None, group=32,
                layout=ri.LAYOUT_ROW_MAJOR):
    payload = {"packed": np.ascontiguousarray(packed, dtype=np.uint8).tobytes()}
    if scales_f32 is not None:
        payload["scales_f32"] = np.ascontiguousarray(scales_f32, dtype=np.float32).tobytes()
    if scales_f16 is not None:
        payload["scales_f16"] = np.ascontiguousarray(scales_f16, dtype=np.float16).tobytes()
    return ri.Record(layer, ri.KIND[kind], ri.ENC_INT4, layout, group, out_f, in_f), payload


def int4_embedding(gh, cfg, seed):
    """An INT4 token embedding (row-major nibbles, fp16-exact f32 scales) and
    its dequantized f32 rows: NIBBLE_TO_OFFSET[u] * scale
    (int4_matmul.zig:3164-3194)."""
    V, D = cfg["vocab_size"], cfg["dim"]
    packed = gh.synth_int4(seed, 0x454D4245, V * D // 2)
    scales = gh.synth_scales_f16(seed, 0x454D4246, V * D // 32).view(np.float16).astype(np.float32)
    u = np.empty(V * D, np.int32)
    u[0::2] = packed & 15
    u[1::2] = packed >> 4
    table = ((u - 7).astype(np.float32) * np.repeat(scales, 32)).reshape(V, D)
    return packed, scales, table


def model_records(cfg, host, emb_packed, emb_scales, tie=False, f16_mirror=False, biases=False):
    """The prepared record set of loader.zig:193-306 for a host model
    (glacier_hip.random_model_host layout): per layer norms and the seven
    INT4 projections, globals final_norm, embedding (INT4, f32 scales) and
    lm_head unless tied."""
    D, F, V = cfg["dim"], cfg["hidden_dim"], cfg["vocab_size"]
    kvd = cfg["num_kv_heads"] * cfg["head_dim"]
    shapes = dict(q=(D, D), k=(kvd, D), v=(kvd, D), o=(D, D), gate=(F, D), up=(F, D), down=(D, F))
    kinds = dict(q="attn_q", k="attn_k", v="attn_v", o="attn_o", gate="mlp_gate", up="mlp_up",
                 down="mlp_down")
    recs = []
    for l, L in enumerate(host["layers"]):
        recs.append(raw_record(l, "input_norm", L["input_norm"]))
        for name in ("q", "k", "v", "o", "gate", "up", "down"):
            n, k = shapes[name]
            s = L["s_" + name]
            recs.append(int4_record(l, kinds[name], L["w_" + name], n, k, scales_f32=s,
                                    scales_f16=s.astype(np.float16) if f16_mirror else None))
        recs.append(raw_record(l, "post_attn_norm", L["post_attn_norm"]))
        if biases:
            for b, kind in (("bq", "attn_q_bias"), ("bk", "attn_k_bias"), ("bv", "attn_v_bias")):
                recs.append(raw_record(l, kind, L[b]))
    G = ri.GLOBAL_LAYER
    recs.append(raw_record(G, "final_norm", host["final_norm"]))
    recs.append(int4_record(G, "embedding", emb_packed, V, D, scales_f32=emb_scales))
    if not tie:
        recs.append(int4_record(G, "lm_head", host["lm_head"], V, D,
                                scales_f32=host["lm_head_scales"]))
    return recs


def model_config(cfg, tie=False):
    return ri.Config(dim=cfg["dim"], hidden_dim=cfg["hidden_dim"], layers=cfg["num_layers"],
                     vocab=cfg["vocab_size"], heads=cfg["num_heads"], head_dim=cfg["head_dim"],
                     kv_heads=cfg["num_kv_heads"], rms_eps=cfg["rms_eps"],
                     rope_theta=cfg["rope_theta"], tie_embeddings=tie)


def repair_crcs(data, version=2):
    """Recompute the index CRC and then the header CRC of an image whose
    index was edited (the reference test helper repairSingleV2IndexAndHeaderCrc,
    runtime_image.zig:1542-1558, for any record count)."""
    b = bytearray(data)
    count = struct.unpack_from("<Q", b, 16)[0]
    rsz = ri.RECORD_SIZE if version == 2 else ri.V1_RECORD_SIZE
    idx = bytes(b[ri.HEADER_SIZE:ri.HEADER_SIZE + count * rsz])
    struct.pack_into("<I", b, 152, ri.crc32(idx))
    struct.pack_into("<I", b, ri.HEADER_CRC_OFFSET, 0)
    struct.pack_into("<I", b, ri.HEADER_CRC_OFFSET, ri.crc32(bytes(b[:ri.HEADER_SIZE])))
    return bytes(b)
