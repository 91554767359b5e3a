"""Builders of portable .glacier containers for the tests (the converter's
output shape, src/model/converter.zig, written with the oracle's container
writer): each tensor is cut into pages of at most 65536 elements (the v1
quantized window, format.zig:310-313) on quantization-group boundaries, a
quantized page carries its qio sub-header, f32 scales and packed codes
(qio.zig:1-21), raw pages hold f32 / fp16 / bf16 bytes."""
import json
import struct

import numpy as np

from oracle import glacier_container as gc

KIND = dict(embedding=0, attn_q=1, attn_k=2, attn_v=3, attn_o=4, mlp_up=5, mlp_down=6,
            mlp_gate=7, input_norm=8, lm_head=9, final_norm=10, post_attn_norm=11,
            attn_q_bias=12, attn_k_bias=13, attn_v_bias=14, attn_o_bias=15, other=255)
PAGE_ELEMS = 65536


def int4_payload(packed_codes, scales, n, group):
    """A QOIT INT4 payload from element codes u (0..15) and f32 scales."""
    u = np.asarray(packed_codes, np.uint8)
    out = np.zeros((n + 1) // 2, np.uint8)
    out[: (n + 1) // 2] |= u[0::2]
    out[: n // 2] |= (u[1::2] << 4).astype(np.uint8)
    return (struct.pack("<IIIB3x", gc.QIO_MAGIC, n, group, gc.Q_INT4) +
            np.asarray(scales, "<f4").tobytes() + out.tobytes())


def unpack_codes(packed, n):
    p = np.frombuffer(packed, np.uint8) if isinstance(packed, bytes) else np.asarray(packed, np.uint8)
    u = np.empty(n, np.uint8)
    u[0::2] = (p & 15)[: (n + 1) // 2]
    u[1::2] = (p >> 4)[: n // 2]
    return u


def int4_pages(layer, kind, packed, scales, n, group=32, page_elems=PAGE_ELEMS):
    """Pages of one INT4 tensor given as packed nibbles + one f32 scale per group."""
    u = unpack_codes(packed, n)
    scales = np.asarray(scales, np.float32)
    step = page_elems - page_elems % group
    pages = []
    for s in range(0, n, step):
        e = min(n, s + step)
        pages.append(dict(layer=layer, kind=KIND[kind], row_start=s, row_end=e,
                          precision=gc.INT4, quant_group=group,
                          payload=int4_payload(u[s:e], scales[s // group:-(-e // group)], e - s,
                                               group)))
    return pages


def quantized_pages(layer, kind, values, precision=gc.Q_INT4, group=32, page_elems=PAGE_ELEMS):
    """Pages of an f32 tensor quantized page by page with qio.encodePage."""
    v = np.asarray(values, np.float32).reshape(-1)
    step = page_elems - page_elems % group
    prec = gc.INT4 if precision == gc.Q_INT4 else gc.INT8
    return [dict(layer=layer, kind=KIND[kind], row_start=s, row_end=min(v.size, s + step),
                 precision=prec, quant_group=group,
                 payload=gc.encode_page(v[s:s + step], precision, group))
            for s in range(0, v.size, step)]


def raw_pages(layer, kind, values, precision=gc.FP32):
    v = np.asarray(values, np.float32).reshape(-1)
    width = 4 if precision == gc.FP32 else 2
    step = gc.PAGE_SIZE_BYTES // width
    pages = []
    for s in range(0, v.size, step):
        part = v[s:s + step]
        if precision == gc.FP32:
            b = part.astype("<f4").tobytes()
        elif precision == gc.FP16:
            b = part.astype("<f2").tobytes()
        else:
            b = (part.astype("<f4").view("<u4") >> 16).astype("<u2").tobytes()
        pages.append(dict(layer=layer, kind=KIND[kind], row_start=s, row_end=s + part.size,
                          precision=precision, quant_group=0, payload=b))
    return pages


def model_pages(cfg, host, emb=None, tie=False, biases=False, page_elems=PAGE_ELEMS):
    """Pages of a host model (glacier_hip.random_model_host layout): per layer
    norms (f32) and the seven INT4 projections, globals at layer 0: final
    norm, the embedding (INT4 (packed, scales) when `emb` is given, else the
    f32 table) and the LM head unless tied."""
    D, F, V = cfg["dim"], cfg["hidden_dim"], cfg["vocab_size"]
    kvd = cfg["num_kv_heads"] * cfg["head_dim"]
    shapes = dict(q=(D, D), k=(kvd, D), v=(kvd, D), o=(D, D), gate=(F, D), up=(F, D), down=(D, F))
    kinds = dict(q="attn_q", k="attn_k", v="attn_v", o="attn_o", gate="mlp_gate", up="mlp_up",
                 down="mlp_down")
    pages = []
    for li, L in enumerate(host["layers"]):
        pages += raw_pages(li, "input_norm", L["input_norm"])
        for name in ("q", "k", "v", "o", "gate", "up", "down"):
            n, k = shapes[name]
            pages += int4_pages(li, kinds[name], L["w_" + name], L["s_" + name], n * k,
                                page_elems=page_elems)
        if biases:
            for b in ("bq", "bk", "bv"):
                pages += raw_pages(li, "attn_%s_bias" % b[1], L[b])
        pages += raw_pages(li, "post_attn_norm", L["post_attn_norm"])
    pages += raw_pages(0, "final_norm", host["final_norm"])
    if emb is not None:
        pages += int4_pages(0, "embedding", emb[0], emb[1], V * D, page_elems=page_elems)
    else:
        pages += raw_pages(0, "embedding", host["embedding"])
    if not tie:
        pages += int4_pages(0, "lm_head", host["lm_head"], host["lm_head_scales"], V * D,
                            page_elems=page_elems)
    return pages


def container(pages, meta=None):
    m = json.dumps(meta if meta is not None else {"format": "glacier-hip-test"}).encode()
    return gc.build_container(m, pages)
