"""Pins the CPU oracle against the reference's own known-answer tests and
against closed forms / brute force, so that a plausible mistake in the
restatement (a swapped nibble, a wrong offset, a dropped term) fails here.
Runs on the CPU only."""
import hashlib
import math
import struct

import numpy as np
import pytest


# ---- a1: INT4 code ---------------------------------------------------------------
def test_int4_zero_midpoint_kat(ora):
    # quant.zig:223-236: four zeros in g4 pack to 0x77 0x77
    rc, packed, scales = ora.int4_quantize(np.zeros(4), 4)
    assert rc == 0 and packed.tolist() == [0x77, 0x77]


def test_int4_group16_full_positive_code_kat(ora):
    # quant.zig:238-256: g16 uses +8 (byte 0x7f, scale 0.125); g8 stays 0x7e
    src = np.zeros(16, np.float32)
    src[0] = 1
    rc, packed, scales = ora.int4_quantize(src, 16)
    assert packed[0] == 0x7F and scales[0] == np.float32(0.125)
    rc, packed, _ = ora.int4_quantize(src[:8], 8)
    assert packed[0] == 0x7E


def test_int4_nibble_order_kat(ora):
    # int4_weights.zig:449-461: bytes 0x80, 0x0f decode to -7, 1, 8, -7
    rc, out = ora.int4_dequantize(np.array([0x80, 0x0F], np.uint8), np.ones(1, np.float32), 4, 4)
    assert rc == 0 and out.tolist() == [-7, 1, 8, -7]


def test_int4_zero_tensor_and_independent_groups(ora):
    rc, packed, scales = ora.int4_quantize(np.zeros(8), 4)
    assert scales.tolist() == [0, 0]
    src = np.concatenate([np.arange(8) * 0.001, np.arange(8) * 10.0]).astype(np.float32)
    rc, packed, scales = ora.int4_quantize(src, 8)
    assert scales[0] < scales[1] / 1000


def test_int4_round_trip_bound(ora):
    rng = np.random.default_rng(42)
    src = ((rng.random(256) * 2 - 1) * 0.1).astype(np.float32)
    rc, packed, scales = ora.int4_quantize(src, 64)
    rc, back = ora.int4_dequantize(packed, scales, 64, src.size)
    assert np.max(np.abs(src - back)) < 0.02


def test_int4_dequant_rejects_truncation(ora):
    rc, _ = ora.int4_dequantize(np.zeros(1, np.uint8), np.ones(1, np.float32), 4, 4)
    assert rc == ora.TRUNCATED


def test_f16_conversion_matches_ieee(ora):
    rng = np.random.default_rng(3)
    vals = np.concatenate([rng.standard_normal(4000) * 10 ** rng.uniform(-9, 5, 4000),
                           [0.0, -0.0, 65504.0, 65520.0, 1e-8, 6e-8, 3e-5]]).astype(np.float32)
    for v in vals:
        want = np.array([v], np.float32).astype(np.float16).view(np.uint16)[0]
        assert ora.lib().go_f32_to_f16(float(v)) == want, v
        assert ora.lib().go_f16_to_f32(int(want)) == np.float32(np.uint16(want).view(np.float16))


# ---- a2/a3: GEMV ----------------------------------------------------------------
def _dequant_rows(packed, scales, out_f, in_f, group):
    u = np.empty(out_f * in_f, np.int64)
    u[0::2] = packed & 0xF
    u[1::2] = packed >> 4
    n = out_f * in_f
    w = (u - 7).astype(np.float64) * np.repeat(scales.astype(np.float64), group)[:n]
    return w.reshape(out_f, in_f)


@pytest.mark.parametrize("out_f,in_f,group", [(8, 64, 64), (9, 64, 32), (16, 256, 32)])
def test_linear_f32_matches_dequant_dot(ora, out_f, in_f, group):
    # int4_matmul.zig:3254-3298 on-the-fly vs full dequant, 2e-6 abs
    rng = np.random.default_rng(42)
    w = ((rng.random(out_f * in_f) * 2 - 1) * 0.1).astype(np.float32)
    rc, packed, scales = ora.int4_quantize(w, group)
    x = (rng.random(in_f) * 2 - 1).astype(np.float32)
    got = ora.linear_int4_f32(x, packed, scales, out_f, in_f, group)[0]
    want = _dequant_rows(packed, scales, out_f, in_f, group) @ x.astype(np.float64)
    assert np.max(np.abs(got - want)) < 2e-6


def test_linear_f32_generic_path_crosses_groups(ora):
    # int4_matmul.zig:3300-3324: in_f 18, group 10, x = 1.25
    w = ((np.arange(54) % 17) - 8).astype(np.float32) / 13.0
    rc, packed, scales = ora.int4_quantize(w, 10)
    x = np.full(18, 1.25, np.float32)
    got = ora.linear_int4_f32(x, packed, scales, 3, 18, 10)[0]
    want = _dequant_rows(packed, scales, 3, 18, 10) @ x.astype(np.float64)
    assert np.max(np.abs(got - want)) < 2e-6


def test_linear_f32_bias(ora):
    rng = np.random.default_rng(5)
    packed = rng.integers(0, 256, 16 * 64 // 2, dtype=np.uint8)
    scales = np.full(16 * 64 // 32, 0.5, np.float32)
    x = rng.standard_normal(64).astype(np.float32)
    b = np.arange(16, dtype=np.float32)
    y0 = ora.linear_int4_f32(x, packed, scales, 16, 64, 32)[0]
    y1 = ora.linear_int4_f32(x, packed, scales, 16, 64, 32, bias=b)[0]
    assert np.allclose(y1 - y0, b, atol=1e-5)


def test_q8_quantize_closed_form(ora):
    x = np.array([0.5, -1.0, 0.25, 0.0] * 8 + [0.0] * 32, np.float32)
    q, s = ora.q8_quantize(x, 32)
    assert s[0] == np.float32(1.0) / np.float32(127.0) and s[1] == 0
    # round half away from zero on x * (1 / s)
    inv = np.float32(1.0) / s[0]
    exp = [int(math.copysign(math.floor(abs(float(np.float32(v) * inv)) + 0.5), v)) for v in x[:32]]
    assert q[:32].tolist() == exp and not q[32:].any()


def test_q8_gemv_exact_group_dots(ora):
    # int4_matmul.zig:365-418: exact integer dot per group, f32 across groups
    rng = np.random.default_rng(7)
    out_f, in_f = 32, 256
    packed = rng.integers(0, 256, out_f * in_f // 2, dtype=np.uint8)
    scales = (np.abs(rng.standard_normal(out_f * in_f // 32)) * 0.02).astype(np.float32)
    x = rng.standard_normal(in_f).astype(np.float32)
    got = ora.linear_int4_q8(x, packed, scales, out_f, in_f, 32)[0]
    q, s = ora.q8_quantize(x, 32)
    u = np.empty(out_f * in_f, np.int64)
    u[0::2] = packed & 0xF
    u[1::2] = packed >> 4
    dots = ((u.reshape(out_f, 8, 32) - 7) * q.astype(np.int64).reshape(1, 8, 32)).sum(-1)
    want = np.zeros(out_f, np.float32)
    for g in range(8):  # sequential f32 accumulation in group order
        t = dots[:, g].astype(np.float32) * scales.reshape(out_f, 8)[:, g]
        t = t * s[g]
        want = want + t
    assert np.array_equal(got, want)


def test_q8_close_to_f32_reference(ora):
    # int4_matmul.zig:3375-3423 (0.08 abs on closed-form inputs)
    src = (((np.arange(64 * 12) * 17) % 31) - 15).astype(np.float32) / 23.0
    x = (((np.arange(64) * 7) % 19) - 9).astype(np.float32) / 11.0
    rc, packed, scales = ora.int4_quantize(src, 32)
    a = ora.linear_int4_q8(x, packed, scales, 12, 64, 32)[0]
    b = _dequant_rows(packed, scales, 12, 64, 32) @ x.astype(np.float64)
    assert np.max(np.abs(a - b)) < 0.08


def test_x86_dispatch_head_and_wide_input_take_f32(ora):
    rng = np.random.default_rng(9)
    x = rng.standard_normal(128).astype(np.float32)
    packed = rng.integers(0, 256, 65552 * 128 // 2, dtype=np.uint8)
    scales = np.full(65552 * 128 // 32, 0.01, np.float32)
    out = np.zeros(65552, np.float32)
    lib = ora.lib()
    rc = lib.go_linear_int4_weight_q8(x.ctypes.data, 1, packed.ctypes.data, scales.ctypes.data,
                                      None, out.ctypes.data, 65552, 128, 32)
    assert rc == 0
    assert np.array_equal(out, ora.linear_int4_f32(x, packed, scales, 65552, 128, 32)[0])


# ---- a5/a8 ---------------------------------------------------------------------------
def test_rmsnorm_kat(ora):
    # kernels.zig:1075-1088
    out = ora.rmsnorm(np.array([[3, 4]], np.float32), np.ones(2, np.float32), 1e-6)
    r = math.sqrt(12.5 + 1e-6)
    assert abs(out[0, 0] - 3 / r) < 1e-5 and abs(out[0, 1] - 4 / r) < 1e-5


def test_rmsnorm_closed_form(ora):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 896)).astype(np.float32)
    w = rng.standard_normal(896).astype(np.float32)
    got = ora.rmsnorm(x, w, 1e-6)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + 1e-6) * w
    assert np.max(np.abs(got - want) / (np.abs(want) + 1e-3)) < 1e-5


def test_silu_mul_closed_form(ora):
    g = np.linspace(-8, 8, 101).astype(np.float32)
    u = np.linspace(2, -2, 101).astype(np.float32)
    got = ora.silu_mul(g, u)
    want = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.max(np.abs(got - want)) < 1e-5


# ---- a6 RoPE ----------------------------------------------------------------------------
def test_rope_known_answers(ora):
    # forward.zig:1265-1287
    row = ora.rope_apply_direct(np.array([1, 0, 0, 0], np.float32), 1, 1, 4, 10000.0)
    assert abs(row[0] - math.cos(1.0)) < 1e-5 and abs(row[2] - math.sin(1.0)) < 1e-5
    row = ora.rope_apply_direct(np.array([3, 7, -2, 5], np.float32), 0, 1, 4, 10000.0)
    assert row.tolist() == [3, 7, -2, 5]


def test_rope_table_matches_direct_formula(ora):
    # generate.zig:5616-5628
    x = np.array([0.25, -0.5, 0.75, -1.0, 1.25, -1.5, 1.75, -2.0, 2.25, -2.5, 2.75, -3.0,
                  3.25, -3.5, 3.75, -4.0], np.float32)
    cs, sn = ora.rope_table(8, 8, 10000.0)
    want = ora.rope_apply_direct(x, 3, 2, 8, 10000.0)
    got = x.copy()
    ora.lib().go_rope_apply(cs.ctypes.data, sn.ctypes.data, 4, got.ctypes.data, 3, 2, 8)
    assert np.max(np.abs(want - got)) < 1e-6


def test_rope_table_closed_form(ora):
    cs, sn = ora.rope_table(64, 64, 1e6)
    pos = np.arange(64)[:, None].astype(np.float64)
    freq = 1.0 / (1e6 ** (np.arange(32) * 2 / 64.0))
    assert np.max(np.abs(cs.reshape(64, 32) - np.cos(pos * freq))) < 2e-5
    assert np.max(np.abs(sn.reshape(64, 32) - np.sin(pos * freq))) < 2e-5


# ---- a7 attention -------------------------------------------------------------------
def _closed_form_kv(seq, kv_dim, q_seq, q_dim):
    # paged_attention.zig:258-263
    k = ((np.arange(seq * kv_dim) % 29) * 0.03125 - 0.4).astype(np.float32)
    v = ((np.arange(seq * kv_dim) % 31) * -0.0234375 + 0.3).astype(np.float32)
    q = ((np.arange(q_seq * q_dim) % 17) * 0.046875 - 0.2).astype(np.float32)
    return q, k, v


def _pool_from_rows(k, v, seq, kv_dim, num_layers=1, layer=0, fp16=False, seed=0):
    pages = -(-seq // 16)
    rng = np.random.default_rng(seed)
    phys = rng.permutation(pages + 3)[:pages].astype(np.int32)
    dt = np.float16 if fp16 else np.float32
    pool = np.zeros((pages + 3, num_layers, 2, 16, kv_dim), dt)
    for j in range(seq):
        pool[phys[j // 16], layer, 0, j % 16] = k[j * kv_dim:(j + 1) * kv_dim]
        pool[phys[j // 16], layer, 1, j % 16] = v[j * kv_dim:(j + 1) * kv_dim]
    return pool, phys


@pytest.mark.parametrize("seq", [1, 15, 16, 17, 31, 32])
@pytest.mark.parametrize("heads", [(4, 2, 8), (3, 3, 5)])
def test_paged_attention_byte_identical(ora, seq, heads):
    # paged_attention.zig:317-324
    Hq, Hkv, hd = heads
    q, k, v = _closed_form_kv(seq, Hkv * hd, 1, Hq * hd)
    want = ora.attention(q, k, v, Hq, Hkv, hd)
    pool, pt = _pool_from_rows(k, v, seq, Hkv * hd)
    got = ora.attention_paged(q, pool, False, pt, seq, 0, 1, Hq, Hkv, hd)
    assert want.tobytes() == got.tobytes()


def test_attention_causal_multi_query_and_textbook(ora):
    Hq, Hkv, hd, seq, q_seq = 4, 2, 8, 17, 3
    q, k, v = _closed_form_kv(seq, Hkv * hd, q_seq, Hq * hd)
    got = ora.attention(q, k, v, Hq, Hkv, hd)
    K = k.reshape(seq, Hkv, hd).astype(np.float64)
    V = v.reshape(seq, Hkv, hd).astype(np.float64)
    Q = q.reshape(q_seq, Hq, hd).astype(np.float64)
    want = np.zeros((q_seq, Hq, hd))
    for i in range(q_seq):
        upto = seq - q_seq + i
        for h in range(Hq):
            s = K[:upto + 1, h // 2] @ Q[i, h] / math.sqrt(hd)
            p = np.exp(s - s.max())
            want[i, h] = (p / p.sum()) @ V[:upto + 1, h // 2]
    assert np.max(np.abs(got.reshape(q_seq, Hq, hd) - want)) < 1e-6


def test_paged_attention_fp16_pool_equals_widened_contiguous(ora):
    Hq, Hkv, hd, seq = 8, 2, 64, 40
    rng = np.random.default_rng(11)
    q = rng.standard_normal(Hq * hd).astype(np.float32)
    k = rng.standard_normal(seq * Hkv * hd).astype(np.float32).astype(np.float16).astype(np.float32)
    v = rng.standard_normal(seq * Hkv * hd).astype(np.float32).astype(np.float16).astype(np.float32)
    pool, pt = _pool_from_rows(k, v, seq, Hkv * hd, num_layers=3, layer=1, fp16=True)
    got = ora.attention_paged(q, pool.view(np.uint16), True, pt, seq, 1, 3, Hq, Hkv, hd)
    want = ora.attention(q, k, v, Hq, Hkv, hd)
    assert want.tobytes() == got.tobytes()


# ---- a12/a13 argmax ---------------------------------------------------------------
def test_argmax_first_max_and_nan_rules(ora):
    assert ora.argmax([1, 5, 2, 4]) == 1  # sampling.zig:216-223
    assert ora.argmax([5, 1, 5]) == 0
    assert ora.argmax([np.nan, 9, 3]) == 0
    assert ora.argmax([1, np.nan, 3]) == 2
    assert ora.argmax([-np.inf, -np.inf]) == 0


def test_eligible_argmax_mask_geometry(ora):
    # sampling.zig:225-251
    z = np.zeros(65, np.float32)
    for words in ([], [1], [1, 0, 0], [0, 0], [1, 0b10]):
        rc, _, _ = ora.argmax_eligible(z, np.array(words, np.uint64))
        assert rc == ora.INVALID_MASK, words
    rc, _, _ = ora.argmax_eligible(np.zeros(0, np.float32), np.zeros(0, np.uint64))
    assert rc == ora.INVALID_MASK


def test_eligible_argmax_known_answers(ora):
    # sampling.zig:253-286
    logits = np.full(130, -100, np.float32)
    logits[0] = np.nan
    logits[5], logits[67], logits[129] = 3.0, 9.0, 8.0
    rc, idx, rows = ora.argmax_eligible(logits, np.array([1 << 5, 1 << 3, 1 << 1], np.uint64))
    assert (rc, idx, rows) == (0, 67, 3)
    rc, _, _ = ora.argmax_eligible(np.array([10, np.nan, 20], np.float32), np.array([0b110], np.uint64))
    assert rc == ora.ELIGIBLE_NAN
    pos = np.array([0, np.inf, 7, np.inf], np.float32)
    assert ora.argmax_eligible(pos, np.array([0b1010], np.uint64))[1] == 1
    neg = np.array([0, -np.inf, 7, -np.inf], np.float32)
    assert ora.argmax_eligible(neg, np.array([0b1010], np.uint64))[1] == 1
    fin = np.array([5, 0, 5, 0], np.float32)
    assert ora.argmax_eligible(fin, np.array([0b0101], np.uint64))[1] == 0


def test_eligible_argmax_brute_force(ora):
    rng = np.random.default_rng(4)
    for trial in range(50):
        n = int(rng.integers(1, 300))
        logits = rng.integers(-3, 4, n).astype(np.float32)
        bits = rng.random(n) < 0.3
        if not bits.any():
            bits[0] = True
        words = np.zeros(-(-n // 64), np.uint64)
        for i in np.nonzero(bits)[0]:
            words[i // 64] |= np.uint64(1) << np.uint64(i % 64)
        rc, idx, rows = ora.argmax_eligible(logits, words)
        elig = np.nonzero(bits)[0]
        best = elig[np.argmax(logits[elig])]
        assert rc == 0 and idx == best and rows == bits.sum()


# ---- a15/a16 paged KV digests and ledgers -------------------------------------------------
def test_capacity_ledger_known_answers(ora):
    # paged_kv_cache.zig:1564-1588
    rc, s = ora.capacity_ledger(24, 128, 128)
    assert rc == 0
    assert (s["page_count_capacity"], s["page_payload_bytes"], s["tensor_capacity_bytes"],
            s["page_map_bytes"], s["allocation_capacity_bytes"],
            s["contiguous_counterfactual_bytes"], s["capacity_reclaimed_bytes"],
            s["capacity_overhead_bytes"], s["padded_positions"]) == (
        8, 393_216, 3_145_728, 128, 3_145_856, 3_146_496, 640, 0, 0)
    rc, l = ora.capacity_ledger(24, 128, 512)
    assert (l["page_count_capacity"], l["page_map_bytes"], l["allocation_capacity_bytes"],
            l["contiguous_counterfactual_bytes"], l["capacity_reclaimed_bytes"]) == (
        32, 512, 12_583_424, 12_583_680, 256)
    rc, p = ora.capacity_ledger(24, 128, 129)
    assert p["padded_positions"] == 15 and p["capacity_overhead_bytes"] > 0
    assert p["capacity_reclaimed_bytes"] == 0
    assert ora.capacity_ledger(0, 128, 128)[0] == ora.SHAPE_MISMATCH


def test_sha256_nist_vectors(ora):
    assert ora.sha256(b"abc").hex() == \
        "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"
    assert ora.sha256(b"").hex() == \
        "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"
    blob = bytes(range(256)) * 5
    assert ora.sha256(blob) == hashlib.sha256(blob).digest()


def test_ownership_digest_formulas(ora):
    # paged_kv_cache.zig:323-353 restated from the field order with hashlib
    want = hashlib.sha256(b"glacier-paged-kv-ownership-v1\x00" +
                          struct.pack("<5Q", 7, 24, 128, 256, 16)).digest()
    e = ora.empty_ownership_digest(7, 24, 128, 256)
    assert e == want
    want2 = hashlib.sha256(b"glacier-paged-kv-root-append-v1\x00" + e +
                           struct.pack("<4Q", 0x4750524600000001, 7, 3, 9)).digest()
    assert ora.append_ownership_digest(e, 7, 3, 9) == want2
    t = ora.token_sequence_sha256([1, 2, 3])
    assert t == hashlib.sha256(b"glacier-output-token-state-v1\x00" +
                               struct.pack("<Q3I", 3, 1, 2, 3)).digest()


def test_xoshiro_seeding_splitmix_known_answer(ora):
    # SplitMix64 with seed 0: first output 0xe220a8397b1dcdaf (published sequence)
    assert ora.xoshiro256_init(0)[0] == 0xE220A8397B1DCDAF


# ---- a9: the layer composition ------------------------------------------------------
def test_forward_layer_f32_matches_reference_layer_composition(ora):
    """go_forward_layer in the reference's int4_activation = .f32 mode against
    tests/golden/layer_qwen05b.npz: one Qwen2.5-0.5B-shaped layer over 8
    positions composed by tests/golden/make_layer_golden.py from the
    reference's own rmsnorm / rope / softmax / silu
    (tools/reference_layer0.py, composition of its main() :107-170) on the
    dequantized weights. Pins RoPE before the KV append, GQA h // group, the
    q/k/v biases, both residuals, the post-attention norm and SiLU(gate) * up.
    Bar 1e-5 max-relative (f32 against f32, different summation order)."""
    import os
    import sys

    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
    import layer_case

    layer, _, x = layer_case.make()
    cfg = layer_case.CFG
    D, V = cfg["dim"], cfg["vocab_size"]
    host = dict(layers=[layer], embedding=np.zeros((V, D), np.float32),
                final_norm=np.ones(D, np.float32),
                lm_head=np.full(V * D // 2, 0x77, np.uint8),
                lm_head_scales=np.zeros(V * D // 32, np.float32))
    fx = np.load(os.path.join(os.path.dirname(__file__), "golden", "layer_qwen05b.npz"))
    assert int(fx["seed"]) == layer_case.SEED and int(fx["T"]) == layer_case.T
    om = ora.OracleModel(cfg, host, act_f32=True)
    got = om.forward_layer(0, x)
    rel = float(np.max(np.abs(got - fx["out"])) / np.max(np.abs(fx["out"])))
    assert rel < 1e-5, rel
    # the default .q8 mode stays close (Q8 activations, int4_matmul.zig:3375)
    q8 = ora.OracleModel(cfg, host).forward_layer(0, x)
    rel_q8 = float(np.max(np.abs(q8 - fx["out"])) / np.max(np.abs(fx["out"])))
    assert 1e-5 < rel_q8 < 5e-2, rel_q8


def _q8_brute(x, packed, scales, out_f, in_f):
    """Closed form of linearInt4Q8OnTheFly (int4_matmul.zig:365-418): per
    32-group s = max|x|/127, q = clamp(round_half_away(x * (1/s)), +-127), exact
    integer group dots, acc += (f32(dot) * w_scale) * s in group order."""
    x = x.astype(np.float32)
    G = in_f // 32
    xs = x.reshape(G, 32)
    s = (np.max(np.abs(xs), axis=1) / np.float32(127)).astype(np.float32)
    inv = np.where(s > 0, np.float32(1) / np.where(s > 0, s, 1), 0).astype(np.float32)
    v = (xs * inv[:, None]).astype(np.float32)
    q = np.clip(np.sign(v) * np.floor(np.abs(v) + np.float32(0.5)), -127, 127).astype(np.int64)
    codes = np.empty(out_f * in_f, np.int64)
    codes[0::2] = packed & 0xF
    codes[1::2] = packed >> 4
    w = (codes - 7).reshape(out_f, G, 32)
    dots = np.einsum("ogk,gk->og", w, q)
    ws = scales.reshape(out_f, G).astype(np.float32)
    acc = np.zeros(out_f, np.float32)
    for g in range(G):
        t = (dots[:, g].astype(np.float32) * ws[:, g]).astype(np.float32)
        acc = (acc + (t * s[g]).astype(np.float32)).astype(np.float32)
    return acc


@pytest.mark.parametrize("in_f", [16384, 16416])
def test_q8_wide_input_fallback_boundary(ora, in_f):
    """int4_matmul.zig:372-374: Q8 activations up to in_f = 16384 (512 groups
    of 32); past it the exact f32 path (linearInt4OnTheFly)."""
    rng = np.random.default_rng(in_f)
    out_f = 16
    x = rng.standard_normal(in_f).astype(np.float32)
    packed = rng.integers(0, 256, out_f * in_f // 2, dtype=np.uint8)
    scales = np.abs(rng.normal(0, 0.02, out_f * in_f // 32)).astype(np.float16).astype(np.float32)
    got = ora.linear_int4_q8(x, packed, scales, out_f, in_f, 32)[0]
    f32 = ora.linear_int4_f32(x, packed, scales, out_f, in_f, 32)[0]
    if in_f > 16384:
        assert np.array_equal(got, f32)
    else:
        assert np.array_equal(got, _q8_brute(x, packed, scales, out_f, in_f))
        assert not np.array_equal(got, f32)
