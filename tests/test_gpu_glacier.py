"""Models loaded from portable .glacier containers onto the GPU
(glacier_hip_model_load_glacier, loader.zig:1214-1592 with compact INT4 and
concatInt4Pages :1636-1720) decode exactly like the same weights set from
host arrays, and like the CPU oracle: identical greedy tokens, logits
bit-identical to the host-set model and within 1e-2 max-relative of the
oracle. A converter-style container (f32 weights quantized page by page by
qio.encodePage) decodes like the oracle model built from the codes and the
fp16-rounded scales the loader uploads. The loader rejects what the
reference rejects and what this device does not run."""
import numpy as np
import pytest

from oracle import glacier_container as gc
import glacier_build as gb

pytestmark = pytest.mark.gpu

TINY = dict(num_layers=2, dim=256, hidden_dim=512, num_heads=4, num_kv_heads=2, head_dim=64,
            vocab_size=4096, group_size=32, rms_eps=1e-6, rope_theta=1e6)
OVERRIDE = dict(num_heads=4, num_kv_heads=2, head_dim=64, rms_eps=1e-6, rope_theta=1e6)
SEED = 0x474C4143


def _host(gh, biases=False):
    host = gh.random_model_host(TINY, SEED)
    for li, L in enumerate(host["layers"]):  # unit-centred norms: varied greedy sequences
        L["input_norm"] = (L["input_norm"] + 1.0).astype(np.float32)
        L["post_attn_norm"] = (L["post_attn_norm"] + 1.0).astype(np.float32)
        if biases:
            kvd = TINY["num_kv_heads"] * TINY["head_dim"]
            L["bq"] = gh.synth_normal_f32(SEED, 0x42510 + 3 * li, TINY["dim"])
            L["bk"] = gh.synth_normal_f32(SEED, 0x42511 + 3 * li, kvd)
            L["bv"] = gh.synth_normal_f32(SEED, 0x42512 + 3 * li, kvd)
    host["final_norm"] = (host["final_norm"] + 1.0).astype(np.float32)
    return host


def _int4_embedding(gh):
    V, D = TINY["vocab_size"], TINY["dim"]
    packed = gh.synth_int4(SEED, 0x454D4245, V * D // 2)
    scales = gh.synth_scales_f16(SEED, 0x454D4246, V * D // 32).view(np.float16).astype(np.float32)
    u = gb.unpack_codes(packed, V * D).astype(np.int32)
    table = ((u - 7).astype(np.float32) * np.repeat(scales, 32)).reshape(-1)
    return packed, scales, table


def _decode(gh, m, prompt, n):
    sess = gh.Session(m, max_lanes=1, max_positions=64)
    try:
        sess.begin(0, seed=3)
        tok, lg0 = sess.prefill(0, prompt, want_logits=True)
        toks, lgs = [tok], [lg0]
        for _ in range(1, n):
            nxt, lg = sess.step([0], [toks[-1]], want_logits=True)
            toks.append(int(nxt[0]))
            lgs.append(lg[0])
        return toks, lgs
    finally:
        sess.close()


def _open(gh, tmp_path, name, pages):
    p = tmp_path / name
    p.write_bytes(gb.container(pages))
    return gh.Glacier(str(p))


@pytest.mark.parametrize("variant", ["plain", "tied", "biases", "small_pages"])
def test_loaded_model_equals_host_model_and_oracle(gh, gctx, ora, tmp_path, variant):
    host = _host(gh, biases=variant == "biases")
    emb = None
    if variant == "tied":
        packed, scales, table = _int4_embedding(gh)
        emb = (packed, scales)
        host["embedding"] = table
        host["lm_head"], host["lm_head_scales"] = packed, scales
    pages = gb.model_pages(TINY, host, emb=emb, tie=variant == "tied", biases=variant == "biases",
                           page_elems=4096 if variant == "small_pages" else gb.PAGE_ELEMS)
    c = _open(gh, tmp_path, f"{variant}.glacier", pages)
    print(f"glacier variant={variant} pages={len(pages)}", flush=True)
    loaded = gh.Model.load_glacier(gctx, c, OVERRIDE, tie_word_embeddings=variant == "tied")
    ref = gh.Model(gctx, TINY)
    ref.set_from_host(host)
    try:
        rep = loaded.report
        assert rep.error == 0 and rep.inexact_scales == 0
        assert rep.int4_tensors == 7 * TINY["num_layers"] + 1
        assert {k: loaded.cfg[k] for k in TINY} == pytest.approx(TINY)
        assert loaded.weight_bytes() == ref.weight_bytes()
        prompt = gh.synth_tokens(SEED, 7, TINY["vocab_size"], 18)
        n = 12
        got, gl = _decode(gh, loaded, prompt, n)
        want, wl = _decode(gh, ref, prompt, n)
        assert got == want
        for a, b in zip(gl, wl):
            assert np.array_equal(a, b)
        otoks, ol, _, _ = ora.OracleModel(TINY, host).generate(prompt, n, logits_steps=[0, n - 1])
        assert got == otoks.tolist()
        for a, b in ((gl[0], ol[0]), (gl[-1], ol[1])):
            assert float(np.max(np.abs(a - b)) / np.max(np.abs(b))) < 1e-2
    finally:
        loaded.close()
        ref.close()
        c.close()


def test_converter_style_container_decodes_like_the_oracle(gh, gctx, ora, tmp_path):
    """f32 projections quantized page by page (qio.encodePage, the spare +8
    code, f32 scales) load with their scales rounded to fp16; the oracle
    model built from the same codes and fp16 scales gives the same tokens."""
    host = _host(gh)
    rng = np.random.default_rng(5)
    D, F = TINY["dim"], TINY["hidden_dim"]
    kvd = TINY["num_kv_heads"] * TINY["head_dim"]
    shapes = dict(q=(D, D), k=(kvd, D), v=(kvd, D), o=(D, D), gate=(F, D), up=(F, D),
                  down=(D, F))
    kinds = dict(q="attn_q", k="attn_k", v="attn_v", o="attn_o", gate="mlp_gate", up="mlp_up",
                 down="mlp_down")
    pages = []
    for li, L in enumerate(host["layers"]):
        pages += gb.raw_pages(li, "input_norm", L["input_norm"])
        pages += gb.raw_pages(li, "post_attn_norm", L["post_attn_norm"], gc.BF16)
        L["post_attn_norm"] = gc._raw_values(pages[-1]["payload"], gc.BF16)
        for name, (n, k) in shapes.items():
            w = (rng.standard_normal(n * k) * 0.05).astype(np.float32)
            qp = gb.quantized_pages(li, kinds[name], w)
            pages += qp
            codes = np.concatenate([gb.unpack_codes(p["payload"][16 + 4 * ((p["row_end"] - p["row_start"]) // 32):],
                                                    p["row_end"] - p["row_start"]) for p in qp])
            s32 = np.concatenate([np.frombuffer(p["payload"], "<f4",
                                                (p["row_end"] - p["row_start"]) // 32, 16)
                                  for p in qp])
            packed = np.zeros(n * k // 2, np.uint8)
            packed |= codes[0::2]
            packed |= (codes[1::2] << 4).astype(np.uint8)
            L["w_" + name] = packed
            L["s_" + name] = s32.astype(np.float16).astype(np.float32)
    pages += gb.raw_pages(0, "final_norm", host["final_norm"], gc.FP16)
    host["final_norm"] = host["final_norm"].astype(np.float16).astype(np.float32)
    pages += gb.raw_pages(0, "embedding", host["embedding"])
    pages += gb.int4_pages(0, "lm_head", host["lm_head"], host["lm_head_scales"],
                           TINY["vocab_size"] * D)
    c = _open(gh, tmp_path, "converted.glacier", pages)
    m = gh.Model.load_glacier(gctx, c, OVERRIDE)
    try:
        assert m.report.inexact_scales > 0  # f32 scales fp16 does not hold
        prompt = gh.synth_tokens(SEED, 9, TINY["vocab_size"], 16)
        n = 10
        got, gl = _decode(gh, m, prompt, n)
        otoks, ol, _, _ = ora.OracleModel(TINY, host).generate(prompt, n, logits_steps=[0])
        assert got == otoks.tolist()
        assert float(np.max(np.abs(gl[0] - ol[0])) / np.max(np.abs(ol[0]))) < 1e-2
    finally:
        m.close()
        c.close()


@pytest.mark.parametrize("case, want", [
    ("missing_lm_head", "MissingTensor"),
    ("missing_post_norm", "MissingTensor"),
    ("o_bias", "Unsupported"),
    ("group16", "Unsupported"),
    ("raw_projection", "Unsupported"),
    ("wrong_heads", "Unsupported"),
    ("short_norm", "BadPayload"),
    ("tied_f32_embedding", "Unsupported"),
])
def test_loader_rejects_like_the_reference(gh, gctx, tmp_path, case, want):
    host = _host(gh)
    D = TINY["dim"]
    pages = gb.model_pages(TINY, host)
    override, tie = dict(OVERRIDE), False
    drop = None
    extra = []
    if case == "missing_lm_head":
        drop = (0, gb.KIND["lm_head"])
    elif case == "missing_post_norm":
        drop = (1, gb.KIND["post_attn_norm"])
    elif case == "o_bias":
        extra = gb.raw_pages(0, "attn_o_bias", np.zeros(D))
    elif case == "group16":
        L = host["layers"][0]
        drop = (0, gb.KIND["attn_o"])
        extra = gb.int4_pages(0, "attn_o", L["w_o"], np.repeat(L["s_o"], 2), D * D, group=16)
    elif case == "raw_projection":
        drop = (0, gb.KIND["attn_o"])
        extra = gb.raw_pages(0, "attn_o", np.zeros(D * D), gc.FP16)
    elif case == "wrong_heads":
        override["num_heads"] = 3
    elif case == "short_norm":
        drop = (0, gb.KIND["input_norm"])
        extra = gb.raw_pages(0, "input_norm", np.ones(D // 2))
    elif case == "tied_f32_embedding":
        tie = True
    if drop is not None:
        pages = [p for p in pages if (p["layer"], p["kind"]) != drop]
    c = _open(gh, tmp_path, f"{case}.glacier", pages + extra)
    try:
        with pytest.raises(gh.GlacierError) as e:
            gh.Model.load_glacier(gctx, c, override, tie_word_embeddings=tie)
        assert e.value.reason == want
    finally:
        c.close()
