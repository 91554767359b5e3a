"""Models loaded from prepared runtime images (.glrt) onto the GPU
(glacier_hip_model_load_glrt, loader.zig:193-390) decode exactly like the
same weights set from host arrays, and like the CPU oracle: identical greedy
tokens, logits bit-identical to the host-set model and within 1e-2
max-relative of the oracle. The loader's record-set rules reject what the
reference rejects and what this device does not run."""
import numpy as np
import pytest

from oracle import runtime_image as ri
from glrt_images import (int4_embedding, int4_record, model_config, model_records, raw_record)

pytestmark = pytest.mark.gpu

TINY = dict(num_layers=2, dim=256, hidden_dim=512, num_heads=4, num_kv_heads=2, head_dim=64,
            vocab_size=4096, group_size=32, rms_eps=1e-6, rope_theta=1e6)
SEED = 0x474C5254


def _host(gh, tie=False, biases=False):
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
    packed, scales, table = int4_embedding(gh, TINY, SEED)
    host["embedding"] = np.ascontiguousarray(table.reshape(-1))
    if tie:
        host["lm_head"], host["lm_head_scales"] = packed, scales
    return host, packed, scales


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


def _write(tmp_path, name, host, packed, scales, **kw):
    tie = kw.pop("tie", False)
    extra = kw.pop("extra", [])
    drop = kw.pop("drop", None)
    recs = model_records(TINY, host, packed, scales, tie=tie, **kw)
    if drop is not None:
        recs = [r for r in recs if (r[0].layer, r[0].kind) != drop]
    p = tmp_path / name
    ri.write_image(str(p), model_config(TINY, tie), ri.fingerprint(name.encode()), recs + extra)
    return p


@pytest.mark.parametrize("variant", ["plain", "f16_mirror", "tied", "biases"])
def test_loaded_model_equals_host_model_and_oracle(gh, gctx, ora, tmp_path, variant):
    host, packed, scales = _host(gh, tie=variant == "tied", biases=variant == "biases")
    p = _write(tmp_path, f"{variant}.glrt", host, packed, scales, tie=variant == "tied",
               f16_mirror=variant == "f16_mirror", biases=variant == "biases")
    img = gh.GlrtImage(str(p))
    print(f"glrt variant={variant} bytes={img.info.file_size}", flush=True)
    loaded = gh.Model.load_glrt(gctx, img)
    ref = gh.Model(gctx, TINY)
    ref.set_from_host(host)
    try:
        rep = loaded.report
        assert rep.error == 0 and rep.separate_mlp == 1 and rep.inexact_scales == 0
        assert rep.int4_records == 7 * TINY["num_layers"] + (1 if variant == "tied" else 2)
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
        img.close()


def test_f32_scales_outside_fp16_are_counted(gh, gctx, tmp_path):
    host, packed, scales = _host(gh)
    s = host["layers"][1]["s_gate"].copy()
    s[:5] = s[:5] * np.float32(1.0 + 2.0 ** -13)  # between fp16 neighbours
    host["layers"][1]["s_gate"] = s
    p = _write(tmp_path, "inexact.glrt", host, packed, scales)
    img = gh.GlrtImage(str(p))
    m = gh.Model.load_glrt(gctx, img)
    try:
        assert m.report.inexact_scales == int(np.sum(s.astype(np.float16).astype(np.float32) != s))
        assert m.report.inexact_scales >= 1
    finally:
        m.close()
        img.close()


@pytest.mark.parametrize("case, want", [
    ("missing_lm_head", "MissingTensor"),
    ("missing_post_norm", "MissingTensor"),
    ("extra_layer_record", "BadPayload"),
    ("lm_head_when_tied", "BadPayload"),
    ("o_bias", "Unsupported"),
    ("group16", "Unsupported"),
    ("wrong_shape", "BadPayload"),
])
def test_loader_rejects_like_the_reference(gh, gctx, tmp_path, case, want):
    host, packed, scales = _host(gh)
    D = TINY["dim"]
    kw = {}
    if case == "missing_lm_head":
        kw["drop"] = (ri.GLOBAL_LAYER, ri.KIND["lm_head"])
    elif case == "missing_post_norm":
        kw["drop"] = (1, ri.KIND["post_attn_norm"])
    elif case == "extra_layer_record":
        kw["extra"] = [raw_record(TINY["num_layers"], "input_norm", np.ones(D))]
    elif case == "lm_head_when_tied":
        kw["tie"] = True
        kw["extra"] = [int4_record(ri.GLOBAL_LAYER, "lm_head", host["lm_head"], TINY["vocab_size"],
                                   D, scales_f32=host["lm_head_scales"])]
    elif case == "o_bias":
        kw["extra"] = [raw_record(0, "attn_o_bias", np.zeros(D))]
    elif case == "group16":
        L = host["layers"][0]
        kw["drop"] = (0, ri.KIND["attn_o"])
        kw["extra"] = [int4_record(0, "attn_o", L["w_o"], D, D,
                                   scales_f32=np.repeat(L["s_o"], 2), group=16)]
    elif case == "wrong_shape":
        kw["drop"] = (0, ri.KIND["input_norm"])
        kw["extra"] = [raw_record(0, "input_norm", np.ones(D // 2))]
    p = _write(tmp_path, f"{case}.glrt", host, packed, scales, **kw)
    img = gh.GlrtImage(str(p))  # a valid image; the loader decides
    try:
        with pytest.raises(gh.GlrtError) as e:
            gh.Model.load_glrt(gctx, img)
        assert e.value.reason == want
    finally:
        img.close()
