"""Prehead eligible greedy on the GPU against the oracle's restatement of
Executor.runGreedyArgmaxEligible (oracle/prehead.py, pinned in
tests/test_prehead.py), through the C ABI.

Bars: the reference's counts exactly (eligible / producer / skipped /
overcomputed rows, producer runs) and the device's streamed rows; the token
equal to the oracle's wherever the top-2 gap among the eligible logits
exceeds the GEMV tolerance (2e-6 of max|y| for Q8, 1e-5 for f32), else a
token whose oracle logit is within that tolerance of the best. A session in
the prehead head domain decodes the same tokens as one in the posthead
domain (the same head arithmetic, empty row blocks skipped).
"""
import ctypes as C

import numpy as np
import pytest

from oracle import prehead

pytestmark = pytest.mark.gpu


def _torch():
    import torch

    return torch


def _words(out_f, ids):
    w = np.zeros(-(-out_f // 64), np.uint64)
    for i in ids:
        w[i // 64] |= np.uint64(1) << np.uint64(i % 64)
    return w


def _masks(out_f, rng):
    full = np.ones(out_f, bool)
    return {
        "sparse2": _words(out_f, [out_f - 3, out_f - 1]),
        "fragmented": _words(out_f, [1, 8, 12, 65, 130]),
        "full": _words(out_f, np.nonzero(full)[0]),
        "one_block": _words(out_f, range(48, 64)),
        "pct1": _words(out_f, np.nonzero(rng.random(out_f) < 0.01)[0].tolist() + [7]),
        "pct30": _words(out_f, np.nonzero(rng.random(out_f) < 0.3)[0]),
    }


def _call(gh, gctx, w, x_dev, in_f, words, act):
    r = gh.EligibleGreedyResult()
    r.token_index = 0xDEAD
    rc = gh.lib().glacier_hip_int4_eligible_greedy(gctx.h, w, x_dev, in_f, words.ctypes.data,
                                                   words.size, act, C.byref(r), None)
    return rc, r


@pytest.mark.parametrize("out_f,in_f", [(1040, 256), (4096, 896)])
@pytest.mark.parametrize("act", ["q8", "f32"])
def test_prehead_matches_oracle(gh, gctx, ora, out_f, in_f, act):
    torch = _torch()
    packed = gh.synth_int4(7, out_f + in_f, out_f * in_f // 2)
    s16 = gh.synth_scales_f16(7, 3 * out_f + in_f, out_f * in_f // 32)
    s32 = s16.view(np.float16).astype(np.float32)
    w = gctx.weight(packed, s16, in_f, out_f)
    rng = np.random.default_rng(out_f)
    x = rng.standard_normal(in_f).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    if act == "q8":
        logits = ora.linear_int4_q8(x, packed, s32, out_f, in_f, 32)[0]
        code, tol = gh.ACT_Q8, 2e-6
    else:
        logits = ora.linear_int4_f32(x, packed, s32, out_f, in_f, 32)[0]
        code, tol = gh.ACT_F32, 1e-5
    try:
        for name, words in _masks(out_f, rng).items():
            want = prehead.eligible_greedy(lambda a, b: logits[a:b], out_f, words)
            rc, r = _call(gh, gctx, w, xd.data_ptr(), in_f, words, code)
            assert rc == 0, (name, rc)
            got = {k: getattr(r, k) for k in want}
            print(f"{out_f}x{in_f} {act} {name}: {got} device_rows={r.device_rows}", flush=True)
            for k in ("eligible_rows", "producer_rows", "skipped_rows", "overcomputed_rows",
                      "producer_runs"):
                assert got[k] == want[k], (name, k)
            assert r.device_rows == prehead.device_rows(words, out_f)
            elig = np.array([(int(words[i // 64]) >> (i % 64)) & 1 for i in range(out_f)], bool)
            vals = np.where(elig, logits, -np.inf)
            top = np.sort(vals[elig])[::-1]
            scale = tol * float(np.max(np.abs(logits)))
            assert elig[r.token_index]
            if len(top) == 1 or top[0] - top[1] > 2 * scale:
                assert r.token_index == want["token_index"], name
            else:
                assert logits[r.token_index] >= top[0] - 2 * scale, name
    finally:
        gh.lib().glacier_hip_int4_weight_destroy(w)


def test_prehead_rejections_write_nothing(gh, gctx, ora):
    torch = _torch()
    out_f, in_f = 1040, 256
    packed = gh.synth_int4(9, 1, out_f * in_f // 2)
    s16 = gh.synth_scales_f16(9, 2, out_f * in_f // 32)
    s16[0] = 0x7E00  # NaN: row 0's first group scale, so row 0's logit is NaN
    w = gctx.weight(packed, s16, in_f, out_f)
    x = torch.from_numpy(np.random.default_rng(1).standard_normal(in_f).astype(np.float32)).cuda()
    W = -(-out_f // 64)
    try:
        bad_masks = [np.zeros(W, np.uint64),                      # empty
                     np.zeros(W + 1, np.uint64),                  # word count
                     _words(out_f + 16, [out_f + 3])[:W]]         # a bit past out_f
        bad_masks[1][0] = 1
        for words in bad_masks:
            rc, r = _call(gh, gctx, w, x.data_ptr(), in_f, words, gh.ACT_Q8)
            assert rc == gh.SHAPE_MISMATCH and r.token_index == 0xDEAD
        # the NaN row outside the mask is never a candidate; inside it fails
        rc, r = _call(gh, gctx, w, x.data_ptr(), in_f, _words(out_f, [1]), gh.ACT_Q8)
        assert rc == 0 and r.token_index == 1 and r.producer_rows == 4
        rc, r = _call(gh, gctx, w, x.data_ptr(), in_f, _words(out_f, [0, 1]), gh.ACT_Q8)
        assert rc == gh.SHAPE_MISMATCH and r.token_index == 0xDEAD
        # a non-finite input is rejected before any launch
        xn = x.clone()
        xn[5] = float("inf")
        rc, r = _call(gh, gctx, w, xn.data_ptr(), in_f, _words(out_f, [1]), gh.ACT_Q8)
        assert rc == gh.SHAPE_MISMATCH and r.token_index == 0xDEAD
        # wrong input width
        rc, r = _call(gh, gctx, w, x.data_ptr(), in_f - 128, _words(out_f, [1]), gh.ACT_Q8)
        assert rc == gh.SHAPE_MISMATCH
    finally:
        gh.lib().glacier_hip_int4_weight_destroy(w)


TINY = dict(num_layers=2, dim=256, hidden_dim=512, num_heads=4, num_kv_heads=2, head_dim=64,
            vocab_size=4096, group_size=32, rms_eps=1e-6, rope_theta=1e6)


@pytest.mark.parametrize("lanes", [1, 3])
@pytest.mark.parametrize("head_act", ["q8", "f32"])
def test_session_prehead_equals_posthead(gh, gctx, lanes, head_act):
    host = gh.random_model_host(TINY, 0x5EED)
    for L in host["layers"]:
        L["input_norm"] = (L["input_norm"] + 1.0).astype(np.float32)
        L["post_attn_norm"] = (L["post_attn_norm"] + 1.0).astype(np.float32)
    host["final_norm"] = (host["final_norm"] + 1.0).astype(np.float32)
    m = gh.Model(gctx, TINY)
    m.set_from_host(host)
    V = TINY["vocab_size"]
    act = gh.ACT_Q8 if head_act == "q8" else gh.ACT_F32
    sess = [gh.Session(m, max_lanes=lanes, max_positions=64, head_activation=act) for _ in range(2)]
    sess[1].set_head_domain(gh.HEAD_DOMAIN_PREHEAD)
    rng = np.random.default_rng(lanes)
    try:
        toks = []
        for s in sess:
            t = []
            for ln in range(lanes):
                s.begin(ln, seed=ln + 1)
                t.append(s.prefill(ln, gh.synth_tokens(3, 40 + ln, V, 9 + ln)))
            toks.append(t)
        assert toks[0] == toks[1]
        cur = toks[0]
        for step in range(12):
            dens = [0.002, 0.01, 0.05, 0.3][step % 4]
            words = np.stack([_words(V, np.nonzero(rng.random(V) < dens)[0].tolist() + [int(rng.integers(V))])
                              for _ in range(lanes)])
            outs = [s.step(list(range(lanes)), cur, eligible=words) for s in sess]
            assert [int(v) for v in outs[0]] == [int(v) for v in outs[1]], step
            for ln in range(lanes):
                i = int(outs[1][ln])
                assert (int(words[ln][i // 64]) >> (i % 64)) & 1
            cur = [int(v) for v in outs[1]]
        # prehead never returns logits of an eligible step; nothing is published
        before = sess[1].root(0).committed_len
        rc, _ = sess[1].step(list(range(lanes)), cur, eligible=words, want_logits=True,
                             raise_on_error=False)
        assert rc == gh.INVALID_ARGUMENT
        assert sess[1].root(0).committed_len == before
        assert sess[0].state(0).sampling_calls == sess[1].state(0).sampling_calls
    finally:
        for s in sess:
            s.close()
        m.close()
