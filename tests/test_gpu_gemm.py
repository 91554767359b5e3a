"""GPU parity of the MFMA GEMM (K2: projections over more than 2 rows, and
3-digit ones from 3 rows; 16-row tiles up to 16 rows, 32-row tiles up to 32
with K split over workgroups, 64-row tiles above)
against the CPU oracle, through the C ABI (glacier_hip_int4_gemv with
m > 5), and of chunked prefill end to end.

Tolerances: as the decode GEMV. Q8: every per-group integer dot is exact and
the group term RN(T * s_w) is the reference's; the activation scale is folded
into the running sum with one fused multiply-add (one rounding fewer per
group than the reference's separate multiply and add) and the across-group
order differs -> 2e-6 of max|y|. F32 (three 7-bit digit planes) -> 1e-5.
At the config sizes (M = 2048, the 7B prefill projections) a sample of the
rows is checked directly against the oracle (linear_int4_q8 /
linear_int4_f32), and the same rows recomputed as 16- and 24-row GEMMs must
agree with the 2048-row one.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _torch():
    import torch

    return torch


def _weights(gh, seed, out_f, in_f):
    packed = gh.synth_int4(seed, 1, out_f * in_f // 2)
    s16 = gh.synth_scales_f16(seed, 2, out_f * in_f // 32)
    return packed, s16, s16.view(np.float16).astype(np.float32)


def _proj(gh, gctx, w, out_f, x_np, act):
    torch = _torch()
    m = x_np.shape[0]
    xd = torch.from_numpy(np.ascontiguousarray(x_np, np.float32)).cuda()
    y = torch.empty((m, out_f), dtype=torch.float32, device="cuda")
    rc = gh.lib().glacier_hip_int4_gemv(gctx.h, w, xd.data_ptr(), gh.F32, m, None, y.data_ptr(),
                                        act, None)
    gh.check(rc, "int4_gemv", gctx.h)
    gctx.sync()
    return y.cpu().numpy()


SHAPES = [(16, 128), (48, 256), (896, 896), (128, 896), (896, 4864), (9728, 896)]


@pytest.mark.parametrize("out_f,in_f", SHAPES)
@pytest.mark.parametrize("m", [6, 9, 16, 17, 24, 32, 33, 64, 130, 300])
def test_gemm_q8_matches_oracle(gh, gctx, ora, out_f, in_f, m):
    packed, s16, s32 = _weights(gh, 300 + out_f + in_f, out_f, in_f)
    w = gctx.weight(packed, s16, in_f, out_f)
    try:
        x = np.random.default_rng(m).standard_normal((m, in_f)).astype(np.float32)
        got = _proj(gh, gctx, w, out_f, x, gh.ACT_Q8)
        want = ora.linear_int4_q8(x, packed, s32, out_f, in_f, 32)
        err = np.max(np.abs(got - want)) / np.max(np.abs(want))
        print(f"gemm q8 {out_f}x{in_f} m={m} rel={err:.3e}", flush=True)
        assert err < 2e-6
    finally:
        gh.lib().glacier_hip_int4_weight_destroy(w)


@pytest.mark.parametrize("out_f,in_f", [(48, 256), (896, 896), (512, 18944)])
@pytest.mark.parametrize("m", [3, 5, 11, 16, 20, 32, 40, 129])
def test_gemm_f32_matches_oracle(gh, gctx, ora, out_f, in_f, m):
    packed, s16, s32 = _weights(gh, 400 + out_f + in_f, out_f, in_f)
    w = gctx.weight(packed, s16, in_f, out_f)
    try:
        x = np.random.default_rng(m + 11).standard_normal((m, in_f)).astype(np.float32)
        got = _proj(gh, gctx, w, out_f, x, gh.ACT_F32)
        want = ora.linear_int4_f32(x, packed, s32, out_f, in_f, 32)
        err = np.max(np.abs(got - want)) / np.max(np.abs(want))
        print(f"gemm f32 {out_f}x{in_f} m={m} rel={err:.3e}", flush=True)
        assert err < 1e-5
    finally:
        gh.lib().glacier_hip_int4_weight_destroy(w)


@pytest.mark.parametrize("out_f,in_f,act", [(3584, 3584, "q8"), (4608, 3584, "q8"),
                                            (3584, 18944, "f32")])
def test_gemm_at_7b_prefill_size_matches_oracle(gh, gctx, ora, out_f, in_f, act):
    """M = 2048 prompt rows (the 7B QKV, O-shaped and the
    3-digit down projection): 32 rows spread over the chunk, the first and
    the last included, match the oracle; the first 16 and 24 of them run
    again as 16-row and 32-row (split-K) GEMMs agree with the 2048-row one."""
    a = gh.ACT_Q8 if act == "q8" else gh.ACT_F32
    packed, s16, _ = _weights(gh, 500 + out_f + in_f, out_f, in_f)
    w = gctx.weight(packed, s16, in_f, out_f)
    try:
        m = 2048
        x = np.random.default_rng(3).standard_normal((m, in_f)).astype(np.float32)
        big = _proj(gh, gctx, w, out_f, x, a)
        pick = np.unique(np.concatenate([[0, 1, 15, 16, 127, 128, m - 1],
                                         np.random.default_rng(4).choice(m, 25, replace=False)]))
        bar = 2e-6 if act == "q8" else 1e-5
        fn = ora.linear_int4_q8 if act == "q8" else ora.linear_int4_f32
        want = fn(x[pick], packed, s16.view(np.float16).astype(np.float32), out_f, in_f, 32)
        err = np.max(np.abs(big[pick] - want)) / np.max(np.abs(want))
        print(f"gemm 2048 rows {out_f}x{in_f} {act} vs oracle on {len(pick)} rows rel={err:.3e}",
              flush=True)
        assert err < bar
        for rows in (pick[:16], pick[:24]):
            small = _proj(gh, gctx, w, out_f, x[rows], a)
            err = np.max(np.abs(big[rows] - small)) / np.max(np.abs(small))
            print(f"gemm vs {len(rows)} rows {out_f}x{in_f} {act} rel={err:.3e}", flush=True)
            assert err < bar
        assert np.all(np.isfinite(big))
    finally:
        gh.lib().glacier_hip_int4_weight_destroy(w)


TINY = dict(num_layers=2, dim=256, hidden_dim=512, num_heads=4, num_kv_heads=2, head_dim=64,
            vocab_size=4096, group_size=32, rms_eps=1e-6, rope_theta=1e6)


@pytest.mark.parametrize("kv", ["f32", "f16"])
@pytest.mark.parametrize("chunk", [48, 100, 0])
def test_chunked_prefill_matches_oracle(gh, gctx, ora, chunk, kv):
    """A 100-token prompt in chunks of 48 (GEMM, GEMM, then a 4-row GEMV),
    in one 100-row chunk, and with the default chunk: identical greedy tokens,
    logits within 1e-2, and the page-map root chain of 100 per-token commits.
    With fp16 KV the chunks of more than 32 rows run the prefill attention
    kernel (the second 48-row chunk starts at position 48); the oracle rounds
    stored K/V rows to fp16 and the logit bar is 5e-2 (fp16 rounding-midpoint
    flips on this 2-layer model, as in the fp16 decode test)."""
    host = gh.random_model_host(TINY, 0x5EED)
    for L in host["layers"]:
        L["input_norm"] = (L["input_norm"] + 1.0).astype(np.float32)
        L["post_attn_norm"] = (L["post_attn_norm"] + 1.0).astype(np.float32)
    host["final_norm"] = (host["final_norm"] + 1.0).astype(np.float32)
    om = ora.OracleModel(TINY, host, kv_fp16=kv == "f16")
    prompt = gh.synth_tokens(0x5EED, 123, TINY["vocab_size"], 100)
    max_new = 12
    want, wl, _, out_sha = om.generate(prompt, max_new, logits_steps=[0, max_new - 1])
    m = gh.Model(gctx, TINY)
    m.set_from_host(host)
    sess = gh.Session(m, max_lanes=1, max_positions=128, prefill_chunk=chunk,
                      kv_dtype=gh.F16 if kv == "f16" else gh.F32)
    try:
        sess.begin(0)
        first, lg0 = sess.prefill(0, prompt, want_logits=True)
        toks = [first]
        lg = None
        for s in range(1, max_new):
            nxt, lg = sess.step([0], [toks[-1]], want_logits=True)
            toks.append(int(nxt[0]))
        rel0 = float(np.max(np.abs(lg0 - wl[0])) / np.max(np.abs(wl[0])))
        rel1 = float(np.max(np.abs(lg[0] - wl[1])) / np.max(np.abs(wl[1])))
        print(f"chunk={chunk} tokens {toks} oracle {want.tolist()} rel {rel0:.2e} {rel1:.2e}",
              flush=True)
        assert toks == want.tolist()
        bar = 5e-2 if kv == "f16" else 1e-2
        assert rel0 < bar and rel1 < bar
        assert bytes(sess.state(0).output_sha256) == out_sha
        r = sess.root(0)
        kvd = TINY["num_kv_heads"] * TINY["head_dim"]
        digest = ora.empty_ownership_digest(r.cache_instance, TINY["num_layers"], kvd, 128)
        n_pos = len(prompt) + max_new - 1
        for page in range((n_pos + 15) // 16):
            digest = ora.append_ownership_digest(digest, r.cache_instance, page, page + 1)
        assert (r.committed_len, r.committed_pages, r.generation) == (
            n_pos, (n_pos + 15) // 16, 1 + n_pos)
        assert bytes(r.ownership_sha256) == digest
    finally:
        sess.close()
        m.close()
