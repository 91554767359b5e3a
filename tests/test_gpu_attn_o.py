"""The one-lane decode launch that fuses attention with the O projection
(glacier_hip_paged_attention_o; sessions use it for one-lane steps at
contexts up to 256 positions with fp16 or f32 KV).

Kernel parity: every KV head's partial vector parts[h] = W_o[:, slice h] .
Q8(attention[slice h]) against the oracle's Q8 matvec (linear_int4_q8,
int4_matmul.zig:380-398) of the attention output with the other slices
zeroed (a zero group quantises to zero codes and scale 0, so it adds exactly
nothing). Up to 256 positions the fused kernel's attention is the same
computation as glacier_hip_paged_attention's (one 256-position work item),
so the Q8 codes are identical and only the f32 order of the group sum
differs: 2e-6 of max|want|, the GEMV bar. Longer contexts merge their
256-position items inside the workgroup (log-sum-exp in registers) instead
of the combine kernel; the attention then differs in the last f32 bits, a
Q8 code can round the other way, and the bar against the oracle's own
attention is 5e-3. Session parity: fused and two-launch sessions give the
same greedy tokens and logits within 5e-2 of each other (the bar of the
fp16-KV tiny-model test, whose 2-layer model amplifies single Q8 code flips),
and the oracle's tokens. With head_dim 64 and 7 query heads per KV head (the
0.5B model's 14 / 2) a slice is 448 columns, 3.5 tiles: the two KV heads
share the middle tile, each adding only its own groups."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _torch():
    import torch

    return torch


def _case(gh, Hq, Hkv, hd, out_f, ctx, seed, L=3):
    rng = np.random.default_rng(seed)
    kvd = Hkv * hd
    npages = -(-ctx // 16)
    total = npages + 7
    pt = rng.permutation(total)[:npages].astype(np.int32)[None, :]
    pool = rng.standard_normal((total, L, 2, 16, kvd)).astype(np.float16)
    q = rng.standard_normal(Hq * hd).astype(np.float32)
    packed = gh.synth_int4(seed, 1, out_f * Hq * hd // 2)
    s16 = gh.synth_scales_f16(seed, 2, out_f * Hq * hd // 32)
    return pool, pt, q, packed, s16


def _run(gh, gctx, pool, pt, q, w, ctx, Hq, Hkv, hd, out_f, L=3, layer=1):
    torch = _torch()
    qd = torch.from_numpy(q).cuda()
    pdv = torch.from_numpy(pool.view(np.uint16)).cuda()
    ptd = torch.from_numpy(pt).cuda()
    cl = torch.from_numpy(np.array([ctx], np.int32)).cuda()
    parts = torch.full((Hkv, out_f), float("nan"), dtype=torch.float32, device="cuda")
    rc = gh.lib().glacier_hip_paged_attention_o(gctx.h, qd.data_ptr(), pdv.data_ptr(),
                                                ptd.data_ptr(), pt.shape[1], cl.data_ptr(), layer,
                                                L, Hq, Hkv, hd, pt.shape[1] * 16, w,
                                                parts.data_ptr(), None)
    gh.check(rc, "paged_attention_o", gctx.h)
    att = torch.empty(Hq * hd, dtype=torch.float32, device="cuda")
    rc = gh.lib().glacier_hip_paged_attention(gctx.h, qd.data_ptr(), pdv.data_ptr(), gh.F16,
                                              ptd.data_ptr(), pt.shape[1], cl.data_ptr(), 1, layer,
                                              L, Hq, Hkv, hd, ctx, att.data_ptr(), None)
    gh.check(rc, "paged_attention", gctx.h)
    gctx.sync()
    return parts.cpu().numpy(), att.cpu().numpy()


@pytest.mark.parametrize("geom,out_f", [((28, 4, 128), 512), ((4, 2, 64), 256),
                                        ((8, 2, 64), 384), ((14, 2, 64), 896)])
@pytest.mark.parametrize("ctx", [1, 15, 16, 17, 100, 255, 256, 257, 300, 700, 1030])
def test_parts_match_oracle(gh, gctx, ora, geom, out_f, ctx):
    Hq, Hkv, hd = geom
    G = Hq // Hkv
    pool, pt, q, packed, s16 = _case(gh, Hq, Hkv, hd, out_f, ctx, seed=ctx + Hq)
    s32 = s16.view(np.float16).astype(np.float32)
    w = gctx.weight(packed, s16, Hq * hd, out_f)
    try:
        print(f"attn_o Hq={Hq} Hkv={Hkv} hd={hd} N={out_f} ctx={ctx}", flush=True)
        parts, att = _run(gh, gctx, pool, pt, q, w, ctx, Hq, Hkv, hd, out_f)
        oatt = ora.attention_paged(q, pool.view(np.uint16), True, pt[0], ctx, 1, 3, Hq, Hkv,
                                   hd)[0]
        assert np.max(np.abs(att - oatt)) < 2e-5
        # one 256-position item: the same attention as the standalone kernel;
        # longer: the oracle's attention, with the Q8 rounding-flip bar
        src, bar = (att, 2e-6) if ctx <= 256 else (oatt, 5e-3)
        for h in range(Hkv):
            masked = np.zeros_like(src)
            masked[h * G * hd:(h + 1) * G * hd] = src[h * G * hd:(h + 1) * G * hd]
            want = ora.linear_int4_q8(masked[None, :], packed, s32, out_f, Hq * hd, 32)[0]
            err = np.max(np.abs(parts[h] - want)) / np.max(np.abs(want))
            print(f"  part {h} rel={err:.2e}", flush=True)
            assert err < bar
    finally:
        gh.lib().glacier_hip_int4_weight_destroy(w)


def test_rejects_unsupported_shapes(gh, gctx):
    torch = _torch()
    d = torch.zeros(1 << 16, dtype=torch.float32, device="cuda")
    p = d.data_ptr()
    packed = gh.synth_int4(3, 1, 512 * 14 * 64 // 2)
    s16 = gh.synth_scales_f16(3, 2, 512 * 14 * 64 // 32)
    w = gctx.weight(packed, s16, 14 * 64, 512)
    try:
        # 9 query heads per KV head: more than the 8 a workgroup takes
        packed9 = gh.synth_int4(3, 1, 512 * 18 * 64 // 2)
        s9 = gh.synth_scales_f16(3, 2, 512 * 18 * 64 // 32)
        w9 = gctx.weight(packed9, s9, 18 * 64, 512)
        try:
            rc = gh.lib().glacier_hip_paged_attention_o(gctx.h, p, p, p, 4, p, 0, 1, 18, 2, 64,
                                                        64, w9, p, None)
            assert rc == gh.SHAPE_MISMATCH
        finally:
            gh.lib().glacier_hip_int4_weight_destroy(w9)
        # weight width must be num_heads * head_dim
        rc = gh.lib().glacier_hip_paged_attention_o(gctx.h, p, p, p, 4, p, 0, 1, 16, 2, 64, 64,
                                                    w, p, None)
        assert rc == gh.SHAPE_MISMATCH
        rc = gh.lib().glacier_hip_paged_attention_o(gctx.h, p, p, p, 4, p, 0, 1, 14, 2, 64, 64,
                                                    None, p, None)
        assert rc == gh.INVALID_ARGUMENT
    finally:
        gh.lib().glacier_hip_int4_weight_destroy(w)


TINY = dict(num_layers=2, dim=256, hidden_dim=512, num_heads=4, num_kv_heads=2, head_dim=64,
            vocab_size=4096, group_size=32, rms_eps=1e-6, rope_theta=1e6)
SEED = 0xA770


@pytest.fixture(scope="module")
def tiny(gh, gctx, ora):
    host = gh.random_model_host(TINY, SEED)
    for L in host["layers"]:
        L["input_norm"] = (L["input_norm"] + 1.0).astype(np.float32)
        L["post_attn_norm"] = (L["post_attn_norm"] + 1.0).astype(np.float32)
    host["final_norm"] = (host["final_norm"] + 1.0).astype(np.float32)
    m = gh.Model(gctx, TINY)
    m.set_from_host(host)
    yield host, m
    m.close()


def _decode(sess, prompt, n):
    sess.begin(0, seed=3)
    first, lg = sess.prefill(0, prompt, want_logits=True)
    toks, logits = [first], [lg]
    for _ in range(n):
        nxt, lg = sess.step([0], [toks[-1]], want_logits=True)
        toks.append(int(nxt[0]))
        logits.append(lg[0])
    return toks, logits


@pytest.mark.parametrize("kv", ["f16", "f32"])
@pytest.mark.parametrize("prompt_len,steps", [(20, 30), (230, 50)])
def test_fused_session_matches_two_launches_and_oracle(gh, tiny, ora, prompt_len, steps, kv):
    """(230, 50) crosses 256 positions: the session switches from the fused
    launch to the two launches mid-run (another cached graph). f32 KV pages
    (the reference's storage) run the fused launch's f32 work item (fp16
    hi + lo MFMA products) against the two-launch path's f32 attention."""
    host, m = tiny
    prompt = gh.synth_tokens(SEED, prompt_len, TINY["vocab_size"], prompt_len)
    runs = {}
    for split in (False, True):
        sess = gh.Session(m, max_lanes=1, max_positions=320,
                          kv_dtype=gh.F16 if kv == "f16" else gh.F32, split_attention_o=split)
        try:
            runs[split] = _decode(sess, prompt, steps)
        finally:
            sess.close()
    (tf, lf), (ts, ls) = runs[False], runs[True]
    print("fused", tf, "\nsplit", ts, flush=True)
    rel = max(float(np.max(np.abs(a - b)) / np.max(np.abs(b))) for a, b in zip(lf, ls))
    print(f"fused vs two launches: max logit rel {rel:.2e}", flush=True)
    assert tf == ts
    assert rel < 5e-2
    if prompt_len <= 32:
        om = ora.OracleModel(TINY, host, kv_fp16=kv == "f16")
        want, _, _, _ = om.generate(prompt, steps + 1, logits_steps=[])
        assert tf == want.tolist()
