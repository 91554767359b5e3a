"""GPU parity of the gfx950 kernels against the CPU oracle, through the C ABI.

Tolerances:
  * Q8 GEMV: the per-group integer dots are exact; only the f32 order of the
    across-group sum differs -> 2e-6 of max|y|.
  * F32 GEMV (three 7-bit digit planes): 1e-5 of max|y| (BASELINE C2 asks 1e-3).
  * BF16 activations: compared with the f32 oracle on the bf16-rounded input, 1e-5.
  * argmax / eligible argmax: bit-exact indices and counts.
  * attention: 2e-5 absolute on N(0,1) inputs (f32 KV) / vs the oracle over the
    same fp16-rounded KV (fp16 KV).
"""
import ctypes as C

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


def _gemv(gh, gctx, w, out_f, x_np, m, act, bf16=False):
    torch = _torch()
    if bf16:
        xd = torch.from_numpy(x_np).to(torch.bfloat16).cuda()
    else:
        xd = torch.from_numpy(np.ascontiguousarray(x_np, np.float32)).cuda()
    y = torch.empty((m, out_f), dtype=torch.float32, device="cuda")
    rc = gh.lib().glacier_hip_int4_gemv(gctx.h, w, xd.data_ptr(), gh.BF16 if bf16 else gh.F32, m,
                                        None, y.data_ptr(), act, None)
    gh.check(rc, "int4_gemv", gctx.h)
    gctx.sync()
    return y.cpu().numpy()


SMALL = [(16, 128), (48, 256), (896, 896), (128, 896), (896, 4864), (9728, 896)]


@pytest.mark.parametrize("out_f,in_f", SMALL)
@pytest.mark.parametrize("m", [1, 2, 4, 8, 16, 32])
def test_gemv_q8_matches_oracle(gh, gctx, ora, out_f, in_f, m):
    packed, s16, s32 = _weights(gh, 100 + out_f + in_f, out_f, in_f)
    w = gctx.weight(packed, s16, in_f, out_f)
    try:
        x = np.random.default_rng(m).standard_normal((m, in_f)).astype(np.float32)
        got = _gemv(gh, gctx, w, out_f, x, m, gh.ACT_Q8)
        want = ora.linear_int4_q8(x, packed, s32, out_f, in_f, 32)
        err = np.max(np.abs(got - want)) / np.max(np.abs(want))
        print(f"q8 {out_f}x{in_f} m={m} rel={err:.3e}", flush=True)
        assert err < 2e-6
    finally:
        gh.lib().glacier_hip_int4_weight_destroy(w)


@pytest.mark.parametrize("out_f,in_f", SMALL + [(512, 18944)])
@pytest.mark.parametrize("m", [1, 3, 8])
def test_gemv_f32_matches_oracle(gh, gctx, ora, out_f, in_f, m):
    packed, s16, s32 = _weights(gh, 200 + out_f + in_f, out_f, in_f)
    w = gctx.weight(packed, s16, in_f, out_f)
    try:
        x = np.random.default_rng(m + 7).standard_normal((m, in_f)).astype(np.float32)
        got = _gemv(gh, gctx, w, out_f, x, m, gh.ACT_F32)
        want = ora.linear_int4_f32(x, packed, s32, out_f, in_f, 32)
        err = np.max(np.abs(got - want)) / np.max(np.abs(want))
        print(f"f32 {out_f}x{in_f} m={m} rel={err:.3e}", flush=True)
        assert err < 1e-5
    finally:
        gh.lib().glacier_hip_int4_weight_destroy(w)


def test_gemv_bf16_activations(gh, gctx, ora):
    torch = _torch()
    out_f, in_f, m = 1024, 3584, 4
    packed, s16, s32 = _weights(gh, 31, out_f, in_f)
    w = gctx.weight(packed, s16, in_f, out_f)
    try:
        x = np.random.default_rng(5).standard_normal((m, in_f)).astype(np.float32)
        xb = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
        got = _gemv(gh, gctx, w, out_f, x, m, gh.ACT_F32, bf16=True)
        want = ora.linear_int4_f32(xb, packed, s32, out_f, in_f, 32)
        assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 1e-5
    finally:
        gh.lib().glacier_hip_int4_weight_destroy(w)


def test_matvec_dispatch_host_buffers(gh, gctx, ora):
    out_f, in_f = 64, 256
    packed, s16, s32 = _weights(gh, 77, out_f, in_f)
    w = gctx.weight(packed, s32, in_f, out_f)
    try:
        x = np.random.default_rng(1).standard_normal(in_f).astype(np.float32)
        y = np.zeros(out_f, np.float32)
        rc = gh.lib().glacier_hip_int4_matvec_dispatch(gctx.h, w, gh.ptr(x), in_f, gh.ptr(y), out_f)
        gh.check(rc, "matvec_dispatch", gctx.h)
        want = ora.linear_int4_f32(x, packed, s32, out_f, in_f, 32)[0]
        assert np.max(np.abs(y - want)) / np.max(np.abs(want)) < 1e-5
        rc = gh.lib().glacier_hip_int4_matvec_dispatch(gctx.h, w, gh.ptr(x), in_f - 1, gh.ptr(y), out_f)
        assert rc == gh.SHAPE_MISMATCH
    finally:
        gh.lib().glacier_hip_int4_weight_destroy(w)


def test_weight_create_rejects_bad_geometry(gh, gctx):
    packed = np.zeros(16 * 100 // 2, np.uint8)
    s = np.ones(16 * 100 // 32 + 1, np.float32)
    w = gh.lib().glacier_hip_int4_weight_create(gctx.h, gh.ptr(packed), packed.size, gh.ptr(s),
                                                s.size, 32, 100, 16)
    assert not w


# ---- argmax --------------------------------------------------------------------------
def _argmax_dev(gh, gctx, logits, words=None):
    torch = _torch()
    rows = logits.shape[0]
    ld = torch.from_numpy(np.ascontiguousarray(logits, np.float32)).cuda()
    res = (gh.ArgmaxResult * rows)()
    if words is None:
        idx = np.zeros(rows, np.uint64)
        rc = gh.lib().glacier_hip_argmax(gctx.h, ld.data_ptr(), logits.shape[1], rows, gh.ptr(idx), None)
        return rc, idx
    wd = torch.from_numpy(np.ascontiguousarray(words, np.uint64).view(np.int64)).cuda()
    rc = gh.lib().glacier_hip_eligible_argmax(gctx.h, ld.data_ptr(), logits.shape[1], wd.data_ptr(),
                                              words.shape[1], rows, res, None)
    return rc, [(r.token_index, r.eligible_rows, r.status) for r in res]


def test_argmax_matches_oracle_random_and_ties(gh, gctx, ora):
    rng = np.random.default_rng(0)
    V = 151936
    logits = rng.integers(-50, 50, (4, V)).astype(np.float32)  # many ties
    rc, idx = _argmax_dev(gh, gctx, logits)
    assert rc == 0
    assert [int(i) for i in idx] == [ora.argmax(r) for r in logits]
    g = rng.standard_normal((3, V)).astype(np.float32)
    rc, idx = _argmax_dev(gh, gctx, g)
    assert [int(i) for i in idx] == [ora.argmax(r) for r in g]


def test_argmax_nan_rules(gh, gctx, ora):
    for row in ([np.nan, 9, 3], [1, np.nan, 3], [-np.inf, -np.inf], [5, 1, 5]):
        a = np.array([row], np.float32)
        rc, idx = _argmax_dev(gh, gctx, a)
        assert int(idx[0]) == ora.argmax(row), row


def _words(bits):
    n = len(bits)
    w = np.zeros(-(-n // 64), np.uint64)
    for i in np.nonzero(bits)[0]:
        w[i // 64] |= np.uint64(1) << np.uint64(i % 64)
    return w


def test_eligible_argmax_known_answers(gh, gctx, ora):
    logits = np.full(130, -100, np.float32)
    logits[0] = np.nan
    logits[5], logits[67], logits[129] = 3.0, 9.0, 8.0
    words = np.array([[1 << 5, 1 << 3, 1 << 1]], np.uint64)
    rc, res = _argmax_dev(gh, gctx, logits[None], words)
    assert rc == 0 and res[0] == (67, 3, 0)
    rc, res = _argmax_dev(gh, gctx, np.array([[10, np.nan, 20]], np.float32),
                          np.array([[0b110]], np.uint64))
    assert rc == gh.ELIGIBLE_NAN and res[0][2] == gh.ELIGIBLE_NAN
    for vals, word, want in (([0, np.inf, 7, np.inf], 0b1010, 1), ([0, -np.inf, 7, -np.inf], 0b1010, 1),
                             ([5, 0, 5, 0], 0b0101, 0)):
        rc, res = _argmax_dev(gh, gctx, np.array([vals], np.float32), np.array([[word]], np.uint64))
        assert rc == 0 and res[0][0] == want


def test_eligible_argmax_invalid_masks(gh, gctx):
    z = np.zeros((1, 65), np.float32)
    for words in ([0, 0], [1, 0b10]):
        rc, res = _argmax_dev(gh, gctx, z, np.array([words], np.uint64))
        assert rc == gh.INVALID_MASK, words
    # wrong word count is rejected on the host before any launch
    rc, res = _argmax_dev(gh, gctx, z, np.array([[1, 0, 0]], np.uint64))
    assert rc == gh.INVALID_MASK


def test_eligible_argmax_brute_force_full_vocab(gh, gctx, ora):
    rng = np.random.default_rng(8)
    V = 152064
    logits = rng.integers(-20, 20, (4, V)).astype(np.float32)
    bits = rng.random((4, V)) < 0.1
    words = np.stack([_words(b) for b in bits])
    rc, res = _argmax_dev(gh, gctx, logits, words)
    assert rc == 0
    for r in range(4):
        orc, oidx, orows = ora.argmax_eligible(logits[r], words[r])
        assert (res[r][0], res[r][1], res[r][2]) == (oidx, orows, 0)


# ---- attention -----------------------------------------------------------------------
def _paged_case(rng, lanes_ctx, Hkv, hd, num_layers, layer, fp16):
    kvd = Hkv * hd
    pages_per = [-(-c // 16) for c in lanes_ctx]
    total = sum(pages_per) + 5
    perm = rng.permutation(total).astype(np.int32)
    max_pages = max(pages_per)
    pt = np.zeros((len(lanes_ctx), max_pages), np.int32)
    dt = np.float16 if fp16 else np.float32
    pool = rng.standard_normal((total, num_layers, 2, 16, kvd)).astype(dt)
    off = 0
    for i, p in enumerate(pages_per):
        pt[i, :p] = perm[off:off + p]
        off += p
    return pool, pt


@pytest.mark.parametrize("fp16", [False, True])
@pytest.mark.parametrize("geom", [(14, 2, 64), (28, 4, 128)])
@pytest.mark.parametrize("ctxs", [[1, 17, 256, 257, 700],  # few workgroups: one query head each
                                  [5, 16, 33, 64, 100, 129, 200, 256, 300, 333, 400, 511,
                                   512, 513, 600, 1030]])  # many: GQA-shared workgroups
def test_paged_attention_matches_oracle(gh, gctx, ora, fp16, geom, ctxs):
    torch = _torch()
    Hq, Hkv, hd = geom
    rng = np.random.default_rng(Hq + fp16 + len(ctxs))
    L, layer = 3, 2
    pool, pt = _paged_case(rng, ctxs, Hkv, hd, L, layer, fp16)
    q = rng.standard_normal((len(ctxs), Hq * hd)).astype(np.float32)
    qd = torch.from_numpy(q).cuda()
    pdv = torch.from_numpy(pool.view(np.uint16) if fp16 else pool).cuda()
    ptd = torch.from_numpy(pt).cuda()
    cl = torch.from_numpy(np.array(ctxs, np.int32)).cuda()
    out = torch.empty((len(ctxs), Hq * hd), dtype=torch.float32, device="cuda")
    rc = gh.lib().glacier_hip_paged_attention(
        gctx.h, qd.data_ptr(), pdv.data_ptr(), gh.F16 if fp16 else gh.F32, ptd.data_ptr(),
        pt.shape[1], cl.data_ptr(), len(ctxs), layer, L, Hq, Hkv, hd, max(ctxs), out.data_ptr(), None)
    gh.check(rc, "paged_attention", gctx.h)
    gctx.sync()  # the entry point is asynchronous on the context stream
    got = out.cpu().numpy()
    pool_host = pool.view(np.uint16) if fp16 else pool
    for i, c in enumerate(ctxs):
        want = ora.attention_paged(q[i], pool_host, fp16, pt[i], c, layer, L, Hq, Hkv, hd)[0]
        err = np.max(np.abs(got[i] - want))
        print(f"attn Hq={Hq} fp16={fp16} ctx={c} abs={err:.2e}", flush=True)
        assert err < 2e-5


def test_rmsnorm_matches_oracle(gh, gctx, ora):
    torch = _torch()
    x = np.random.default_rng(2).standard_normal((3, 3584)).astype(np.float32)
    w = np.random.default_rng(3).standard_normal(3584).astype(np.float32)
    xd, wd = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    out = torch.empty_like(xd)
    gh.check(gh.lib().glacier_hip_rmsnorm(gctx.h, xd.data_ptr(), wd.data_ptr(), 3, 3584, 1e-6,
                                          out.data_ptr(), None), "rmsnorm")
    gctx.sync()
    want = ora.rmsnorm(x, w, 1e-6)
    assert np.max(np.abs(out.cpu().numpy() - want) / (np.abs(want) + 1e-3)) < 1e-5


def test_paged_attention_c3_config_matches_oracle(gh, gctx, ora):
    """BASELINE config 3 geometry: 28 q / 4 kv heads, hd 128, fp16 KV in
    scattered 16-position pages, 4 lanes at contexts 512, 2048, 4096, 8192
    (above the reference's 4096 cap, which the oracle lifts unchanged)."""
    torch = _torch()
    Hq, Hkv, hd = 28, 4, 128
    ctxs = [512, 2048, 4096, 8192]
    rng = np.random.default_rng(0xC3)
    L, layer = 2, 1
    pool, pt = _paged_case(rng, ctxs, Hkv, hd, L, layer, True)
    q = rng.standard_normal((len(ctxs), Hq * hd)).astype(np.float32)
    qd = torch.from_numpy(q).cuda()
    pdv = torch.from_numpy(pool.view(np.uint16)).cuda()
    ptd = torch.from_numpy(pt).cuda()
    cl = torch.from_numpy(np.array(ctxs, np.int32)).cuda()
    out = torch.empty((len(ctxs), Hq * hd), dtype=torch.float32, device="cuda")
    rc = gh.lib().glacier_hip_paged_attention(
        gctx.h, qd.data_ptr(), pdv.data_ptr(), gh.F16, ptd.data_ptr(), pt.shape[1], cl.data_ptr(),
        len(ctxs), layer, L, Hq, Hkv, hd, max(ctxs), out.data_ptr(), None)
    gh.check(rc, "paged_attention", gctx.h)
    gctx.sync()  # the entry point is asynchronous on the context stream
    got = out.cpu().numpy()
    for i, c in enumerate(ctxs):
        want = ora.attention_paged(q[i], pool.view(np.uint16), True, pt[i], c, layer, L, Hq, Hkv,
                                   hd)[0]
        err = np.max(np.abs(got[i] - want))
        print(f"c3 ctx={c} abs={err:.2e}", flush=True)
        assert err < 2e-5


@pytest.mark.parametrize("geom", [(28, 4, 128), (14, 2, 64)])
@pytest.mark.parametrize("pos0,T", [(0, 512), (768, 256), (5, 37)])
def test_prefill_attention_matches_oracle(gh, gctx, ora, geom, pos0, T):
    """The prompt-chunk kernel (causal attention of T consecutive query rows
    over one lane's fp16 pages, glacier_hip_paged_attention_prefill) against
    the oracle's attentionMultiHead with q_seq = T, query_start = pos0, at
    the 7B geometry (28 q / 4 kv heads, hd 128) and the
    0.5B one, chunks starting at page boundaries and inside a page; pages
    scattered by a seeded permutation. Bar 2e-5 absolute on N(0, 1) inputs
    (the oracle reads the same fp16 KV)."""
    torch = _torch()
    Hq, Hkv, hd = geom
    rng = np.random.default_rng(pos0 + T + Hq)
    L, layer = 2, 1
    kv_seq = pos0 + T
    pool, pt = _paged_case(rng, [kv_seq], Hkv, hd, L, layer, True)
    q = rng.standard_normal((T, Hq * hd)).astype(np.float32)
    qd = torch.from_numpy(q).cuda()
    pdv = torch.from_numpy(pool.view(np.uint16)).cuda()
    ptd = torch.from_numpy(np.ascontiguousarray(pt[0])).cuda()
    out = torch.empty((T, Hq * hd), dtype=torch.float32, device="cuda")
    print(f"prefill attention {Hq}/{Hkv}x{hd} pos0={pos0} T={T}", flush=True)
    rc = gh.lib().glacier_hip_paged_attention_prefill(
        gctx.h, qd.data_ptr(), pdv.data_ptr(), ptd.data_ptr(), pt.shape[1], pos0, T, layer, L,
        Hq, Hkv, hd, out.data_ptr(), None)
    gh.check(rc, "paged_attention_prefill", gctx.h)
    gctx.sync()
    got = out.cpu().numpy()
    want = ora.attention_paged(q, pool.view(np.uint16), True, pt[0], kv_seq, layer, L, Hq, Hkv, hd)
    err = float(np.max(np.abs(got - want)))
    print(f"  abs {err:.2e}", flush=True)
    assert err < 2e-5
