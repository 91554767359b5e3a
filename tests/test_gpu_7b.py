"""The Qwen2.5-7B-shaped model on the GPU (the headline batch-1 decode model,
BASELINE configs 4 and 5) against the oracle's committed greedy runs
(tests/golden/make_7b_golden.py; model in tests/golden/q7b_case.py).

Two activation modes, because Q8 activations make this random 28-layer model
chaotic: a code that sits on a rounding boundary moves by a whole
quantisation step when its input changes in the last bit, and the layers
amplify it; the oracle's own f32-KV and fp16-KV runs differ by 6% of the
largest logit at step 0. So:
  * f32 activations (the reference's int4_activation = .f32; the GPU's
    three-digit planes), fp16 and f32 KV: the 16-token prompt, 32 greedy
    tokens and the output digest equal the oracle's; logits within 1e-2
    max-relative (4096 sampled + top-32 indices) at steps 0, 1, 16 and 31.
    Every 7B projection and the head run at their real shapes.
  * Q8 activations (the default and the headline's mode): the first four
    greedy tokens equal the oracle's, and the step-0 / step-1 logits differ
    from the oracle's by less than the oracle's own fp16-vs-f32-KV
    difference at those steps. The Q8 kernels themselves are pinned at
    2e-6 at these shapes (tests/test_gpu_c2.py, test_gpu_gemm.py).
  * 32 lanes decoding together (the GEMM path with the plane-emitting
    finishing passes) give every lane the tokens of its own batch-1 run (f32
    mode), and in Q8 mode the same first decode token.
  * config 4: 512- and 2048-token prompts prefilled as one chunk and in small
    chunks give the same first and next token, logits within 1e-2 and K/V
    rows within 1e-2 (f32 mode).
"""
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import q7b_case  # noqa: E402

CFG = q7b_case.Q7B
V = CFG["vocab_size"]


@pytest.fixture(scope="module")
def q7b(gh, gctx):
    print("building the 7B test model", flush=True)
    host = q7b_case.make_host(gh)
    m = gh.Model(gctx, CFG)
    m.set_from_host(host)
    del host
    yield m
    m.close()


def _fx(name):
    return np.load(os.path.join(HERE, "golden", f"q7b_{name}.npz"))


def _session(gh, q7b, lanes, max_pos, kv, f32, chunk=0):
    act = gh.ACT_F32 if f32 else gh.ACT_AUTO
    return gh.Session(q7b, max_lanes=lanes, max_positions=max_pos, kv_dtype=kv,
                      layer_activation=act, head_activation=act, prefill_chunk=chunk)


def _logit_err(got, fx, i):
    return max(np.max(np.abs(got[fx["sample_idx"]] - fx["sample_logits"][i])),
               np.max(np.abs(got[fx["top_idx"][i]] - fx["top_val"][i]))) / fx["max_abs"][i]


def _run_fixture(gh, q7b, fx, kv, f32):
    sess = _session(gh, q7b, 1, 64, kv, f32)
    try:
        sess.begin(0)
        steps = fx["steps"].tolist()
        first, lg = sess.prefill(0, fx["prompt"], want_logits=True)
        toks, logits = [first], {0: lg}
        for s in range(1, len(fx["tokens"])):
            nxt, lg = sess.step([0], [toks[-1]], want_logits=True)
            toks.append(int(nxt[0]))
            if s in steps:
                logits[s] = lg[0]
        return toks, [_logit_err(logits[s], fx, i) for i, s in enumerate(steps)], \
            bytes(sess.state(0).output_sha256)
    finally:
        sess.close()


@pytest.mark.parametrize("variant", ["symf32_kvf16", "symf32"])
def test_7b_f32_batch1_greedy_matches_oracle(gh, q7b, variant):
    fx = _fx(variant)
    kv = gh.F16 if variant.endswith("kvf16") else gh.F32
    toks, errs, out_sha = _run_fixture(gh, q7b, fx, kv, True)
    want = fx["tokens"].tolist()
    print(f"{variant}: gpu {toks}\n  oracle {want}\n  logit max-rel {['%.2e' % e for e in errs]} "
          f"top-2 gaps {fx['top2_gap'].tolist()}", flush=True)
    assert len(set(want)) > 8  # a discriminative sequence
    assert max(errs) < 1e-2
    assert toks == want
    assert out_sha == fx["output_sha256"].tobytes()


@pytest.mark.parametrize("variant", ["sym_kvf16", "sym"])
def test_7b_q8_batch1_within_model_sensitivity(gh, q7b, variant):
    fx = _fx(variant)
    a, b = _fx("sym"), _fx("sym_kvf16")
    # the oracle against itself under fp16 rounding of the stored K/V rows
    sens = [float(np.max(np.abs(a["sample_logits"][i] - b["sample_logits"][i])) / a["max_abs"][i])
            for i in range(2)]
    kv = gh.F16 if variant.endswith("kvf16") else gh.F32
    toks, errs, _ = _run_fixture(gh, q7b, fx, kv, False)
    want = fx["tokens"].tolist()
    n_same = next((i for i, (x, y) in enumerate(zip(toks, want)) if x != y), len(want))
    print(f"{variant}: first divergence at {n_same}; logit max-rel {['%.2e' % e for e in errs]}; "
          f"oracle fp16-KV sensitivity {['%.2e' % e for e in sens]}", flush=True)
    assert toks[:4] == want[:4]
    assert errs[0] < sens[0] and errs[1] < sens[1]


@pytest.mark.parametrize("f32", [True, False])
def test_7b_32_lanes_match_batch1_runs(gh, q7b, f32):
    """f32 mode: 8 decode steps of 32 lanes together equal each lane's batch-1
    run. Q8 mode (chaotic, see the module docstring): the first decode step's
    logits of each lane stay within the oracle's fp16-KV sensitivity (6e-2)
    of its batch-1 logits, and the token agrees wherever the batch-1 top-2
    gap is wider than that band."""
    lanes = 32
    steps = 8 if f32 else 1
    fx = _fx("symf32_kvf16" if f32 else "sym_kvf16")
    prompts = [fx["prompt"]] + [gh.synth_tokens(q7b_case.SEED, 0x700 + i, V, 8 + (7 * i) % 41)
                                for i in range(1, lanes)]
    one = _session(gh, q7b, 1, 64, gh.F16, f32)
    want, want_lg = [], []
    try:
        for p in prompts:
            one.begin(0)
            t = [one.prefill(0, p)]
            for _ in range(steps):
                nxt, lg = one.step([0], [t[-1]], want_logits=True)
                t.append(int(nxt[0]))
            want.append(t)
            want_lg.append(lg[0])
    finally:
        one.close()
    assert want[0] == fx["tokens"][:steps + 1].tolist()
    wide = _session(gh, q7b, lanes, 64, gh.F16, f32)
    try:
        toks = []
        for i, p in enumerate(prompts):
            wide.begin(i)
            toks.append([wide.prefill(i, p)])
        ids = list(range(lanes))
        lg = None
        for _ in range(steps):
            nxt, lg = wide.step(ids, [toks[i][-1] for i in ids], want_logits=True)
            for i in ids:
                toks[i].append(int(nxt[i]))
        if f32:
            bad = [i for i in ids if toks[i] != want[i]]
        else:
            bad = []
            for i in ids:
                w = want_lg[i]
                err = float(np.max(np.abs(lg[i] - w)) / np.max(np.abs(w)))
                srt = np.sort(w)
                wide_gap = (srt[-1] - srt[-2]) > 6e-2 * np.max(np.abs(w))
                if err >= 6e-2 or (wide_gap and toks[i] != want[i]):
                    bad.append((i, err))
        print(f"f32={f32}: lanes differing from their batch-1 run: {bad}", flush=True)
        assert not bad
    finally:
        wide.close()


@pytest.mark.parametrize("T,small", [(512, 64), (2048, 256)])
def test_7b_prefill_one_chunk_equals_small_chunks(gh, q7b, T, small):
    prompt = gh.synth_tokens(q7b_case.SEED, 0x4C4F4E47 + T, V, T)
    kvd = CFG["num_kv_heads"] * CFG["head_dim"]
    res = []
    for chunk in (2048, small):
        sess = _session(gh, q7b, 1, T + 8, gh.F16, True, chunk)
        try:
            sess.begin(0)
            first, lg = sess.prefill(0, prompt, want_logits=True)
            nxt = int(sess.step([0], [first])[0])
            rows = {(l, v, p): sess.kv_row(0, l, v, p, kvd) for l in (0, 27) for v in (0, 1)
                    for p in (0, T // 2 - 1, T - 1)}
            res.append((first, lg, nxt, rows))
        finally:
            sess.close()
    (f1, l1, n1, r1), (f2, l2, n2, r2) = res
    err = float(np.max(np.abs(l2 - l1)) / np.max(np.abs(l1)))
    kv_err = max(float(np.max(np.abs(r2[k] - r1[k])) / np.max(np.abs(r1[k]))) for k in r1)
    print(f"T={T}: first {f1}/{f2} next {n1}/{n2} logit rel {err:.2e} kv rel {kv_err:.2e}", flush=True)
    assert (f1, n1) == (f2, n2)
    assert err < 1e-2
    assert kv_err < 1e-2
