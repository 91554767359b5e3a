"""Write tests/golden/c1_qwen05b.npz: the oracle's greedy run of the
Qwen2.5-0.5B-shaped random-init model.

Model: 24 layers, hidden 896, 14 q heads / 2 kv heads, head_dim 64, SwiGLU
4864, vocab 151936, eps 1e-6, theta 1e6, INT4 g32 fp16 scales |N(0,0.02)|,
f32 embeddings / norms N(0,0.02), untied INT4 LM head, no biases. Weights come
from the product's synthetic generator (glacier_hip_synth_*), the same bytes
glacier_hip_model_init_random uploads; the oracle (oracle/glacier_oracle.c)
runs the reference's serial oracle mode on them.

Stored: the 128 greedy tokens, the logical-KV and output digests, and for
generated steps 0, 1, 64 and 127 the logits at 4096 fixed random indices plus
the top-32 indices/values.

A second fixture, c1_qwen05b_unitnorm.npz, uses the same tensors except
that every RMSNorm weight is 1 + N(0, 0.02): with the config's N(0, 0.02)
norm weights the residual stream is dominated by the attention average and
greedy decoding repeats one token, which makes token identity a weak check;
the unit-norm variant produces a varied sequence.

A third fixture, c1_qwen05b_unitnorm_kvf16.npz, is the unit-norm model with
fp16 KV pages (BASELINE configs 3 and 5 ask for fp16 KV; the reference stores
f32): the oracle rounds every K/V row to fp16 on store.

A fourth fixture, c1_qwen05b_sym.npz, is discriminative in the headline's
Q8 mode: unit-centred norms and symmetric codes (every nibble 15 decoded as
7, as tests/golden/q7b_case.py does for the 7B model; codes uniform on 0..15
give every projection the same rank-one mean component), f32 KV, and the
logits of all 128 steps (1024 fixed random indices, the top 32, the top-2
gap), so a device run fed the oracle's tokens is compared at every step,
and the oracle's own one-ulp sensitivity at every step (the same run fed the
same tokens with the prompt's embedding rows one ulp off).

Run: python tests/golden/make_c1_golden.py [spec|unitnorm|unitnorm_kvf16|sym]  (~2 min each on 8 cores)
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "glacier-engine_amd")]

import glacier_hip as gh  # noqa: E402
import oracle  # noqa: E402

sys.path.insert(0, HERE)
from q7b_case import symmetric_codes  # noqa: E402

C1 = dict(num_layers=24, dim=896, hidden_dim=4864, num_heads=14, num_kv_heads=2, head_dim=64,
          vocab_size=151936, group_size=32, rms_eps=1e-6, rope_theta=1e6)
SEED = 0x474C4143
PROMPT_ID = 0x50524F4D
PROMPT_LEN = 128
MAX_NEW = 128
STEPS = [0, 1, 64, 127]


def unit_norm(host):
    for L in host["layers"]:
        L["input_norm"] = (L["input_norm"] + 1.0).astype(np.float32)
        L["post_attn_norm"] = (L["post_attn_norm"] + 1.0).astype(np.float32)
    host["final_norm"] = (host["final_norm"] + 1.0).astype(np.float32)
    return host


def main(variant):
    oracle.build()
    oracle.set_threads(os.cpu_count() or 1)
    t = time.time()
    host = gh.random_model_host(C1, SEED)
    if variant.startswith("unitnorm") or variant == "sym":
        host = unit_norm(host)
    if variant == "sym":
        host = symmetric_codes(host)
    steps = list(range(MAX_NEW)) if variant == "sym" else STEPS
    prompt = gh.synth_tokens(SEED, PROMPT_ID, C1["vocab_size"], PROMPT_LEN)
    print(f"weights generated in {time.time() - t:.1f}s", flush=True)
    om = oracle.OracleModel(C1, host, kv_fp16=variant.endswith("kvf16"))
    t = time.time()
    toks, logits, kv_sha, out_sha = om.generate(prompt, MAX_NEW, logits_steps=steps)
    print(f"oracle generate in {time.time() - t:.1f}s", flush=True)
    extra = {}
    if variant == "sym":
        # the oracle fed the same tokens with the prompt's embedding rows one
        # ulp off: its own sensitivity to the last bit of its input, per step
        pert = symmetric_codes(unit_norm(gh.random_model_host(C1, SEED)))
        emb = pert["embedding"].reshape(C1["vocab_size"], C1["dim"])
        for tkn in set(prompt.tolist()):
            emb[tkn] = np.nextafter(emb[tkn], np.float32(np.inf))
        ptoks, plog = oracle.OracleModel(C1, pert).generate_forced(prompt, toks[:-1],
                                                                   logits_steps=steps)
    rng = np.random.default_rng(1234)
    idx = np.sort(rng.choice(C1["vocab_size"], 1024 if variant == "sym" else 4096,
                             replace=False)).astype(np.int32)
    top_idx = np.argsort(-logits, axis=1)[:, :32].astype(np.int32)
    top_val = np.take_along_axis(logits, top_idx, axis=1)
    srt = np.sort(logits, axis=1)
    if variant == "sym":  # on the stored indices, as the tests measure the device
        d = np.maximum(np.abs(plog[:, idx] - logits[:, idx]).max(1),
                       np.abs(np.take_along_axis(plog, top_idx, 1) - top_val).max(1))
        sens = (d / np.abs(logits).max(1)).astype(np.float32)
        extra = dict(ulp_sensitivity=sens,
                     ulp_argmax_moved=np.nonzero(ptoks != toks)[0].astype(np.int32))
        print(f"one-ulp sensitivity: max {sens.max():.2e} mean {sens.mean():.2e}; argmax moves "
              f"at {extra['ulp_argmax_moved'].tolist()}", flush=True)
    np.savez_compressed(
        os.path.join(HERE, "c1_qwen05b.npz" if variant == "spec" else f"c1_qwen05b_{variant}.npz"),
        tokens=toks, prompt=prompt,
        steps=np.array(steps, np.int32), sample_idx=idx, sample_logits=logits[:, idx],
        top_idx=top_idx, top_val=top_val, max_abs=np.abs(logits).max(1),
        top2_gap=(srt[:, -1] - srt[:, -2]).astype(np.float32),
        kv_sha256=np.frombuffer(kv_sha, np.uint8), output_sha256=np.frombuffer(out_sha, np.uint8),
        seed=np.array([SEED], np.uint64), **extra)
    print("tokens", toks.tolist(), "distinct", len(set(toks.tolist())))
    print("smallest top-2 gaps", np.sort(srt[:, -1] - srt[:, -2])[:5].tolist())


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "spec")
