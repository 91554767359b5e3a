"""Write tests/golden/q7b_<variant>.npz: the oracle's greedy run of the
Qwen2.5-7B-shaped random-init model (the headline batch-1 decode model and
BASELINE configs 4/5).

Model: 28 layers, hidden 3584, 28 q heads / 4 kv heads, head_dim 128, SwiGLU
18944, vocab 152064, eps 1e-6, theta 1e6, INT4 g32 fp16 scales |N(0,0.02)|,
f32 embeddings N(0,0.02), untied INT4 LM head, no biases, with the two
changes of q7b_case.py (unit-centred norms, symmetric codes) that make greedy
decoding discriminative. The oracle (oracle/glacier_oracle.c) runs the
reference's serial oracle mode: Q8 activations for Q/K/V/O/gate/up, the f32
path for down (in_f 18944 > 16384) and the vocabulary head
(int4_matmul.zig:372-374,461-463).

Variants: "sym" (f32 KV, as the reference stores it) and "sym_kvf16" (fp16
KV pages, the headline configuration; the oracle rounds every stored K/V row
to fp16) run the default Q8 activation mode; "symf32" and "symf32_kvf16" the
reference's int4_activation = .f32 mode (generate.zig:925,3550-3596) for
every projection and the head. Q8 activations make this 28-layer model
sensitive to perturbations far below f32 rounding of the inputs: a code that
sits on a rounding boundary moves by a whole quantisation step, and the
layers amplify it (the oracle's own f32-KV and fp16-KV runs differ by 6% at
step 0). The f32 mode is continuous, so it carries the 1e-2 bar and long
greedy identity at the 7B shapes; the Q8 fixtures bound the Q8 run by the
model's measured sensitivity.

Stored: the 16-token prompt, 32 greedy tokens, the output digest, and for
generated steps 0, 1, 16 and 31 the logits at 4096 fixed random indices,
the top-32 indices/values and the top-2 gap (a near-tie audit).

Shallow variants "l2sym" (f32 KV) and "l2sym_kvf16" (fp16 KV): the same
geometry and weights with the first two layers only (q7b_case.shallow_cfg),
Q8 activations (the headline's mode), 128 greedy tokens, with the logits of
every step (1024 fixed random indices, the top 32, the top-2 gap), so a
device run fed the oracle's tokens can be compared at all 128 steps; and the
oracle's own one-ulp sensitivity at every step (ulp_sensitivity below).

Variant suffix "_ulp" (e.g. "sym_kvf16_ulp"): the same run with every
element of the prompt's embedding rows moved one ulp toward +inf; its logits
against the unperturbed fixture's are the model's own sensitivity to its
input in the last bit, the bound for the 28-layer Q8 comparison.

Run: python tests/golden/make_7b_golden.py [sym|sym_kvf16|symf32|symf32_kvf16|l2sym|l2sym_kvf16|sym_kvf16_ulp]
(~2-4 min on 8 cores for the 28-layer variants, well under a minute for the shallow ones)
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "glacier-engine_amd"), HERE]

import glacier_hip as gh  # noqa: E402
import oracle  # noqa: E402

from q7b_case import (MAX_NEW, Q7B, SHALLOW_MAX_NEW, STEPS, make_host,  # noqa: E402
                      prompt as make_prompt, shallow_cfg)


def ulp_sensitivity(cfg, variant, prompt, toks, logits):
    """The oracle against itself, fed the same tokens, with every element of
    the prompt's embedding rows moved one ulp toward +inf: per step, max
    |perturbed - base| over all logits / max |base logit|, and the steps
    whose argmax moves. No implementation that is not bit-identical to the
    oracle can be held closer than this on this model."""
    host = make_host(gh, cfg)
    emb = host["embedding"].reshape(cfg["vocab_size"], cfg["dim"])
    for tkn in set(prompt.tolist()):
        emb[tkn] = np.nextafter(emb[tkn], np.float32(np.inf))
    om = oracle.OracleModel(cfg, host, kv_fp16=variant.endswith("kvf16"))
    n = len(toks)
    ptoks, plog = om.generate_forced(prompt, toks[:-1], logits_steps=list(range(n)))
    return ptoks, plog


def subset_deviation(other, logits, idx, top_idx):
    """Per step: max |other - logits| over the stored indices (the fixed
    sample and the step's top 32) / max |logit|, as the tests measure."""
    d = np.maximum(np.abs(other[:, idx] - logits[:, idx]).max(1),
                   np.abs(np.take_along_axis(other, top_idx, 1) -
                          np.take_along_axis(logits, top_idx, 1)).max(1))
    return (d / np.abs(logits).max(1)).astype(np.float32)


def main(variant):
    oracle.build()
    oracle.set_threads(os.cpu_count() or 1)
    shallow = variant.startswith("l2")
    cfg = shallow_cfg() if shallow else Q7B
    max_new = SHALLOW_MAX_NEW if shallow else MAX_NEW
    steps = list(range(SHALLOW_MAX_NEW)) if shallow else STEPS
    t = time.time()
    host = make_host(gh, cfg)
    prompt = make_prompt(gh)
    print(f"weights generated in {time.time() - t:.1f}s", flush=True)
    if variant.endswith("_ulp"):
        # the model's sensitivity to its input in the last bit: every element
        # of the prompt's embedding rows moved one ulp toward +inf
        variant_base = variant[:-4]
        emb = host["embedding"].reshape(cfg["vocab_size"], cfg["dim"])
        for tkn in set(prompt.tolist()):
            emb[tkn] = np.nextafter(emb[tkn], np.float32(np.inf))
    else:
        variant_base = variant
    om = oracle.OracleModel(cfg, host, kv_fp16=variant_base.endswith("kvf16"),
                            act_f32=variant.startswith("symf32"))
    t = time.time()
    toks, logits, _, out_sha = om.generate(prompt, max_new, logits_steps=steps)
    print(f"oracle generate in {time.time() - t:.1f}s", flush=True)
    pert = ulp_sensitivity(cfg, variant_base, prompt, toks, logits) if shallow else None
    srt_all = np.sort(logits, axis=1)
    rel_gaps = (srt_all[:, -1] - srt_all[:, -2]) / np.abs(logits).max(1)
    rng = np.random.default_rng(1234)
    idx = np.sort(rng.choice(Q7B["vocab_size"], 1024 if shallow else 4096,
                             replace=False)).astype(np.int32)
    top_idx = np.argsort(-logits, axis=1)[:, :32].astype(np.int32)
    top_val = np.take_along_axis(logits, top_idx, axis=1)
    srt = np.sort(logits, axis=1)
    gap = (srt[:, -1] - srt[:, -2]).astype(np.float32)
    extra = {}
    if pert is not None:
        sens = subset_deviation(pert[1], logits, idx, top_idx)
        moved = np.nonzero(pert[0] != toks)[0].astype(np.int32)
        extra = dict(ulp_sensitivity=sens, ulp_argmax_moved=moved)
        print(f"one-ulp sensitivity: max {sens.max():.2e} mean {sens.mean():.2e}; argmax moves "
              f"at {moved.tolist()}", flush=True)
    np.savez_compressed(
        os.path.join(HERE, f"q7b_{variant}.npz"),
        tokens=toks, prompt=prompt, steps=np.array(steps, np.int32), sample_idx=idx,
        sample_logits=logits[:, idx], top_idx=top_idx, top_val=top_val,
        max_abs=np.abs(logits).max(1), top2_gap=gap, rel_gap_every_step=rel_gaps,
        output_sha256=np.frombuffer(out_sha, np.uint8), **extra)
    print("tokens", toks.tolist(), "distinct", len(set(toks.tolist())))
    print("smallest relative top-2 gaps", np.sort(rel_gaps)[:5].tolist())
    print("top-2 gaps at stored steps", gap.tolist(), "max |logit|", np.abs(logits).max(1).tolist())


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "sym_kvf16")
