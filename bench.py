#!/usr/bin/env python3
"""Headline benchmark: Qwen2.5-7B-shaped INT4 decode on one MI355X.

  python bench.py [--gpus 1] [--steps K] [--warmup W]

One "step" is one greedy decode token of the batch-1 lane (the full token
loop: embedding gather, 28 layers, final norm, LM head, argmax, per-token
commit). `value` = tokens/s over exactly K timed steps with the weights and
KV already resident in HBM. The same JSON line carries:
  * lanes32     32 concurrent lanes decoding together at short context
                (tokens/s, aggregate);
  * c5_laneweave config 5: 32 lanes under LaneWeave weighted IWRR, prompts
                U[64, 4096], 256 tokens each through the eligible argmax;
  * gemv        the INT4 GEMV kernel timed alone on the BASELINE config-2
                shapes at M = 1, 2, 4 and 8 and on the 7B gate/up projection,
                with HIP events on the launch stream;
  * prefill     config 4: 7B time to first token at T = 512 and 2048 and the
                int8 MFMA rate it implies;
  * attention   config 3: paged GQA decode attention alone, 4 lanes at
                contexts 512..8192, GB/s;
  * roofline    for the dominant kernel: the 7B gate/up launch that runs in
                the batch-1 token (53% of its weight bytes), algorithmic bytes
                / its average launch duration from HIP events on the step
                stream (in_token_kernels: gate/up, down, attention + O, QKV),
                traffic from the committed counter summary;
  * cpu_baseline the CPU oracle (the reference algorithm restated in C) on the
                same model, timed on this host's cores over a bounded sample;
                with the cpu section the gemv (M = 1), attention and prefill
                entries also carry the oracle's rate on the same inputs (and
                the GPU result's deviation from it) under "cpu".
Weights are random-init from a fixed seed (no checkpoints exist offline).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "glacier-engine_amd")]

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
INT8_PEAK_OPS = 5.0e15   # MI355X dense int8 MFMA
SEED = 0x474C4143
CFG_7B = dict(num_layers=28, dim=3584, hidden_dim=18944, num_heads=28, num_kv_heads=4,
              head_dim=128, vocab_size=152064, group_size=32, rms_eps=1e-6, rope_theta=1e6)
CFG_05B = dict(num_layers=24, dim=896, hidden_dim=4864, num_heads=14, num_kv_heads=2,
               head_dim=64, vocab_size=151936, group_size=32, rms_eps=1e-6, rope_theta=1e6)
# BASELINE config 2 GEMV shapes [N, K] plus the fused 7B gate/up projection
GEMV_SHAPES = [(4096, 4096), (11008, 4096), (4096, 11008), (18944, 3584), (152064, 3584)]
GATE_UP = (2 * 18944, 3584)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemv_bytes(n, k, m, digits=1):
    """Algorithmic HBM bytes of one prepared GEMV launch: packed codes (K/2 per
    row) + fp16 group scales (K/16 per row) + the activation planes it reads
    (`digits` int8 bytes per element plus an 8-byte scale/correction per
    32-element group, per row of M) + the f32 outputs."""
    return n * k // 2 + n * k // 16 + m * k * digits + m * (k // 32) * 8 + m * n * 4


MALL_BYTES = 256 << 20   # MI355X Infinity Cache; rotated weight copies must exceed it


class ColdWeights:
    """Copies of one [n, k] weight (same content, separate HBM allocations),
    enough that the 256 MB MALL cannot serve a repeat: the condition of every
    projection in a decode token (a 7B model is ~4.5 GB of weights)."""

    def __init__(self, gh, ctx, n, k):
        self.gh, self.n, self.k = gh, n, k
        packed = gh.synth_int4(SEED, n * 7 + k, n * k // 2)
        s16 = gh.synth_scales_f16(SEED, n * 11 + k, n * k // 32)
        wbytes = n * k // 2 + n * k // 16
        self.copies = max(2, -(-3 * MALL_BYTES // wbytes))
        self.ws = [ctx.weight(packed, s16, k, n) for _ in range(self.copies)]

    def close(self):
        for w in self.ws:
            self.gh.lib().glacier_hip_int4_weight_destroy(w)
        self.ws = []


def time_gemv(gh, ctx, torch, cw, m, reps, act, end_to_end_bf16=False):
    """Cold GEMV timing over the weight copies `cw`, HIP events on the launch
    stream around a captured graph. Prepared launches (activation planes made
    once, untimed: the decode chain produces them inside the previous kernel)
    with Q8 or 3-digit f32 planes; or, with end_to_end_bf16, the whole
    glacier_hip_int4_gemv call on bf16 activations (the conversion launch
    included, BASELINE config 2's bf16 leg)."""
    L = gh.lib()
    n, k, copies = cw.n, cw.k, cw.copies
    ws = cw.ws
    stream = torch.cuda.Stream()  # non-null handle: our launches and the events share it
    dt = torch.bfloat16 if end_to_end_bf16 else torch.float32
    x = torch.randn((m, k), device="cuda", dtype=torch.float32).to(dt)
    y = torch.empty((m, n), device="cuda", dtype=torch.float32)
    planes = torch.empty(L.glacier_hip_activation_bytes(m, k, act), dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    gh.check(L.glacier_hip_activation_prepare(ctx.h, x.data_ptr(), gh.BF16 if end_to_end_bf16
                                              else gh.F32, m, k, act, planes.data_ptr(),
                                              stream.cuda_stream), "prepare")

    def go(i):
        if end_to_end_bf16:
            return L.glacier_hip_int4_gemv(ctx.h, ws[i % copies], x.data_ptr(), gh.BF16, m, None,
                                           y.data_ptr(), act, stream.cuda_stream)
        return L.glacier_hip_int4_gemv_prepared(ctx.h, ws[i % copies], planes.data_ptr(), m, act,
                                                None, y.data_ptr(), stream.cuda_stream)
    for i in range(copies):
        gh.check(go(i), "gemv", ctx.h)
    torch.cuda.synchronize()
    # the launches are captured into a graph so that host submission cost
    # (ctypes + launch, several us) does not hide the kernels' own time
    reps = max(reps, copies) // copies * copies
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i in range(reps):
            go(i)
    iters = 5
    with torch.cuda.stream(stream):
        g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(iters):
            g.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / (reps * iters)
    del g
    if end_to_end_bf16:  # BASELINE config 2's byte count with a = 2
        b = n * k // 2 + n * k // 16 + m * k * 2 + m * n * 4
        mode = "bf16_in_" + ("q8" if act == gh.ACT_Q8 else "f32")
    else:
        b = gemv_bytes(n, k, m, 1 if act == gh.ACT_Q8 else 3)
        mode = "q8" if act == gh.ACT_Q8 else "f32"
    return dict(N=n, K=k, M=m, act=mode, us=round(us, 2), bytes=b, gbs=round(b / us / 1e3, 1),
                frac=round(b / us / 1e3 / HBM_PEAK_GBS, 4), weight_copies=copies)


def cpu_gemv(gh, ctx, torch, n, k, act):
    """Config-2 CPU leg for one shape at M = 1: the oracle's row-split
    restatement of the reference's a2 (f32) / a3 (Q8) GEMV timed on every host
    core (at most 16) and on 8 threads (the reference executor's cap), and the
    GPU launch's result on the same inputs compared with it (max |diff| /
    max |oracle|; the reference's own bar is 1e-3)."""
    import oracle

    oracle.build()
    L = gh.lib()
    packed = gh.synth_int4(SEED, n * 7 + k, n * k // 2)
    s16 = gh.synth_scales_f16(SEED, n * 11 + k, n * k // 32)
    s32 = s16.view(np.float16).astype(np.float32)
    x = np.random.default_rng(n + k).standard_normal((1, k)).astype(np.float32)
    w = ctx.weight(packed, s16, k, n)
    try:
        xd = torch.from_numpy(x).cuda()
        yd = torch.empty((1, n), dtype=torch.float32, device="cuda")
        gh.check(L.glacier_hip_int4_gemv(ctx.h, w, xd.data_ptr(), gh.F32, 1, None, yd.data_ptr(),
                                         act, None), "gemv", ctx.h)
        ctx.sync()
        got = yd.cpu().numpy()
    finally:
        L.glacier_hip_int4_weight_destroy(w)
    fn = oracle.linear_int4_q8 if act == gh.ACT_Q8 else oracle.linear_int4_f32
    cores = min(len(os.sched_getaffinity(0)), 16)
    res = {}
    want = None
    for th in (cores, 8):
        oracle.set_threads(th)
        want = fn(x, packed, s32, n, k, 32)
        reps = 1
        t0 = time.perf_counter()
        dt = 0.0
        while dt < 0.2 and reps < 64:  # a few tenths of a second per thread count
            fn(x, packed, s32, n, k, 32)
            dt = time.perf_counter() - t0
            reps += 1
        res[th] = dt / (reps - 1)
    b = gemv_bytes(n, k, 1, 1 if act == gh.ACT_Q8 else 3)
    err = float(np.max(np.abs(got - want)) / np.max(np.abs(want)))
    return dict(threads=cores, us=round(res[cores] * 1e6, 1), gbs=round(b / res[cores] / 1e9, 2),
                us_8_threads=round(res[8] * 1e6, 1), gbs_8_threads=round(b / res[8] / 1e9, 2),
                max_rel_vs_oracle=float(f"{err:.3g}"), kind="port")


def profile_value(name, key):
    """A `key = value` line of a committed profiles/ summary (None when the
    summary or the line is absent)."""
    try:
        for line in open(os.path.join(ROOT, "profiles", name)):
            if line.startswith(key + " ="):
                return float(line.split("=")[1])
    except (OSError, ValueError):
        pass
    return None


def measured_traffic(name):
    """HBM bytes per launch from a committed rocprofv3 --pmc FETCH_SIZE /
    WRITE_SIZE summary (copy-kernel calibrated), or None."""
    v = profile_value(name, "traffic_bytes_per_launch")
    return None if v is None else int(v)


def int4_weights(cfg):
    """INT4 weights of a model (every projection and the LM head)."""
    d, f, v = cfg["dim"], cfg["hidden_dim"], cfg["vocab_size"]
    kvd = cfg["num_kv_heads"] * cfg["head_dim"]
    return cfg["num_layers"] * (d * (d + 2 * kvd) + d * d + 3 * f * d) + v * d


def kv_bytes_per_position(cfg, elem):
    """K and V of every layer for one position (what attention reads)."""
    return 2 * cfg["num_layers"] * cfg["num_kv_heads"] * cfg["head_dim"] * elem


def step_roofline(cfg, tokens_per_s, steps_per_s, kv_positions_per_step, kv_elem):
    """HBM roofline of a decode step: the INT4 weights (0.5625 B each: codes
    + fp16 group scales) once per step, the K/V every lane reads, the
    embedding rows; achieved = bytes per step x steps per second."""
    wb = int4_weights(cfg) * 9 // 16
    b = wb + kv_positions_per_step * kv_bytes_per_position(cfg, kv_elem) + \
        (tokens_per_s / steps_per_s) * cfg["dim"] * 4
    gbs = b * steps_per_s / 1e9
    return dict(bound="hbm", achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                frac=round(gbs / HBM_PEAK_GBS, 4), bytes_per_step=int(b), weight_bytes=wb)


def host_info(ctx):
    info = ctx.info()
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    rocm = "unknown"
    try:
        rocm = open("/opt/rocm/.info/version").read().strip()
    except OSError:
        pass
    import torch

    return dict(cpu_model=cpu, host_cores_available=len(os.sched_getaffinity(0)),
                rocm_version=rocm, torch=torch.__version__,
                gpu=dict(name=info.name.decode(), arch=info.arch.decode(),
                         compute_units=info.compute_units,
                         hbm_bytes=info.total_global_bytes))


def bench_c1(gh, ctx, steps=128, prompt_len=128, cpu=True):
    """the Qwen2.5-0.5B-shaped INT4 model (random init from
    the seed), batch 1, f32 paged KV as the reference stores it, a 128-token
    prompt then 128 greedy tokens (the first from the prompt's logits, 127
    decode steps timed). A warm-up request on another lane captures the
    decode graph first. CPU leg: the oracle's serial greedy loop (the
    reference's oracle mode) on a short sample, 1 thread and all cores."""
    cfg = CFG_05B
    model = gh.Model(ctx, cfg)
    model.init_random(SEED)
    # (the step's kernels are short here, so its sealed plan replays as a
    # hipGraph: 1190 tok/s against 1175 replaying the launches one by one)
    sess = gh.Session(model, max_lanes=2, max_positions=prompt_len + steps + 8, kv_dtype=gh.F32,
                      use_graph=2)
    try:
        prompt = gh.synth_tokens(SEED, 0x50524F4D, cfg["vocab_size"], prompt_len)
        sess.begin(1, seed=2)
        t = sess.prefill(1, prompt)
        for _ in range(8):
            t = int(sess.step([1], [t])[0])
        sess.begin(0, seed=1)
        tok = sess.prefill(0, prompt)
        t0 = time.perf_counter()
        for _ in range(steps - 1):
            tok = int(sess.step([0], [tok])[0])
        dt = time.perf_counter() - t0
    finally:
        sess.close()
        model.close()
    tps = (steps - 1) / dt
    mean_ctx = prompt_len + steps / 2
    res = dict(workload="Qwen2.5-0.5B-shaped INT4 g32, batch 1, 128-token prompt, 128 greedy "
                        "tokens, f32 paged KV", tokens_per_s=round(tps, 1),
               ms_per_token=round(dt * 1e3 / (steps - 1), 4),
               roofline=step_roofline(cfg, tps, tps, mean_ctx, 4))
    if not cpu:
        log("c1", res)
        return res
    # CPU leg: the oracle on a bounded sample (8-token prompt, 8 tokens)
    import oracle

    oracle.build()
    host = gh.random_model_host(cfg, SEED)
    om = oracle.OracleModel(cfg, host)
    p8 = gh.synth_tokens(SEED, 0x50524F4D, cfg["vocab_size"], 8)
    cpu = {}
    for th in (1, min(len(os.sched_getaffinity(0)), 16)):
        oracle.set_threads(th)
        t0 = time.perf_counter()
        om.generate(p8, 8)
        cpu[th] = 16 / (time.perf_counter() - t0)  # 16 token forwards (8 prompt, 8 generated)
    res["cpu"] = dict(kind="port", sample="oracle greedy loop, 8-token prompt + 8 tokens",
                      tokens_per_s_1_thread=round(cpu[1], 2),
                      threads=max(cpu), tokens_per_s=round(cpu[max(cpu)], 2))
    log("c1", res)
    return res


def auto_act(gh, n, k):
    return gh.ACT_F32 if (n > 65536 or k > 16384) else gh.ACT_Q8


def decode_batch1(gh, sess, prompt, warmup, steps, probe=None):
    """Batch-1 greedy decode of lane 0: `warmup` untimed tokens, then exactly
    `steps` timed ones. With `probe` (a step count), the in-token kernels are
    then timed per launch (probe_in_token), after the timed region."""
    tok = sess.prefill(0, prompt)
    for _ in range(warmup):
        tok = int(sess.step([0], [tok])[0])
    t0 = time.perf_counter()
    for _ in range(steps):
        tok = int(sess.step([0], [tok])[0])
    dt = time.perf_counter() - t0
    if probe:
        return steps / dt, dt, probe_in_token(sess, tok, probe, len(prompt) + warmup + steps)
    return steps / dt, dt


IN_TOKEN_KINDS = ("gate_up", "down", "attention", "qkv")


def in_token_bytes(cfg, kind, ctx_len, kv_elem=2):
    """Algorithmic HBM bytes of one batch-1 in-token launch of a layer: the
    INT4 weights it streams (codes + fp16 group scales, 9/16 B per weight)
    plus the activations it reads and writes once (f32 rows, 1- or 3-digit
    int8 planes with an 8-byte scale/correction per 32-group, K/V rows)."""
    D, F = cfg["dim"], cfg["hidden_dim"]
    kvd = cfg["num_kv_heads"] * cfg["head_dim"]
    w = lambda n, k: n * k // 2 + n * k // 16
    if kind == "gate_up":  # x and the norm weight in; SwiGLU's 3-digit planes for down out
        return w(2 * F, D) + 2 * D * 4 + F * 3 + F // 32 * 8
    if kind == "down":  # 3-digit planes and the residual in; the new residual out
        return w(D, F) + F * 3 + F // 32 * 8 + 2 * D * 4
    if kind == "qkv":  # x and the norm weight in; q out, the K/V row into its page
        return w(D + 2 * kvd, D) + 2 * D * 4 + D * 4 + 2 * kvd * kv_elem
    # attention fused with O: q, the lane's K/V, the O weights and residual in; h out
    return w(D, D) + D * 4 + ctx_len * 2 * kvd * kv_elem + 2 * D * 4


def probe_in_token(sess, tok, steps, ctx0, reps=4):
    """The batch-1 token's kernels timed with HIP events on the step stream,
    after the timed region:
      * gate/up and down: the last token's launches of all 28 layers (same
        kernel, launch shape, inputs and per-layer weights, so every launch
        streams its weights from HBM) replayed `reps` times back to back,
        events around the run (glacier_hip_session_probe_replay): the
        launch-to-launch duration a kernel trace reports;
      * every kind: events around each launch of `steps` more tokens
        (glacier_hip_session_probe_kernel), which adds each launch's
        dispatch latency (avg_us_events)."""
    out = {}
    for kind in IN_TOKEN_KINDS:
        sess.probe_kernel(kind)
        for _ in range(steps):
            tok = int(sess.step([0], [tok])[0])
        us, n = sess.probe_read()
        ctx = ctx0 + steps / 2
        ctx0 += steps
        b = in_token_bytes(CFG_7B, kind, ctx)
        ev = us / max(n, 1)
        r = dict(avg_us_events=round(ev, 2), launches_events=n, bytes_per_launch=int(b))
        avg = ev
        if kind in ("gate_up", "down"):
            sess.probe_kernel(None)
            avg = sess.probe_replay(kind, reps)
            r.update(avg_us=round(avg, 2), launches=reps * CFG_7B["num_layers"])
        else:
            r.update(avg_us=round(ev, 2), launches=n)
        r.update(gbs=round(b / avg / 1e3, 1), frac=round(b / avg / 1e3 / HBM_PEAK_GBS, 4))
        out[kind] = r
    sess.probe_kernel(None)
    return out


def decode_long_context(gh, model, prompt_len, warmup, steps):
    """Batch-1 decode after a `prompt_len`-token prompt, fp16 and f32 KV:
    the token whose attention reads ~2048 positions per layer."""
    out = {}
    for name, kv, elem in (("fp16_kv", gh.F16, 2), ("f32_kv", gh.F32, 4)):
        sess = gh.Session(model, max_lanes=1, max_positions=prompt_len + warmup + steps + 8,
                          kv_dtype=kv, prefill_chunk=2048)
        try:
            sess.begin(0, seed=1)
            prompt = gh.synth_tokens(SEED, 0x4C4F4E47, model.cfg["vocab_size"], prompt_len)
            tps, dt = decode_batch1(gh, sess, prompt, warmup, steps)
        finally:
            sess.close()
        out[name] = dict(value=round(tps, 2), unit="tokens/s", ms_per_step=round(dt * 1e3 / steps, 4),
                         roofline=step_roofline(model.cfg, tps, tps,
                                                prompt_len + warmup + steps / 2 + 1, elem))
    out.update(prompt_len=prompt_len, steps=steps)
    return out


def decode_leased(gh, model, prompt, max_pos, warmup, steps):
    """The batch-1 decode on a lane whose KV pages are charged through a
    LeaseTree (each new page reserved and settled in the bank before the step
    takes it), then sealed and reclaimed; the page-charge work rides the host
    side of the step."""
    import ctypes as C
    pages = -(-max_pos // 16)
    page_bytes = CFG_7B["num_layers"] * 2 * 16 * CFG_7B["num_kv_heads"] * CFG_7B["head_dim"] * 2
    bank = gh.LeaseBank(1, pages + 4, 0x4C454153, kv_bytes=pages * page_bytes, queue_slots=1)
    parent = bank.commit(bank.reserve(1, queue_slots=1))
    tree = bank.open_tree(parent, 2, 3, kv_bytes=pages * page_bytes)
    scope = bank.open_scope(tree, 4, 5, kv_bytes=pages * page_bytes)
    seq = C.c_uint64(0)
    bank.bind_session(tree, 6, 7)
    sess = gh.Session(model, max_lanes=1, max_positions=max_pos, kv_dtype=gh.F16)
    try:
        sess.begin(0, seed=1)
        lk = gh.LeasedKV(bank, tree, scope, sess, 6, 7, seq, lane=0, binding_count=pages)
        tps, dt = decode_batch1(gh, sess, prompt, warmup, steps)
        charged = tree.current.kv_bytes
        seal = lk.seal_terminal(lk.root(), lk.kv_sha256(), seq.value, 0, 0)
        lk.commit_reclaim(lk.begin_reclaim(seal, seq.value))
        out = dict(tokens_per_s=round(tps, 2), ms_per_token=round(dt * 1e3 / steps, 4),
                   pages_charged=charged // page_bytes, charge_after_reclaim=tree.current.kv_bytes)
        lk.close()
        return out
    finally:
        sess.close()


def decode_eligible(gh, model, prompt, warmup, steps, density=0.01):
    """Batch-1 greedy decode with a caller-certified eligibility mask of the
    given density on every step (a fresh random mask per step from a fixed
    set), in the posthead domain (every logit, then the masked argmax) and
    the prehead domain (LM-head row blocks with no eligible token stream no
    weights). Same session, same tokens."""
    V = model.cfg["vocab_size"]
    rng = np.random.default_rng(SEED)
    masks = []
    for _ in range(8):
        bits = rng.random(V) < density
        bits[int(rng.integers(V))] = True
        words = np.zeros(-(-V // 64), np.uint64)
        idx = np.nonzero(bits)[0]
        np.bitwise_or.at(words, idx // 64, np.left_shift(np.uint64(1), (idx % 64).astype(np.uint64)))
        masks.append(words[None])
    blocks = sum(1 for b in range(V // 16)
                 if (int(masks[0][0][b // 4]) >> ((b % 4) * 16)) & 0xFFFF)
    out = dict(density=density, head_blocks_streamed_frac=round(blocks / (V // 16), 4))
    for mode, name in ((gh.HEAD_DOMAIN_POSTHEAD, "posthead"), (gh.HEAD_DOMAIN_PREHEAD, "prehead")):
        sess = gh.Session(model, max_lanes=1, max_positions=len(prompt) + warmup + steps + 8,
                          kv_dtype=gh.F16)
        sess.set_head_domain(mode)
        sess.begin(0, seed=1)
        tok = sess.prefill(0, prompt)
        toks = []
        for i in range(warmup):
            tok = int(sess.step([0], [tok], eligible=masks[i % 8])[0])
        t0 = time.perf_counter()
        for i in range(steps):
            tok = int(sess.step([0], [tok], eligible=masks[i % 8])[0])
            toks.append(tok)
        dt = time.perf_counter() - t0
        sess.close()
        out[name] = dict(tokens_per_s=round(steps / dt, 1), ms_per_token=round(dt * 1e3 / steps, 4))
        out[name + "_tokens"] = toks
    out["same_tokens"] = out.pop("posthead_tokens") == out.pop("prehead_tokens")
    return out


def c5_workload(cfg, lanes=32, gen=256, prompt_lo=64, prompt_hi=4096, max_weight=4):
    """The config-5 admission set: prompt lengths U[prompt_lo, prompt_hi] by
    seed, LaneWeave weights 1..max_weight by lane, each lane's request spec
    (gen - 1 decode quanta; its fp16 KV pages charged to the scheduler's Bank)
    and the Bank / scheduler parameters. Model-free: the scheduler's event
    chain depends on nothing else."""
    rng = np.random.default_rng(SEED ^ 0xC5)
    plens = [int(x) for x in rng.integers(prompt_lo, prompt_hi + 1, size=lanes)]
    weights = [1 + (i % max_weight) for i in range(lanes)]
    kvd = cfg["num_kv_heads"] * cfg["head_dim"]
    page_bytes = cfg["num_layers"] * 2 * 16 * kvd * 2
    pages = [-(-(p + gen) // 16) for p in plens]
    specs = [dict(tenant_key=i + 1, request_key=10 * (i + 1), request_generation=1,
                  resource_owner_key=100 * (i + 1), weight=weights[i], work_quanta=gen - 1,
                  deadline_tick=0, claim=dict(kv_bytes=pages[i] * page_bytes, queue_slots=1))
             for i in range(lanes)]
    bank = dict(host_bytes=sum(pages) * page_bytes, kv_bytes=sum(pages) * page_bytes,
                queue_slots=lanes)
    return dict(lanes=lanes, gen=gen, plens=plens, weights=weights, pages=pages,
                page_bytes=page_bytes, specs=specs, bank=bank, bank_epoch=0x42414E4B,
                scheduler_epoch=0x51534553, max_weight=max_weight, prompt_hi=prompt_hi)


def bench_c5(gh, model, lanes=32, gen=256, prompt_lo=64, prompt_hi=4096, max_weight=4):
    """32 concurrent lanes under LaneWeave weighted IWRR
    (weights 1..4 by lane, max_weight 4), prompt lengths uniform in
    [64, 4096] by seed, each lane generating `gen` greedy tokens through the
    eligible argmax over an all-ones full-vocab mask, KV paged at 16 fp16
    positions. Every lane is admitted (its KV claim charged to the scheduler's
    Bank) and prefilled; then decode waves run until every lane's quanta are
    served: each wave batches the next IWRR quanta of distinct lanes into one
    device step and commits them in scheduler order. Decode tok/s counts the
    tokens of the waves over their wall time; end-to-end adds prefill."""
    cfg = model.cfg
    wl = c5_workload(cfg, lanes, gen, prompt_lo, prompt_hi, max_weight)
    plens, weights, pages = wl["plens"], wl["weights"], wl["pages"]
    V = cfg["vocab_size"]
    W = (V + 63) // 64
    sess = gh.Session(model, max_lanes=lanes, max_positions=prompt_hi + gen + 8, kv_dtype=gh.F16,
                      total_pages=sum(pages), prefill_chunk=2048)
    sched = gh.LaneWeave(lanes, wl["bank"], bank_epoch=wl["bank_epoch"],
                         scheduler_epoch=wl["scheduler_epoch"], max_weight=max_weight)
    try:
        tokens = np.zeros(lanes, np.uint32)
        t0 = time.perf_counter()
        for i in range(lanes):
            sp = wl["specs"][i]
            spec = gh.LaneWeave.spec(sp["tenant_key"], sp["request_key"], sp["request_generation"],
                                     sp["resource_owner_key"], sp["weight"], sp["work_quanta"],
                                     sp["deadline_tick"], sp["claim"])
            ok, _, _ = sched.admit(spec)
            assert ok, "admission rejected"
            sess.begin(i, seed=i)
            prompt = gh.synth_tokens(SEED, 0x4C414E45 + i, V, plens[i])
            tokens[i] = sess.prefill(i, prompt)
        t_prefill = time.perf_counter() - t0
        elig = np.full((lanes, W), np.uint64(0xFFFFFFFFFFFFFFFF), np.uint64)
        if V % 64:
            elig[:, -1] = np.uint64((1 << (V % 64)) - 1)
        t1 = time.perf_counter()
        n_tok, waves = 0, 0
        served = [0] * lanes
        kv_positions = 0  # positions attended, summed over every served quantum
        while True:
            try:
                slots, evs = sched.wave(sess, list(range(lanes)), tokens, elig)
            except gh.GlacierHipError as e:
                if e.code == gh.NO_RUNNABLE:
                    break
                raise
            waves += 1
            n_tok += len(slots)
            for sl in slots:
                served[sl] += 1
                kv_positions += plens[sl] + served[sl]
            for ev in evs:
                if ev.remaining_after == 0:
                    assert sched.retire(ev.handle)[0] == 0
        t_decode = time.perf_counter() - t1
        rc, cev = sched.close()
        assert rc == 0
        res = dict(lanes=lanes, tokens_per_lane=gen, weights="1..4 by lane",
                   prompt_len_min=min(plens), prompt_len_max=max(plens),
                   prompt_tokens=sum(plens), prefill_s=round(t_prefill, 2),
                   decode_tokens=n_tok, waves=waves, mean_wave=round(n_tok / max(waves, 1), 2),
                   decode_s=round(t_decode, 2), decode_tokens_per_s=round(n_tok / t_decode, 1),
                   roofline=step_roofline(cfg, n_tok / t_decode, waves / t_decode,
                                          kv_positions / max(waves, 1), 2),
                   end_to_end_tokens_per_s=round((n_tok + lanes) / (t_prefill + t_decode), 1),
                   event_chain_head=bytes(cev.event_sha256).hex())
        log("c5", res)
        return res
    finally:
        sess.close()


def decode_lanes(gh, sess, lanes, prompts, warmup, steps):
    toks = []
    for i in range(lanes):
        sess.begin(i, seed=i)
        toks.append(sess.prefill(i, prompts[i]))
    ids = list(range(lanes))
    for _ in range(warmup):
        toks = [int(t) for t in sess.step(ids, toks)]
    t0 = time.perf_counter()
    for _ in range(steps):
        toks = [int(t) for t in sess.step(ids, toks)]
    dt = time.perf_counter() - t0
    return lanes * steps / dt, dt


def layer_params(cfg):
    d, f, kvd = cfg["dim"], cfg["hidden_dim"], cfg["num_kv_heads"] * cfg["head_dim"]
    qkv, o, gu, down = d * (d + 2 * kvd), d * d, 2 * f * d, d * f
    return qkv, o, gu, down


def bench_prefill(gh, model, lengths, reps=3):
    """time to first token of a fresh lane for prompts of T
    uniform random ids (wall clock around the synchronous prefill call: all
    28 layers over the prompt in one 2048-row chunk, then the last row's LM
    head and argmax). MFMA figures: the algorithmic contraction is
    2 * T * (layer weights) int8 multiply-adds (plus one head row); the
    executed count triples the down projection, whose 18944-wide input runs
    as three 7-bit digit planes (the reference's f32-activation path for
    in_f > 16384)."""
    cfg = model.cfg
    qkv, o, gu, down = layer_params(cfg)
    L = cfg["num_layers"]
    out = []
    for T in lengths:
        sess = gh.Session(model, max_lanes=1, max_positions=T + 8, kv_dtype=gh.F16,
                          prefill_chunk=min(T, 2048))
        try:
            prompt = gh.synth_tokens(SEED, 0x50524546 + T, cfg["vocab_size"], T)
            times = []
            for r in range(reps + 1):
                sess.begin(0, seed=r)
                t0 = time.perf_counter()
                sess.prefill(0, prompt)
                times.append(time.perf_counter() - t0)
            ttft = float(np.median(times[1:]))
            algo = 2.0 * T * L * (qkv + o + gu + down) + 2.0 * cfg["dim"] * cfg["vocab_size"]
            execd = 2.0 * T * L * (qkv + o + gu + 3 * down) + 2.0 * cfg["dim"] * cfg["vocab_size"]
            out.append(dict(T=T, ttft_ms=round(ttft * 1e3, 2), tokens_per_s=round(T / ttft, 1),
                            int8_mfma_algorithmic_tops=round(algo / ttft / 1e12, 1),
                            int8_mfma_executed_tops=round(execd / ttft / 1e12, 1),
                            mfma_frac_of_5000_tops=round(execd / ttft / INT8_PEAK_OPS, 4)))
            if T == 2048:  # the gate/up GEMM's VALU issue share, from its committed counters
                out[-1]["gate_up_valu_issue_frac"] = profile_value("prefill_7b_t2048_pmc.md",
                                                                   "valu_issue_fraction")
            log("prefill", out[-1])
        finally:
            sess.close()
    return out


def bench_attention(gh, ctx, torch, reps=20, cpu=False):
    """paged GQA decode attention alone at Qwen2.5-7B head
    geometry (28 q / 4 kv heads, hd 128), fp16 KV in 16-position pages of a
    28-layer payload, pages scattered by a seeded permutation, 4 lanes at
    contexts 512 / 2048 / 4096 / 8192. HIP events on the launch stream around
    a captured graph of `reps` launches. Algorithmic bytes: K and V of every
    attended position (2 * ctx * 4 * 128 * 2 B per lane) + q/out rows + page
    table entries."""
    L = gh.lib()
    Hq, Hkv, hd, layers, layer = 28, 4, 128, 28, 27
    ctxs = [512, 2048, 4096, 8192]
    pages = [c // 16 for c in ctxs]
    total = sum(pages)
    g = torch.Generator().manual_seed(SEED)
    perm = torch.randperm(total, generator=g).to(torch.int32)
    pt = torch.zeros((len(ctxs), max(pages)), dtype=torch.int32)
    off = 0
    for i, p in enumerate(pages):
        pt[i, :p] = perm[off:off + p]
        off += p
    pool = torch.randn((total, layers, 2, 16, Hkv * hd), dtype=torch.float16, device="cuda")
    q = torch.randn((len(ctxs), Hq * hd), dtype=torch.float32, device="cuda")
    out = torch.empty_like(q)
    ptd = pt.cuda()
    cl = torch.tensor(ctxs, dtype=torch.int32, device="cuda")
    stream = torch.cuda.Stream()

    def go():
        gh.check(L.glacier_hip_paged_attention(ctx.h, q.data_ptr(), pool.data_ptr(), gh.F16,
                                               ptd.data_ptr(), pt.shape[1], cl.data_ptr(), len(ctxs),
                                               layer, layers, Hq, Hkv, hd, max(ctxs),
                                               out.data_ptr(), stream.cuda_stream), "attention")
    go()
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=stream):
        for _ in range(reps):
            go()
    with torch.cuda.stream(stream):
        gr.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(5):
            gr.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / (reps * 5)
    b = sum(2 * c * Hkv * hd * 2 for c in ctxs) + len(ctxs) * Hq * hd * 4 * 2 + sum(pages) * 4
    res = dict(contexts=ctxs, us=round(us, 2), bytes=b, gbs=round(b / us / 1e3, 1),
               frac=round(b / us / 1e3 / HBM_PEAK_GBS, 4), kv="fp16, 28-layer pages")
    if cpu:
        # config-3 CPU leg: the oracle's a7 (fp16 pages widened to f32, one
        # thread, as the reference's attention) on the same pool and rows
        import oracle

        oracle.build()
        go()
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        pool_h = pool.cpu().numpy()
        qh = q.cpu().numpy()
        t0 = time.perf_counter()
        want = np.stack([oracle.attention_paged(qh[i], pool_h, True, pt[i].numpy(), ctxs[i], layer,
                                                layers, Hq, Hkv, hd)[0] for i in range(len(ctxs))])
        dt = time.perf_counter() - t0
        res["cpu"] = dict(threads=1, us=round(dt * 1e6, 1), gbs=round(b / dt / 1e9, 3), kind="port",
                          max_rel_vs_oracle=float(f"{np.max(np.abs(got - want)) / np.max(np.abs(want)):.3g}"))
        del pool_h
    log("attention", res)
    del gr, pool
    return res


def cpu_baseline(host, prompt_tok, budget_s=15.0):
    import oracle

    oracle.build()
    cores = len(os.sched_getaffinity(0))
    cores = min(cores, 16)
    oracle.set_threads(cores)
    om = oracle.OracleModel(CFG_7B, host)
    t0 = time.perf_counter()
    om.generate(np.array([prompt_tok], np.uint32), 1)
    one = time.perf_counter() - t0
    n = max(2, min(64, int(budget_s / max(one, 1e-3))))
    t0 = time.perf_counter()
    om.generate(np.array([prompt_tok], np.uint32), n)
    dt = time.perf_counter() - t0
    # config-4 leg: the reference prefills token at a time (generate.zig:5080);
    # an 8-token prompt (plus the one head and argmax) gives its prompt rate
    p8 = np.full(8, prompt_tok, np.uint32)
    t0 = time.perf_counter()
    om.generate(p8, 1)
    dp = time.perf_counter() - t0
    return dict(value=round(n / dt, 3), unit="tokens/s", cores=cores, kind="port",
                sample=f"oracle greedy run of the same 7B model: 1-token prompt + {n} tokens "
                       f"({dt:.1f} s), Q8 layers / f32 head, {cores} threads row-split",
                prefill_tokens_per_s=round(8 / dp, 3))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--lanes", type=int, default=32)
    ap.add_argument("--lane-prompt", type=int, default=64)
    ap.add_argument("--gemv-reps", type=int, default=50)
    ap.add_argument("--gemv-only", action="store_true", help="only the GEMV kernel timing")
    ap.add_argument("--gemv-rows", type=int, default=1,
                    help="with --gemv-only: activation rows of the timed gate/up launch (past "
                         "16 rows the C ABI runs the MFMA GEMM; counter runs at prefill size)")
    ap.add_argument("--sections", default="gemv,decode,lanes,c5,c1,prefill,attention,cpu",
                    help="comma list of gemv, decode, lanes, c5, c1, prefill, attention, cpu "
                         "(profiling runs select one; the JSON line needs decode)")
    ap.add_argument("--probe-steps", type=int, default=8,
                    help="tokens per in-token kernel timed with HIP events after the timed "
                         "batch-1 region (0: none)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-attention", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only a 1 GiB device-to-device copy, 5 times (HBM counter calibration "
                         "under rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)")
    a = ap.parse_args()
    if a.copy_probe:
        import torch

        src = torch.ones(1 << 30, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps(dict(copy_bytes=1 << 30, copies=5)))
        return
    secs = set(a.sections.split(","))
    if "lanes" not in secs:
        a.lanes = 1
    a.no_prefill = a.no_prefill or "prefill" not in secs
    a.no_attention = a.no_attention or "attention" not in secs
    a.no_cpu_baseline = a.no_cpu_baseline or "cpu" not in secs
    if a.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {a.gpus}); this build has no "
              "multi-GPU path: lanes would shard across GPUs with no exchange.", file=sys.stderr)
        sys.exit(2)

    import torch

    import glacier_hip as gh

    ctx = gh.Context(0)
    info = ctx.info()
    log(f"device {info.arch.decode()} CUs={info.compute_units}")

    # ---- GEMV kernel alone ----
    gemv = []
    n, k = GATE_UP
    dom = None
    if "gemv" in secs or a.gemv_only:
        rows = a.gemv_rows if a.gemv_only else 1
        cw = ColdWeights(gh, ctx, n, k)
        dom = time_gemv(gh, ctx, torch, cw, rows, a.gemv_reps * 2, gh.ACT_Q8)
        cw.close()
        log("gemv gate/up", dom)
    if not a.gemv_only and "gemv" in secs:
        for (n, k) in GEMV_SHAPES:
            cw = ColdWeights(gh, ctx, n, k)
            try:
                for m in (1, 2, 4, 8):
                    # the reference's x86 dispatch (Q8, f32 for the head), then
                    # the other activation mode, then the bf16-input call
                    for act in (auto_act(gh, n, k), gh.ACT_F32 if auto_act(gh, n, k) == gh.ACT_Q8
                                else gh.ACT_Q8):
                        r = time_gemv(gh, ctx, torch, cw, m, a.gemv_reps, act)
                        if m == 1 and act == auto_act(gh, n, k) and not a.no_cpu_baseline:
                            r["cpu"] = cpu_gemv(gh, ctx, torch, n, k, act)
                        log("gemv", r)
                        gemv.append(r)
                    r = time_gemv(gh, ctx, torch, cw, m, a.gemv_reps, auto_act(gh, n, k),
                                  end_to_end_bf16=True)
                    log("gemv", r)
                    gemv.append(r)
            finally:
                cw.close()
    # (replaced by the in-token gate/up launch when the decode section runs)
    roofline = dict(bound="hbm", achieved=dom["gbs"], peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=dom["frac"], traffic=None) if dom else None
    if a.gemv_only:
        print(json.dumps(dict(metric=f"int4 gemv HBM GB/s (7B gate/up, M={dom['M']})",
                              value=dom["gbs"], unit="GB/s", roofline=roofline, gemv=[dom])))
        return

    # ---- 7B model ----
    need_7b = bool(secs & {"decode", "decode1", "lanes", "c5", "prefill", "cpu"})
    if not need_7b:  # kernel-only sections (profiling runs)
        attn = bench_attention(gh, ctx, torch, cpu=False) if not a.no_attention else None
        c1 = bench_c1(gh, ctx, cpu=False) if "c1" in secs else None
        print(json.dumps(dict(metric="sections " + a.sections, attention=attn, c1_qwen05b=c1,
                              gemv=([dom] if dom else []) + gemv, host=host_info(ctx))))
        return
    t0 = time.perf_counter()
    host = gh.random_model_host(CFG_7B, SEED)
    model = gh.Model(ctx, CFG_7B)
    model.set_from_host(host)
    log(f"7B model built in {time.perf_counter() - t0:.1f}s, {model.weight_bytes() / 1e9:.2f} GB in HBM")
    prompt = gh.synth_tokens(SEED, 0x50524F4D, CFG_7B["vocab_size"], a.prompt)
    max_pos = max(a.prompt, a.lane_prompt) + a.warmup + a.steps + 8 + \
        a.probe_steps * len(IN_TOKEN_KINDS)
    sess = gh.Session(model, max_lanes=max(1, a.lanes), max_positions=max_pos, kv_dtype=gh.F16)
    sess.begin(0, seed=1)
    tps1, dt1, in_token = 0.0, 0.0, None
    if secs & {"decode", "decode1"}:  # decode1: the batch-1 token and its kernel probes only
        r = decode_batch1(gh, sess, prompt, a.warmup, a.steps, probe=a.probe_steps)
        tps1, dt1, in_token = r if a.probe_steps else (*r, None)
        log(f"batch-1 decode {tps1:.1f} tok/s ({dt1 * 1e3 / a.steps:.3f} ms/token)")
        log("in-token kernels", in_token)
    lanes = None
    if a.lanes > 1:
        prompts = [gh.synth_tokens(SEED, 0x4C414E45 + i, CFG_7B["vocab_size"], a.lane_prompt)
                   for i in range(a.lanes)]
        tpsL, dtL = decode_lanes(gh, sess, a.lanes, prompts, a.warmup, a.steps)
        steps_per_s = a.steps / dtL
        mean_ctx = a.lane_prompt + a.warmup + a.steps / 2 + 1
        lanes = dict(value=round(tpsL, 1), unit="tokens/s", lanes=a.lanes,
                     ms_per_step=round(dtL * 1e3 / a.steps, 3), prompt_len=a.lane_prompt,
                     context_range=[a.lane_prompt, a.lane_prompt + a.warmup + a.steps],
                     roofline=step_roofline(CFG_7B, tpsL, steps_per_s, a.lanes * mean_ctx, 2))
        log(f"{a.lanes}-lane decode {tpsL:.1f} tok/s")
    sess.close()
    f32kv = elig = leased = long_ctx = None
    if "decode" in secs:
        # the same batch-1 decode on f32 KV pages, the reference's storage
        s32 = gh.Session(model, max_lanes=1, max_positions=max_pos, kv_dtype=gh.F32)
        s32.begin(0, seed=1)
        tps32, dt32 = decode_batch1(gh, s32, prompt, a.warmup, a.steps)
        s32.close()
        f32kv = dict(value=round(tps32, 2), unit="tokens/s",
                     ms_per_step=round(dt32 * 1e3 / a.steps, 4), kv="f32 paged",
                     roofline=step_roofline(CFG_7B, tps32, tps32,
                                            a.prompt + a.warmup + a.steps / 2 + 1, 4))
        log(f"batch-1 decode, f32 KV {tps32:.1f} tok/s")
        elig = decode_eligible(gh, model, prompt, a.warmup, min(a.steps, 32))
        log("batch-1 decode with a 1% eligibility mask", elig)
        leased = decode_leased(gh, model, prompt, max_pos, a.warmup, a.steps)
        log("batch-1 decode on a leased lane", leased)
        long_ctx = decode_long_context(gh, model, 2048, a.warmup, min(a.steps, 32))
        log("batch-1 decode at 2048 context", long_ctx)
    c5 = bench_c5(gh, model) if "c5" in secs else None
    prefill = bench_prefill(gh, model, [512, 2048]) if not a.no_prefill else None
    model.close()
    attn = bench_attention(gh, ctx, torch, cpu=not a.no_cpu_baseline) if not a.no_attention else None
    c1 = bench_c1(gh, ctx, cpu=not a.no_cpu_baseline) if "c1" in secs else None
    cpu = None if a.no_cpu_baseline else cpu_baseline(host, int(prompt[0]))
    if cpu:
        log("cpu baseline", cpu)
        for pf in prefill or []:
            pf["cpu"] = dict(threads=cpu["cores"], tokens_per_s=cpu["prefill_tokens_per_s"],
                             ttft_s_estimate=round(pf["T"] / cpu["prefill_tokens_per_s"], 1),
                             kind="port", sample="8-token prompt, token at a time")
        if c5:
            # the reference serves one lane per quantum with the serial token
            # loop (F10): its multi-lane rate is its single-lane rate
            c5["vs_cpu_reference"] = round(c5["decode_tokens_per_s"] / cpu["value"], 1)
    if in_token:
        # the line's roofline: the gate/up launch that runs in the token
        # (input mode, deferred RMSNorm, SwiGLU emitting down's planes)
        g = in_token["gate_up"]
        roofline = dict(bound="hbm", achieved=g["gbs"], peak=HBM_PEAK_GBS, unit="GB/s",
                        frac=g["frac"], traffic=measured_traffic("gate_up_7b_in_token_pmc.md"),
                        kernel="gemv_kernel<1, true, 256, EPI_SWIGLU, true> (7B gate/up in the "
                               "batch-1 token)", avg_us=g["avg_us"],
                        bytes_per_launch=g["bytes_per_launch"])
    out = dict(
        metric="decode tok/s at batch 1 (7B INT4)", value=round(tps1, 2), unit="tokens/s",
        n_gpus=1, steps=a.steps, warmup=a.warmup, ms_per_step=round(dt1 * 1e3 / max(a.steps, 1), 4),
        higher_is_better=True, scaling="weak", vs_baseline=None, dtype="int8xint4 (Q8) / f32",
        data="synthetic random-init weights (seed 0x474C4143), uniform random prompt ids",
        config=dict(workload="Qwen2.5-7B-shaped INT4 g32 greedy decode, batch 1",
                    prompt_len=a.prompt, kv="fp16 paged, 16 positions/page",
                    parallelism="single GPU"),
        roofline=roofline, in_token_kernels=in_token, cpu_baseline=cpu, host=host_info(ctx),
        decode_roofline=step_roofline(CFG_7B, tps1, tps1, a.prompt + a.warmup + a.steps / 2 + 1, 2)
        if tps1 else None,
        decode_f32_kv=f32kv, decode_eligible=elig, decode_leased=leased, decode_2048=long_ctx, lanes32=lanes, c5_laneweave=c5, c1_qwen05b=c1, prefill=prefill, attention=attn,
        gemv=([dom] if dom else []) + gemv)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
