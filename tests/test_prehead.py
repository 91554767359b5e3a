"""Pins the prehead restatement (oracle/prehead.py) against the reference's
own known answers for Executor.runGreedyArgmaxEligible
(int4_executor.zig:5652-5803 sparse / fragmented / full masks, :5851-5940
invalid masks and a NaN row outside / inside the mask) and against brute
force: the token equals the already pinned eligible argmax over the full
logits, and the counts equal the rows4 groups counted directly. CPU only."""
import numpy as np
import pytest

from oracle import prehead

U64 = (1 << 64) - 1


def kat_weights(out_f, in_f, rows_0x88):
    """int4_executor.zig:5664-5688: 0x77 everywhere (w = 0), 0x88 (w = +1)
    on the listed rows, f32 scales 1.0."""
    packed = np.full(out_f * in_f // 2, 0x77, np.uint8)
    for r in rows_0x88:
        packed[r * in_f // 2:(r + 1) * in_f // 2] = 0x88
    return packed


@pytest.mark.parametrize("group", [8, 16])
def test_reference_sparse_fragmented_full_known_answers(ora, group):
    in_f, out_f = 16, 64 * 2 + 4
    winner = out_f - 3
    packed = kat_weights(out_f, in_f, [winner, out_f - 1])
    scales = np.ones(out_f * in_f // group, np.float32)
    logits = ora.linear_int4_q8(np.ones(in_f), packed, scales, out_f, in_f, group)[0]
    assert ora.argmax(logits) == winner  # :5716-5722

    def rows(a, b):
        return logits[a:b]

    sparse = [0, 0, 0]
    sparse[winner // 64] |= 1 << (winner % 64)
    sparse[(out_f - 1) // 64] |= 1 << ((out_f - 1) % 64)
    r = prehead.eligible_greedy(rows, out_f, sparse)
    assert r == dict(token_index=winner, eligible_rows=2, producer_rows=4, skipped_rows=out_f - 4,
                     overcomputed_rows=2, producer_runs=1)

    frag_ids = [1, 8, 12, 65, 130]
    frag = [0, 0, 0]
    for t in frag_ids:
        frag[t // 64] |= 1 << (t % 64)
    best = frag_ids[0]
    for t in frag_ids[1:]:
        if logits[t] > logits[best] or (logits[t] == logits[best] and t < best):
            best = t
    r = prehead.eligible_greedy(rows, out_f, frag)
    assert (r["token_index"], r["eligible_rows"], r["producer_rows"], r["producer_runs"]) == \
        (best, 5, 20, 4)

    r = prehead.eligible_greedy(rows, out_f, [U64, U64, 0x0F])
    assert r == dict(token_index=winner, eligible_rows=out_f, producer_rows=out_f, skipped_rows=0,
                     overcomputed_rows=0, producer_runs=3)


def test_reference_invalid_masks_and_nan_rows(ora):
    # int4_executor.zig:5851-5940: 4 rows x 16, all codes 0x88, scales 1;
    # a NaN first scale makes row 0's logit NaN
    in_f, out_f, group = 16, 4, 8
    packed = np.full(out_f * in_f // 2, 0x88, np.uint8)
    scales = np.ones(out_f * in_f // group, np.float32)
    for bad in ([], [0], [0x10], [1, 0]):
        with pytest.raises(prehead.ShapeMismatch):
            prehead.eligible_greedy(lambda a, b: np.zeros(b - a), out_f, bad)
    scales[0] = np.nan
    logits = ora.linear_int4_q8(np.ones(in_f), packed, scales, out_f, in_f, group)[0]
    assert np.isnan(logits[0]) and not np.isnan(logits[1:]).any()
    r = prehead.eligible_greedy(lambda a, b: logits[a:b], out_f, [0b0010])
    assert (r["token_index"], r["eligible_rows"], r["producer_rows"]) == (1, 1, 4)
    with pytest.raises(prehead.ShapeMismatch):
        prehead.eligible_greedy(lambda a, b: logits[a:b], out_f, [0b0001])


def _groups4_brute(words, out_f):
    bits = [(int(words[i // 64]) >> (i % 64)) & 1 for i in range(out_f)]
    groups = [any(bits[4 * g:4 * g + 4]) for g in range(out_f // 4)]
    runs = 0
    for t in range(0, out_f // 4, 16):  # runs never cross a 64-row tile
        prev = False
        for g in range(t, min(t + 16, out_f // 4)):
            if groups[g] and not prev:
                runs += 1
            prev = groups[g]
    return 4 * sum(groups), runs, sum(bits)


@pytest.mark.parametrize("seed", range(6))
def test_brute_force_token_and_counts(ora, seed):
    rng = np.random.default_rng(seed)
    out_f = int(rng.choice([64, 132, 1040, 4100]))
    logits = rng.standard_normal(out_f).astype(np.float32)
    logits[rng.integers(0, out_f, 3)] = logits.max()  # exact ties
    W = -(-out_f // 64)
    density = [0.005, 0.05, 0.3, 0.9, 1.0][seed % 5]
    bits = rng.random(out_f) < density
    bits[rng.integers(0, out_f)] = True
    words = [0] * W
    for i in np.nonzero(bits)[0]:
        words[i // 64] |= 1 << int(i % 64)
    calls = []

    def rows(a, b):
        calls.append((a, b))
        return logits[a:b]

    r = prehead.eligible_greedy(rows, out_f, words)
    rc, idx, n = ora.argmax_eligible(logits, np.array(words, np.uint64))
    assert rc == 0 and r["token_index"] == idx and r["eligible_rows"] == n
    producer, runs, eligible = _groups4_brute(words, out_f)
    assert (r["producer_rows"], r["producer_runs"], r["eligible_rows"]) == (producer, runs, eligible)
    # only the producer rows are ever dotted (rows4 runs, never an empty group)
    assert sum(b - a for a, b in calls) == producer
    # the reference's own consistency bounds (int4_executor.zig:1943-1950)
    assert producer % 4 == 0 and eligible <= producer <= min(out_f, 4 * eligible)
    assert -(-producer // 64) <= runs <= producer // 4
    # a device that skips 16-row blocks streams at least the rows4 walk's rows
    if out_f % 16 == 0:
        assert producer <= prehead.device_rows(words, out_f) <= out_f
