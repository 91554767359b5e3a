"""Restatement of the reference's prehead eligible greedy projection.

TEST INFRASTRUCTURE ONLY: the checker for glacier_hip_int4_eligible_greedy
and the session's prehead head domain. Only tests/, __graft_entry__.smoke()
and bench.py's CPU leg use it.

Follows /root/reference/src/int4_executor.zig:
  validateEligibleWords (used by runGreedyArgmaxEligible :1880-1885): exactly
      ceil(out_f / 64) words, no bits past out_f, at least one bit set
  EligibleGreedyContext.run :986-1150: 64-row tiles, one mask word each;
      an empty tile is skipped; a fully eligible tile is one producer run of
      all its rows; otherwise every maximal run of 4-row groups holding an
      eligible row is one producer run, computed whole (ineligible rows of a
      computed group are dotted but never candidates); a NaN among the
      eligible rows fails the call
  updateGreedyCandidate :1152-1163: value > best, or equal with a lower index
  runGreedyArgmaxEligible totals :1939-1966: skipped = out_f - producer,
      overcomputed = producer - eligible
Every failure is the reference's TensorError.ShapeMismatch.
"""
import numpy as np


class ShapeMismatch(Exception):
    pass


def eligible_rows(words, out_f):
    """validateEligibleWords: the eligible row count, or ShapeMismatch."""
    words = [int(w) for w in words]
    expected = out_f // 64 + (1 if out_f % 64 else 0)
    if expected == 0 or len(words) != expected:
        raise ShapeMismatch("word count")
    if out_f % 64 and words[-1] >> (out_f % 64):
        raise ShapeMismatch("bits past out_f")
    rows = sum(bin(w).count("1") for w in words)
    if rows == 0 or rows > out_f:
        raise ShapeMismatch("empty mask")
    return rows


def eligible_greedy(row_logits, out_f, words):
    """The reference's prehead walk. row_logits(start, end) returns the
    logits of rows start..end-1 (called only for the rows a producer run
    computes). Returns the EligibleGreedyResult fields as a dict."""
    n_eligible = eligible_rows(words, out_f)
    if out_f % 4:
        raise ShapeMismatch("rows4")
    best_v, best_i = None, None
    producer_rows = producer_runs = 0

    def consider(v, i):
        nonlocal best_v, best_i
        if best_v is None or v > best_v or (v == best_v and i < best_i):
            best_v, best_i = v, i

    for t in range(len(words)):
        row_start = 64 * t
        row_count = min(64, out_f - row_start)
        valid = (1 << 64) - 1 if row_count == 64 else (1 << row_count) - 1
        e = int(words[t]) & valid
        if e == 0:
            continue
        if e == valid:
            vals = np.asarray(row_logits(row_start, row_start + row_count), dtype=np.float32)
            if np.isnan(vals).any():  # the full-tile kernel reports any NaN
                raise ShapeMismatch("eligible NaN")
            for r in range(row_count):
                consider(float(vals[r]), row_start + r)
            producer_rows += row_count
            producer_runs += 1
            continue
        g = 0
        while g < row_count // 4:
            if (e >> (4 * g)) & 0xF == 0:
                g += 1
                continue
            run_start = g
            g += 1
            while g < row_count // 4 and (e >> (4 * g)) & 0xF:
                g += 1
            lo, hi = 4 * run_start, 4 * g
            vals = np.asarray(row_logits(row_start + lo, row_start + hi), dtype=np.float32)
            producer_rows += hi - lo
            producer_runs += 1
            for r in range(lo, hi):
                if not (e >> r) & 1:
                    continue
                v = float(vals[r - lo])
                if np.isnan(v):
                    raise ShapeMismatch("eligible NaN")
                consider(v, row_start + r)
    if best_i is None:
        raise ShapeMismatch("no candidate")
    return dict(token_index=best_i, eligible_rows=n_eligible, producer_rows=producer_rows,
                skipped_rows=out_f - producer_rows, overcomputed_rows=producer_rows - n_eligible,
                producer_runs=producer_runs)


def device_rows(words, out_f):
    """Rows a device that skips whole 16-row blocks streams: 16 per block
    holding an eligible row."""
    n = 0
    for b in range(out_f // 16):
        if (int(words[b // 4]) >> ((b % 4) * 16)) & 0xFFFF:
            n += 16
    return n
