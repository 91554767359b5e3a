"""Decoding an oracle fixture's own greedy sequence on the device: the
prompt is prefilled, then step s is fed the oracle's token s - 1, so the
device and the oracle see the same context at every step and their logits
are comparable at all of them, however a near tie resolves on either side.
Used by the Q8 parity tests of the 7B-geometry and C1 models."""
import numpy as np


def logit_err(got, fx, i):
    """max |device - oracle| over the fixture's sampled and top-32 indices of
    step i, over the oracle's max |logit| of that step."""
    return max(np.max(np.abs(got[fx["sample_idx"]] - fx["sample_logits"][i])),
               np.max(np.abs(got[fx["top_idx"][i]] - fx["top_val"][i]))) / fx["max_abs"][i]


def forced_decode(sess, fx):
    """Returns (per-step logit errors, near-tie list) over every stored step.

    A step whose device token differs from the oracle's is listed as
    (step, oracle top-2 gap, device deviation on the oracle's two best
    entries); the caller asserts each is a near tie (gap < 2 * deviation)."""
    want = fx["tokens"].tolist()
    n = len(want)
    assert fx["steps"].tolist() == list(range(n))
    sess.begin(0)
    first, lg = sess.prefill(0, fx["prompt"], want_logits=True)
    got, logits = [first], [lg]
    for s in range(1, n):
        nxt, lg = sess.step([0], [want[s - 1]], want_logits=True)
        got.append(int(nxt[0]))
        logits.append(lg[0])
    errs = [logit_err(logits[s], fx, s) for s in range(n)]
    ties = []
    for s in range(n):
        if got[s] != want[s]:
            dev = float(np.max(np.abs(logits[s][fx["top_idx"][s, :2]] - fx["top_val"][s, :2])))
            ties.append((s, float(fx["top2_gap"][s]), dev))
    return errs, ties


def check_against_sensitivity(errs, ties, fx, label):
    """The bar for a Q8 run of a random model: 1e-2 max-relative, or twice
    the oracle's own one-ulp sensitivity (fx["ulp_sensitivity"]: the oracle
    fed the same tokens with the prompt's embedding rows one ulp off) where
    that is larger -- in the worst step and on average; a differing greedy
    token only at near ties, and not many more of them than the oracle's
    own one-ulp run has (fx["ulp_argmax_moved"])."""
    sens = fx["ulp_sensitivity"]
    moved = len(fx["ulp_argmax_moved"])
    bar_max = max(1e-2, 2 * float(sens.max()))
    bar_mean = max(2.5e-3, 2 * float(sens.mean()))
    print(f"{label}: logit max-rel max {max(errs):.2e} mean {np.mean(errs):.2e} (oracle one-ulp "
          f"sensitivity max {sens.max():.2e} mean {sens.mean():.2e}); greedy token differs at "
          f"{len(ties)} steps {ties} (the one-ulp oracle run at {moved})", flush=True)
    assert max(errs) < bar_max
    assert np.mean(errs) < bar_mean
    assert all(gap < 2 * dev for _, gap, dev in ties)
    assert len(ties) <= max(4, 3 * moved)
