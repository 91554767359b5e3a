"""BASELINE config 2 on the GPU: the INT4 GEMV / GEMM at the five Llama/Qwen-7B
decode shapes, M = 1, 2, 4, 8, Q8 and f32 activation semantics, f32 and bf16
activation inputs, through glacier_hip_int4_gemv, against the oracle.

The device runs the full matrix (so every launch plan is the real one for
that shape); the oracle computes a sample of 416 output rows (rows are
independent: the first and last 16 and 384 seeded random rows) from the same
packed codes and fp16 scales.

Bars (max |gpu - oracle| over the sampled rows / max |oracle|): Q8 2e-6 (exact
integer group dots, only the across-group f32 order differs); f32 1e-5 (three
7-bit digit planes); BASELINE's own bar is 1e-3. bf16 inputs are compared with
the oracle on the bf16 values widened to f32.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SHAPES = [(4096, 4096), (11008, 4096), (4096, 11008), (18944, 3584), (152064, 3584)]
_W = {}


@pytest.fixture(scope="module")
def weights(gh, gctx):
    yield _W
    for w, *_ in _W.values():
        gh.lib().glacier_hip_int4_weight_destroy(w)
    _W.clear()


def _get(gh, gctx, weights, n, k):
    if (n, k) not in weights:
        seed = 0x474C4143 + n + k
        packed = gh.synth_int4(seed, 1, n * k // 2)
        s16 = gh.synth_scales_f16(seed, 2, n * k // 32)
        w = gctx.weight(packed, s16, k, n)
        rng = np.random.default_rng(n ^ k)
        rows = np.unique(np.concatenate([np.arange(16), np.arange(n - 16, n),
                                         rng.choice(n, 384, replace=False)]))
        sub_p = np.ascontiguousarray(packed.reshape(n, k // 2)[rows]).reshape(-1)
        sub_s = np.ascontiguousarray(s16.view(np.float16).astype(np.float32)
                                     .reshape(n, k // 32)[rows]).reshape(-1)
        weights[(n, k)] = (w, rows, sub_p, sub_s)
    return weights[(n, k)]


@pytest.mark.parametrize("n,k", SHAPES)
@pytest.mark.parametrize("m", [1, 2, 4, 8])
@pytest.mark.parametrize("act", ["q8", "f32"])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_c2_shape_matches_oracle(gh, gctx, ora, weights, n, k, m, act, xdt):
    import torch

    w, rows, sub_p, sub_s = _get(gh, gctx, weights, n, k)
    x = np.random.default_rng(1000 * m + k).standard_normal((m, k)).astype(np.float32)
    if xdt == "bf16":
        xd = torch.from_numpy(x).to(torch.bfloat16).cuda()
        x = xd.float().cpu().numpy()
    else:
        xd = torch.from_numpy(x).cuda()
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    mode = gh.ACT_Q8 if act == "q8" else gh.ACT_F32
    print(f"case {n}x{k} m={m} {act} x={xdt}", flush=True)
    rc = gh.lib().glacier_hip_int4_gemv(gctx.h, w, xd.data_ptr(), gh.BF16 if xdt == "bf16" else gh.F32,
                                        m, None, y.data_ptr(), mode, None)
    gh.check(rc, "int4_gemv", gctx.h)
    gctx.sync()
    got = y.cpu().numpy()[:, rows]
    fn = ora.linear_int4_q8 if act == "q8" else ora.linear_int4_f32
    want = fn(x, sub_p, sub_s, rows.size, k, 32)
    err = float(np.max(np.abs(got - want)) / np.max(np.abs(want)))
    print(f"  rel {err:.2e}", flush=True)
    assert err < (2e-6 if act == "q8" else 1e-5)
