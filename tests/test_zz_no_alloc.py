"""glacier_hip_int4_gemv_noalloc (the GEMV entry point that allocates
nothing: its planes and split-K partial sums live in a fixed per-GPU array)
against glacier_hip_int4_gemv, through the C ABI, on two calls in a row with
the second smaller, for the GEMV (<= 2 rows) and GEMM (split-K) paths in Q8
and f32 activation modes. Bars as the GEMV tests: Q8 2e-6, f32 1e-5 of
max |y| (the two entry points run the same kernels; only a K split may
differ). The context's device bytes do not move across the calls."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _dev(gh, gctx):
    r, c = C.c_uint64(), C.c_uint64()
    assert gh.lib().glacier_hip_live_device_bytes(gctx.h, C.byref(r), C.byref(c)) == 0
    return r.value, c.value


@pytest.mark.parametrize("n,k,act,rows", [(4096, 4096, "q8", (5, 2)), (4608, 3584, "q8", (64, 24)),
                                          (3584, 18944, "f32", (16, 3)),
                                          (152064, 3584, "f32", (8, 1))])
def test_noalloc_gemv_equals_gemv(gh, gctx, n, k, act, rows):
    import torch

    L = gh.lib()
    seed = 0x4E41 + n + k
    packed = gh.synth_int4(seed, 1, n * k // 2)
    s16 = gh.synth_scales_f16(seed, 2, n * k // 32)
    w = gctx.weight(packed, s16, k, n)
    mode = gh.ACT_Q8 if act == "q8" else gh.ACT_F32
    bar = 2e-6 if act == "q8" else 1e-5
    try:
        for m in rows:  # second call smaller than the first
            x = torch.from_numpy(np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)).cuda()
            ref = torch.empty((m, n), dtype=torch.float32, device="cuda")
            got = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
            gh.check(L.glacier_hip_int4_gemv(gctx.h, w, x.data_ptr(), gh.F32, m, None, ref.data_ptr(),
                                            mode, None), "int4_gemv", gctx.h)
            gctx.sync()
            before = _dev(gh, gctx)
            print(f"noalloc {n}x{k} {act} m={m}", flush=True)
            gh.check(L.glacier_hip_int4_gemv_noalloc(gctx.h, w, x.data_ptr(), gh.F32, m, None,
                                                    got.data_ptr(), mode, None),
                     "int4_gemv_noalloc", gctx.h)
            gctx.sync()
            assert _dev(gh, gctx) == before
            r, g = ref.cpu().numpy(), got.cpu().numpy()
            err = float(np.max(np.abs(g - r)) / np.max(np.abs(r)))
            print(f"  rel {err:.2e}", flush=True)
            assert np.all(np.isfinite(g)) and err < bar
        # more rows than the fixed scratch holds: refused, output untouched
        x = torch.zeros((65, k), dtype=torch.float32, device="cuda")
        y = torch.full((65, n), 7.0, dtype=torch.float32, device="cuda")
        rc = L.glacier_hip_int4_gemv_noalloc(gctx.h, w, x.data_ptr(), gh.F32, 65, None, y.data_ptr(),
                                             mode, None)
        gctx.sync()
        assert rc == gh.SHAPE_MISMATCH and bool(torch.all(y == 7.0))
    finally:
        L.glacier_hip_int4_weight_destroy(w)
