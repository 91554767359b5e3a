"""Projections on two streams of one context (glacier_hip_int4_gemv with a
caller stream): each stream has its own activation planes and split-K
partial sums, so calls queued on two streams without a synchronisation in
between give exactly the outputs each gives alone (the GEMV's planes at 1
row, the GEMM's planes and partial sums at 8 rows)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m", [1, 8])
def test_two_streams_do_not_share_scratch(gh, gctx, m):
    import torch

    out_f, in_f = 4096, 4096
    packed = gh.synth_int4(77, 1, out_f * in_f // 2)
    s16 = gh.synth_scales_f16(77, 2, out_f * in_f // 32)
    w = gctx.weight(packed, s16, in_f, out_f)
    try:
        rng = np.random.default_rng(m)
        xs = [torch.from_numpy(rng.standard_normal((m, in_f)).astype(np.float32)).cuda()
              for _ in range(2)]
        streams = [torch.cuda.Stream(), torch.cuda.Stream()]
        torch.cuda.synchronize()

        def run(i, y):
            rc = gh.lib().glacier_hip_int4_gemv(gctx.h, w, xs[i].data_ptr(), gh.F32, m, None,
                                                y.data_ptr(), gh.ACT_Q8, streams[i].cuda_stream)
            gh.check(rc, "int4_gemv", gctx.h)

        alone = []
        for i in range(2):
            y = torch.empty((m, out_f), dtype=torch.float32, device="cuda")
            run(i, y)
            streams[i].synchronize()
            alone.append(y.cpu().numpy())
        assert not np.array_equal(alone[0], alone[1])
        print(f"two streams m={m}", flush=True)
        ys = [[torch.empty((m, out_f), dtype=torch.float32, device="cuda") for _ in range(2)]
              for _ in range(6)]
        for r in range(6):  # interleaved, no synchronisation between the calls
            run(0, ys[r][0])
            run(1, ys[r][1])
        torch.cuda.synchronize()
        for r in range(6):
            for i in range(2):
                assert np.array_equal(ys[r][i].cpu().numpy(), alone[i]), (r, i)
    finally:
        gh.lib().glacier_hip_int4_weight_destroy(w)
