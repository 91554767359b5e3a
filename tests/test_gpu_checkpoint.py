"""Paged-KV checkpoint page images of device sessions
(glacier_hip_session_encode_page_image / _restore_checkpoint): the images a
lane's HBM pages give are byte-identical to the oracle's encoding of the same
committed rows (oracle/page_image.py, continuation_paged_kv_restore.zig), a
restore remaps them onto fresh generations exactly as restoreCheckpointV1
does (paged_kv_cache.zig:608-762), and the restored lane continues decoding
with the tokens and bit-identical logits of the lane it was taken from."""
import numpy as np
import pytest

from oracle import page_image as pi
from oracle.paged_kv import Root

pytestmark = pytest.mark.gpu

TINY = dict(num_layers=2, dim=256, hidden_dim=512, num_heads=4, num_kv_heads=2, head_dim=64,
            vocab_size=4096, group_size=32, rms_eps=1e-6, rope_theta=1e6)
SEED = 0x43484B50
CHALLENGE = bytes(range(1, 33))
MAXPOS = 96


@pytest.fixture(scope="module")
def model(gh, gctx):
    host = gh.random_model_host(TINY, SEED)
    for L in host["layers"]:
        L["input_norm"] = (L["input_norm"] + 1.0).astype(np.float32)
        L["post_attn_norm"] = (L["post_attn_norm"] + 1.0).astype(np.float32)
    host["final_norm"] = (host["final_norm"] + 1.0).astype(np.float32)
    m = gh.Model(gctx, TINY)
    m.set_from_host(host)
    yield m
    m.close()


def _py_root(r):
    return Root(r.cache_instance, r.generation, r.committed_len, r.committed_pages,
                bytes(r.ownership_sha256))


def _run(sess, lane, prompt, n):
    toks = [sess.prefill(lane, prompt)]
    for _ in range(n):
        toks.append(int(sess.step([lane], [toks[-1]])[0]))
    return toks


def _canonical(sess, lane, page, rows):
    kvd = TINY["num_kv_heads"] * TINY["head_dim"]
    parts = []
    for l in range(TINY["num_layers"]):
        for v in (0, 1):
            for r in range(rows):
                parts.append(sess.kv_row(lane, l, v, 16 * page + r, kvd))
    return np.concatenate(parts).astype("<f4").tobytes()


@pytest.mark.parametrize("kv", ["f32", "f16"])
def test_images_match_oracle_and_restore_continues_identically(gh, model, kv):
    dt = gh.F32 if kv == "f32" else gh.F16
    sess = gh.Session(model, max_lanes=2, max_positions=MAXPOS, kv_dtype=dt)
    try:
        prompt = gh.synth_tokens(SEED, 1, TINY["vocab_size"], 21)
        sess.begin(0, seed=5)
        toks = _run(sess, 0, prompt, 16)  # 37 positions: pages of 16, 16, 5 rows
        src = sess.root(0)
        assert src.committed_len == 37 and src.committed_pages == 3
        print(f"checkpoint kv={kv} root gen={src.generation}", flush=True)
        images = []
        for p in range(3):
            img, info = sess.encode_page_image(0, p, CHALLENGE)
            rows = min(16, 37 - 16 * p)
            gen = sess.page_generation(0, p)
            want = pi.encode_canonical(_py_root(src), TINY["num_layers"],
                                       TINY["num_kv_heads"] * TINY["head_dim"], MAXPOS,
                                       (src.cache_instance, p, gen), rows,
                                       _canonical(sess, 0, p, rows), CHALLENGE)
            assert img == want
            assert info.committed_rows == rows and bytes(info.image_sha256) == want[-32:]
            images.append(img)
        # restore into lane 1 and continue both lanes with the same token
        restore, refs = sess.restore_checkpoint(1, images, CHALLENGE, seed=5)
        tgt = sess.root(1)
        oroot, orefs, _ = pi.restore(images, CHALLENGE, tgt.cache_instance, TINY["num_layers"],
                                     TINY["num_kv_heads"] * TINY["head_dim"], MAXPOS)
        assert _py_root(tgt) == oroot and _py_root(restore.target_root) == oroot
        assert _py_root(restore.source_root) == _py_root(src)
        assert tgt.cache_instance != src.cache_instance and tgt.generation == 2
        assert [(r.cache_instance, r.logical_page, r.ownership_generation) for r in refs] == orefs
        assert restore.restored_pages == 3 and restore.abi_version == pi.CHECKPOINT_RESTORE_ABI
        assert sess.kv_sha256(1) == sess.kv_sha256(0)
        last = toks[-1]
        a, b = [last], [last]
        for _ in range(8):
            na, la = sess.step([0], [a[-1]], want_logits=True)
            nb, lb = sess.step([1], [b[-1]], want_logits=True)
            a.append(int(na[0]))
            b.append(int(nb[0]))
            assert np.array_equal(la[0], lb[0])
        assert a == b
        # the restored lane's next root comes from generation 3 on
        assert sess.root(1).generation == 3 + 8 - 1
        # images of the restored lane carry the same rows under the new refs
        img1, info1 = sess.encode_page_image(1, 1, CHALLENGE)
        assert img1[208:-32] == images[1][208:-32]
        assert info1.source_ref.ownership_generation == 2
    finally:
        sess.close()


def test_restore_rejects_like_the_reference(gh, model):
    sess = gh.Session(model, max_lanes=3, max_positions=MAXPOS, kv_dtype=gh.F32)
    try:
        sess.begin(0, seed=1)
        _run(sess, 0, gh.synth_tokens(SEED, 2, TINY["vocab_size"], 20), 4)  # 24 positions
        sess.begin(2, seed=2)
        _run(sess, 2, gh.synth_tokens(SEED, 3, TINY["vocab_size"], 20), 4)
        imgs = [sess.encode_page_image(0, p, CHALLENGE)[0] for p in range(2)]
        other = [sess.encode_page_image(2, p, CHALLENGE)[0] for p in range(2)]

        def reason(images, challenge=CHALLENGE):
            with pytest.raises(gh.PageImageError) as e:
                sess.restore_checkpoint(1, images, challenge)
            r = sess.root(1)
            assert r.committed_len == 0 and r.generation == 1  # begun and empty
            return e.value.reason

        assert reason(imgs, bytes(range(2, 34))) == "InvalidPageImage"  # other challenge
        assert reason(imgs[::-1]) == "InvalidRestorePlan"               # out of order
        assert reason([imgs[0], other[1]]) == "ForeignCheckpoint"      # another lane's page
        assert reason(imgs[:1]) == "InvalidCheckpoint"                  # a page missing
        bad = bytearray(imgs[1])
        bad[300] ^= 1
        assert reason([imgs[0], bytes(bad)]) == "InvalidPageImage"      # corrupted rows
        # a valid f32 checkpoint whose values fp16 does not hold: an fp16
        # session refuses it rather than rounding
        s16 = gh.Session(model, max_lanes=1, max_positions=MAXPOS, kv_dtype=gh.F16)
        try:
            with pytest.raises(gh.PageImageError) as e:
                s16.restore_checkpoint(0, imgs, CHALLENGE)
            assert e.value.reason == "InvalidCheckpoint"
        finally:
            s16.close()
        # and the lane restores fine afterwards
        restore, _ = sess.restore_checkpoint(1, imgs, CHALLENGE)
        assert restore.target_root.committed_len == 24
    finally:
        sess.close()
