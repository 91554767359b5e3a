"""The host C++ of the runtime under sanitizers: the LaneWeave scheduler,
the paged-KV page map and row transactions, the publication digests, the
page-image codec and the prepared runtime image reader (csrc/*.cpp, the
code that runs on the host around the device kernels) are compiled with
g++ under AddressSanitizer + UndefinedBehaviorSanitizer, and the scheduler's
concurrent mode under ThreadSanitizer, together with the exerciser in
tests/native/host_sanitize.cpp, which drives the same C ABI the device
library exports through random traces and malformed inputs and checks each
module's invariants. SHA-256 and the fp16 conversions are also compared
with hashlib and numpy. CPU only."""
import hashlib
import os
import random
import shutil
import struct
import subprocess

import numpy as np
import pytest

from oracle import runtime_image as ri
from glrt_images import int4_record, raw_record, reference_test_config, repair_crcs

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "glacier-engine_amd", "csrc")
HOST_SOURCES = ["host_util.cpp", "lane_weave.cpp", "paged_kv.cpp", "publication.cpp",
                "runtime_image.cpp", "page_image.cpp", "lease_bank.cpp", "leased_kv.cpp"]
ENV = dict(os.environ, ASAN_OPTIONS="halt_on_error=1:detect_leaks=1",
           UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
           TSAN_OPTIONS="halt_on_error=1")


def _build(out, flags):
    cmd = (["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-Wall",
            "-I", os.path.join(ROOT, "include"), "-I", CSRC] + flags +
           [os.path.join(ROOT, "tests", "native", "host_sanitize.cpp")] +
           [os.path.join(CSRC, s) for s in HOST_SOURCES] + ["-o", out, "-lpthread"])
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    return out


@pytest.fixture(scope="module")
def binaries(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    d = tmp_path_factory.mktemp("host_sanitize")
    asan = _build(str(d / "asan"), ["-fsanitize=address,undefined", "-fno-sanitize-recover=all"])
    tsan = _build(str(d / "tsan"), ["-fsanitize=thread"])
    return asan, tsan


def _run(binary, *args, timeout=240):
    r = subprocess.run([binary] + [str(a) for a in args], capture_output=True, text=True,
                       env=ENV, timeout=timeout)
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-6000:])
    assert "runtime error" not in r.stderr and "Sanitizer" not in r.stderr, r.stderr[-6000:]
    return r.stdout


def test_sha256_matches_hashlib(binaries):
    out = _run(binaries[0], "sha", 300).split()
    assert len(out) == 300
    for n, h in enumerate(out):
        buf = bytes((i * 131 + 7) & 0xFF for i in range(n))
        assert h == hashlib.sha256(buf).hexdigest(), n


def test_fp16_conversions_match_numpy(binaries, tmp_path):
    path = tmp_path / "f16.bin"
    _run(binaries[0], "f16", path)
    words = np.fromfile(path, np.uint32)
    halves = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    got = words[:65536].view(np.float32)
    nan = np.isnan(halves)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), halves[~nan].view(np.uint32))
    pairs = words[65536:].reshape(-1, 2)
    src = pairs[:, 0].view(np.float32)
    with np.errstate(over="ignore"):
        want = src.astype(np.float16)  # IEEE round to nearest even, overflow to inf
    have = pairs[:, 1].astype(np.uint16).view(np.float16)
    wnan = np.isnan(want)
    assert np.array_equal(np.isnan(have), wnan)
    assert np.array_equal(have[~wnan].view(np.uint16), want[~wnan].view(np.uint16))


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_lane_weave_traces(binaries, seed):
    out = _run(binaries[0], "laneweave", seed, 3000)
    counts = dict(kv.split("=") for kv in out.split())
    assert int(counts["admitted"]) > 100 and int(counts["waves"]) > 100
    assert int(counts["failed_waves"]) > 10


@pytest.mark.parametrize("seed", [1, 2])
def test_paged_kv_transactions_and_page_images(binaries, seed):
    out = _run(binaries[0], "pagedkv", seed, 3000)
    counts = dict(kv.split("=") for kv in out.split())
    for k in ("commits", "aborts", "resets", "images", "decoded", "refused"):
        assert int(counts[k]) > 0, k


def test_lane_weave_concurrent_callers_under_tsan(binaries):
    _run(binaries[1], "threads", 5, 3000)
    _run(binaries[0], "threads", 6, 3000)


def _images(tmp_path):
    src = ri.fingerprint(b"sanitizer-source")
    cfg = reference_test_config()
    packed = np.arange(64, dtype=np.uint8)
    recs = [raw_record(0, "final_norm", [1.25, -2.5, 3.75, 4.0]),
            int4_record(0, "attn_q", packed, 4, 32, scales_f32=np.full(4, 0.5, np.float32),
                        scales_f16=np.full(4, 0.5, np.float16)),
            int4_record(1, "mlp_up", packed, 8, 16, scales_f32=np.full(8, 0.25, np.float32),
                        group=16),
            raw_record(ri.GLOBAL_LAYER, "input_norm", np.linspace(0, 1, 16))]
    v2 = tmp_path / "valid_v2.glrt"
    data2 = ri.write_image(str(v2), cfg, src, recs)
    v1 = tmp_path / "valid_v1.glrt"
    ri.write_image_v1(str(v1), cfg, src, [(0, ri.KIND["final_norm"], [1.5, -2.0, 3.25, 4.5]),
                                          (1, ri.KIND["input_norm"], [0.5] * 16)])
    data1 = v1.read_bytes()
    return [str(v2), str(v1)], [(data2, 2), (data1, 1)]


def test_runtime_image_reader_on_edited_images(binaries, tmp_path):
    valid, datas = _images(tmp_path)
    rng = random.Random(0x5A11)
    edited = []
    for i in range(240):
        data, version = datas[i % 2]
        b = bytearray(data)
        count = struct.unpack_from("<Q", b, 16)[0]
        rsz = ri.RECORD_SIZE if version == 2 else ri.V1_RECORD_SIZE
        end = ri.HEADER_SIZE + count * rsz
        for _ in range(rng.randint(1, 3)):
            # an index or header field: small, huge or random (CRCs repaired,
            # so the descriptor, bounds and overlap checks run)
            off = rng.randrange(ri.HEADER_SIZE if rng.random() < 0.7 else 0, end - 8) & ~3
            v = rng.choice([rng.randrange(64), (1 << 64) - 1 - rng.randrange(4096),
                            rng.getrandbits(64), len(b) - rng.randrange(128)])
            width = rng.choice([4, 8])
            struct.pack_into("<Q" if width == 8 else "<I", b, off, v & ((1 << (8 * width)) - 1))
        b = repair_crcs(bytes(b), version)
        if rng.random() < 0.2:
            b = b[:rng.randrange(len(b))]
        p = tmp_path / f"edited_{i}.glrt"
        p.write_bytes(b)
        edited.append(str(p))
    out = _run(binaries[0], "glrt", 7, tmp_path, len(valid), *valid, *edited)
    counts = dict(kv.split("=") for kv in out.split()[1:])
    opened, rejected = int(counts["opened"]), int(counts["rejected"])
    print(f"edited images: {opened} opened, {rejected} rejected")
    assert opened > 0 and rejected > 0


def test_leased_page_maps_under_asan_ubsan_and_tsan(binaries):
    """Leased page maps (lease_bank.cpp, leased_kv.cpp) under random rows,
    aborts, pool limits, seals, reclaims and renewals: the tree's charge equals
    the live bindings and the pages the maps hold after every step; four trees
    on one bank from four threads under ThreadSanitizer."""
    for seed in (1, 2, 3):
        out = _run(binaries[0], "lease", seed, 3000, 1)
        assert int(out.split("lease_ops=")[1]) == 3000
    out = _run(binaries[1], "lease", 9, 1500, 4)
    assert int(out.split("lease_ops=")[1]) == 6000
