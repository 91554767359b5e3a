"""CPU-side checks of the C ABI: the library loads, exports every symbol that
include/glacier_hip.h declares, rejects bad arguments without a device, and
the synthetic generator is deterministic with the documented statistics."""
import os
import re
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "glacier_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(glacier_hip_[a-z0-9_]+)\s*\(", text)))


def test_header_declarations_are_exported(gh):
    out = subprocess.run(["nm", "-D", "--defined-only", gh.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\s[TW]\s(glacier_hip_\w+)", out))
    missing = [s for s in _declared() if s not in exported]
    assert not missing, missing
    assert set(_declared()) == set(gh.exported_symbols())


def test_header_is_c_only():
    # a Zig @cImport needs plain C: compile it with the C compiler, pedantic
    r = subprocess.run(["gcc", "-std=c11", "-pedantic", "-Wall", "-Werror", "-fsyntax-only", "-x",
                        "c", HEADER], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_abi_version(gh):
    assert gh.lib().glacier_hip_abi_version() == 0x4748495000000001


def test_null_handles_rejected_without_device(gh):
    L = gh.lib()
    assert L.glacier_hip_deinit(None) == gh.INVALID_HANDLE
    assert L.glacier_hip_synchronize(None) == gh.INVALID_HANDLE
    assert L.glacier_hip_int4_gemv(None, None, None, 0, 1, None, None, 0, None) == gh.INVALID_HANDLE
    assert L.glacier_hip_session_lane_begin(None, 0, 0) == gh.INVALID_HANDLE
    assert L.glacier_hip_argmax(None, None, 4, 1, None, None) == gh.INVALID_ARGUMENT


def test_synth_deterministic_and_distributed(gh):
    a = gh.synth_int4(1, 2, 1 << 16)
    b = gh.synth_int4(1, 2, 1 << 16)
    c = gh.synth_int4(1, 3, 1 << 16)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    nib = np.concatenate([a & 15, a >> 4])
    counts = np.bincount(nib, minlength=16)
    assert counts.min() > 0.9 * nib.size / 16 and counts.max() < 1.1 * nib.size / 16
    s = gh.synth_scales_f16(1, 4, 1 << 16).view(np.float16).astype(np.float64)
    assert (s >= 0).all() and abs(s.mean() - 0.02 * np.sqrt(2 / np.pi)) < 5e-4
    z = gh.synth_normal_f32(9, 9, 1 << 16).astype(np.float64)
    assert abs(z.mean()) < 5e-4 and abs(z.std() - 0.02) < 5e-4
    t = gh.synth_tokens(3, 3, 151936, 4096)
    assert t.max() < 151936 and len(set(t.tolist())) > 4000


def test_f16_helper_matches_numpy(gh):
    for v in (0x3C00, 0x0001, 0x7BFF, 0x8000, 0xC500):
        assert gh.lib().glacier_hip_f16_to_f32(v) == np.uint16(v).view(np.float16).astype(np.float32)
