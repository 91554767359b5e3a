"""Writes tests/golden/digests.json: input/output vectors of three digests
the reference restates in stdlib-only Python beside its Zig code:

* tokenSequenceSha256 (generate.zig:3193-3203) as
  `derive_output_token_sha256` (bench/lane4_event_evidence.py:428-442);
* logicalKvPrefixSha256 (generate.zig:3150-3172, paged twin
  paged_kv_cache.zig:1347-1350) as `logical_kv_root`
  (bench/prepared_text_checkpoint.py:123-140) over the canonical
  [layer][K, V][position][kv_dim] little-endian f32 payload;
* capabilityRootV1 (device_capability_contract.zig) as `capability_root`
  (bench/device_capability_contract.py:270-293).

Run in the build container only (the GPU box has no /root/reference):
    python tests/golden/make_digest_golden.py
The reference modules are imported read-only to compute the expected
digests; only the vectors (inputs and digests) are written. Inputs are
seeded and include the edge cases the digests must keep apart: empty and
u32-max token lists, -0.0 / NaN / inf bit patterns in the KV payload, and
zero / all-ones capability fields.
"""
import importlib.util
import json
import os
import random
import struct
import sys

REF_BENCH = "/root/reference/bench"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "digests.json")


def _load(name):
    spec = importlib.util.spec_from_file_location(name, os.path.join(REF_BENCH, name + ".py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod  # dataclasses resolve their module by name
    spec.loader.exec_module(mod)
    return mod


def token_cases(rng):
    cases = [[], [0], [1, 2, 3], [0xFFFFFFFF], [0xFFFFFFFF, 0, 0x80000000]]
    cases.append([rng.randrange(152064) for _ in range(128)])
    cases.append([rng.randrange(1 << 32) for _ in range(37)])
    return cases


def kv_cases(rng):
    specials = [0x80000000, 0x7FC00000, 0x7F800000, 0xFF800000, 0x00000001, 0x3F800000]
    out = []
    for layers, kv_dim, positions in ((1, 1, 1), (2, 8, 3), (3, 16, 17), (2, 128, 2)):
        words = [rng.getrandbits(32) for _ in range(layers * 2 * positions * kv_dim)]
        for i, s in enumerate(specials):
            if i < len(words):
                words[(i * 7) % len(words)] = s
        out.append((layers, kv_dim, positions, struct.pack(f"<{len(words)}I", *words)))
    return out


def capability_cases(mod, rng):
    fields = ("abi_version", "backend_kind", "device_class", "operation_profile_bits",
              "operator_bits", "element_type_bits", "numerical_policy_bits", "feature_bits",
              "max_single_allocation_bytes", "max_total_device_bytes", "max_queue_slots")
    digests = ("backend_sha256", "device_sha256", "driver_sha256", "placement_sha256")
    cases = [mod.DeviceCapabilityV1()]
    cases.append(mod.DeviceCapabilityV1(**{f: (1 << 64) - 1 for f in fields},
                                        **{d: b"\xff" * 32 for d in digests}))
    for _ in range(3):
        kw = {f: rng.getrandbits(rng.choice((3, 16, 40, 64))) for f in fields}
        kw.update({d: bytes(rng.getrandbits(8) for _ in range(32)) for d in digests})
        cases.append(mod.DeviceCapabilityV1(**kw))
    rows = []
    for c in cases:
        rec = {f: getattr(c, f) for f in fields}
        rec.update({d: getattr(c, d).hex() for d in digests})
        rows.append((rec, mod.capability_root(c).hex()))
    return rows


def main():
    ev = _load("lane4_event_evidence")
    ck = _load("prepared_text_checkpoint")
    dc = _load("device_capability_contract")
    rng = random.Random(0x444947)
    golden = {
        "token_sequence": [{"tokens": t, "sha256": ev.derive_output_token_sha256(t)}
                           for t in token_cases(rng)],
        "logical_kv": [{"num_layers": L, "kv_dim": d, "positions": p, "payload_hex": b.hex(),
                        "sha256": ck.logical_kv_root(L, d, p, b).hex()}
                       for L, d, p, b in kv_cases(rng)],
        "capability": [{"record": r, "sha256": h} for r, h in capability_cases(dc, rng)],
    }
    with open(OUT, "w") as f:
        json.dump(golden, f, indent=1)
        f.write("\n")
    print("wrote", OUT, {k: len(v) for k, v in golden.items()})


if __name__ == "__main__":
    main()
