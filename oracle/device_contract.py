"""Restatement of the reference's device capability contract.

TEST INFRASTRUCTURE ONLY: the checker for glacier_hip_device_capability_v1.
Only tests/ use it.

Follows /root/reference/src/core/device_capability_contract.zig:
  bit sets                      :58-114
  validateCapabilityShapeV1     :248-327
  validateCapabilityV1          :236-246
  capabilityRootV1              :329-350
  profileOperatorBitsV1 / profileElementTypeBitsV1 /
  profileNumericalPolicyBitsV1  :820-853
"""
import hashlib
import struct

CAPABILITY_ABI = 0x4744434100000001
BACKEND_KINDS = (1, 2, 3, 4)            # cpu, metal, portable_compute, provider
DEVICE_CLASSES = (1, 2)                 # cpu, accelerator

PROFILE_DEQUANT_INT4_F16, PROFILE_MATMUL_F16, PROFILE_MATVEC_INT4_F32 = 1, 2, 4
PROFILE_ALL = 7
OPERATOR_ALL = 7
ELEMENT_PACKED_INT4, ELEMENT_F16, ELEMENT_F32 = 1, 2, 4
ELEMENT_ALL = 7
POLICY_EXACT_INTEGER, POLICY_BOUNDED_F32, POLICY_BOUNDED_F16 = 1, 2, 4
POLICY_ALL = 7
(F_ALLOCATION, F_DISPATCH, F_COMPLETION_FENCE, F_PERSISTENT_WEIGHTS, F_COMMAND_BUFFER_TIME,
 F_ALLOCATED_BYTES, F_CANCELLATION, F_DEVICE_LOSS) = (1 << i for i in range(8))
FEATURE_ALL = 0xFF


def profile_operator_bits(p):
    r = 0
    if p & PROFILE_DEQUANT_INT4_F16:
        r |= 1
    if p & PROFILE_MATMUL_F16:
        r |= 2
    if p & PROFILE_MATVEC_INT4_F32:
        r |= 4
    return r


def profile_element_type_bits(p):
    r = 0
    if p & PROFILE_DEQUANT_INT4_F16:
        r |= ELEMENT_PACKED_INT4 | ELEMENT_F16
    if p & PROFILE_MATMUL_F16:
        r |= ELEMENT_F16
    if p & PROFILE_MATVEC_INT4_F32:
        r |= ELEMENT_PACKED_INT4 | ELEMENT_F32
    return r


def profile_numerical_policy_bits(p):
    r = 0
    if p & PROFILE_DEQUANT_INT4_F16:
        r |= POLICY_BOUNDED_F16
    if p & PROFILE_MATMUL_F16:
        r |= POLICY_BOUNDED_F16
    if p & PROFILE_MATVEC_INT4_F32:
        r |= POLICY_BOUNDED_F32
    return r


def capability_root_v1(c):
    h = hashlib.sha256(b"glacier-device-capability-v1\x00")
    for f in ("abi_version", "backend_kind", "device_class", "operation_profile_bits",
              "operator_bits", "element_type_bits", "numerical_policy_bits", "feature_bits",
              "max_single_allocation_bytes", "max_total_device_bytes", "max_queue_slots"):
        h.update(struct.pack("<Q", getattr(c, f)))
    for f in ("backend_sha256", "device_sha256", "driver_sha256", "placement_sha256"):
        h.update(bytes(getattr(c, f)))
    return h.digest()


def shape_errors(c):
    """The conditions of validateCapabilityShapeV1 that the record violates."""
    bad = []
    zero = bytes(32)
    if c.abi_version != CAPABILITY_ABI:
        bad.append("abi")
    if c.backend_kind not in BACKEND_KINDS or c.device_class not in DEVICE_CLASSES:
        bad.append("kind/class")
    for f, allowed in (("operation_profile_bits", PROFILE_ALL), ("operator_bits", OPERATOR_ALL),
                       ("element_type_bits", ELEMENT_ALL), ("numerical_policy_bits", POLICY_ALL),
                       ("feature_bits", FEATURE_ALL)):
        v = getattr(c, f)
        if v == 0 or v & ~allowed:
            bad.append(f)
    for f in ("backend_sha256", "device_sha256", "placement_sha256"):
        if bytes(getattr(c, f)) == zero:
            bad.append(f)
    p = c.operation_profile_bits
    if (c.operator_bits != profile_operator_bits(p) or
            c.element_type_bits != profile_element_type_bits(p) or
            c.numerical_policy_bits != profile_numerical_policy_bits(p)):
        bad.append("profile-derived bits")
    if (c.backend_kind == 1) != (c.device_class == 1):
        bad.append("cpu kind/class")
    if (c.max_single_allocation_bytes and c.max_total_device_bytes and
            c.max_single_allocation_bytes > c.max_total_device_bytes):
        bad.append("ceilings")
    f = c.feature_bits
    for feat, needs in ((F_DISPATCH, F_ALLOCATION), (F_COMPLETION_FENCE, F_DISPATCH),
                        (F_PERSISTENT_WEIGHTS, F_ALLOCATION), (F_COMMAND_BUFFER_TIME,
                                                               F_COMPLETION_FENCE),
                        (F_ALLOCATED_BYTES, F_ALLOCATION), (F_CANCELLATION, F_DISPATCH),
                        (F_DEVICE_LOSS, F_DISPATCH)):
        if f & feat and not f & needs:
            bad.append(f"feature {feat:#x} without {needs:#x}")
    return bad


def validate_capability_v1(c):
    """[] when validateCapabilityV1 accepts the record."""
    bad = shape_errors(c)
    if bytes(c.capability_sha256) == bytes(32) or bytes(c.capability_sha256) != capability_root_v1(c):
        bad.append("capability_sha256")
    return bad
