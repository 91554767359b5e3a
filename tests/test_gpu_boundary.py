"""The device boundary's contracts through the C ABI:

  * capability (device_capability_contract.zig): the record the backend
    emits passes validateCapabilityV1 restated in oracle/device_contract.py
    (shape rules :248-327, capabilityRootV1 :329-350), with the profile-
    derived operator / element / policy bits;
  * allocation lease AdapterV1 (device_allocation_lease.zig:323-348): quote
    is replay-safe and side-effect free, a failed allocate creates nothing, a
    foreign or tampered quote is refused, release returns live counts to zero;
  * asynchronous registered dispatch (backend.zig:600-668, shim.m): submit ->
    poll / wait -> output read -> finalize, the binding and exact-completion
    checks, buffers pinned by a live command, live_command_count.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import device_contract as dc

pytestmark = pytest.mark.gpu


def test_capability_record_passes_reference_validation(gh, gctx):
    cap = gh.Capability()
    assert gh.lib().glacier_hip_device_capability_v1(gctx.h, C.byref(cap)) == 0
    assert dc.validate_capability_v1(cap) == []
    assert bytes(cap.capability_sha256) == dc.capability_root_v1(cap)
    assert (cap.backend_kind, cap.device_class) == (3, 2)  # portable_compute accelerator
    assert cap.operation_profile_bits & dc.PROFILE_MATVEC_INT4_F32
    assert cap.max_single_allocation_bytes <= cap.max_total_device_bytes
    # deterministic: a second emission is byte-identical
    cap2 = gh.Capability()
    assert gh.lib().glacier_hip_device_capability_v1(gctx.h, C.byref(cap2)) == 0
    assert bytes(cap2) == bytes(cap)
    # the oracle's validator is not vacuous: a tampered record fails it
    cap2.feature_bits |= dc.F_CANCELLATION
    assert dc.validate_capability_v1(cap2) == ["capability_sha256"]
    cap2.operator_bits = 1
    assert "profile-derived bits" in dc.shape_errors(cap2)


def _count(gh, gctx):
    v = C.c_uint64()
    assert gh.lib().glacier_hip_live_buffer_count(gctx.h, C.byref(v)) == 0
    return v.value


def test_allocation_lease_quote_allocate_free(gh, gctx):
    L = gh.lib()
    base = _count(gh, gctx)
    q1, q2 = gh.AllocationQuote(), gh.AllocationQuote()
    assert L.glacier_hip_allocation_quote(gctx.h, 3 << 20, C.byref(q1)) == 0
    assert L.glacier_hip_allocation_quote(gctx.h, 3 << 20, C.byref(q2)) == 0
    assert bytes(q1) == bytes(q2) and _count(gh, gctx) == base  # replay-safe, no side effect
    assert q1.charged_bytes >= q1.requested_bytes and q1.charged_bytes % (2 << 20) == 0
    # a tampered quote (charge below the granularity rounding) and a foreign one are refused
    bad = gh.AllocationQuote(q1.requested_bytes, q1.charged_bytes - 1, q1.context_epoch)
    tok = gh.BufferToken()
    assert L.glacier_hip_allocation_allocate(gctx.h, C.byref(bad), C.byref(tok)) == gh.INVALID_ARGUMENT
    bad = gh.AllocationQuote(q1.requested_bytes, q1.charged_bytes, q1.context_epoch ^ 1)
    assert L.glacier_hip_allocation_allocate(gctx.h, C.byref(bad), C.byref(tok)) == gh.INVALID_ARGUMENT
    assert _count(gh, gctx) == base
    # beyond the device's memory there is no quote; a quote of the whole
    # memory (some of it is in use) fails at allocate and creates nothing
    huge = gh.AllocationQuote()
    assert L.glacier_hip_allocation_quote(gctx.h, 1 << 50, C.byref(huge)) == gh.OUT_OF_MEMORY
    total = gctx.info().total_global_bytes
    assert L.glacier_hip_allocation_quote(gctx.h, total, C.byref(huge)) == 0
    rc = L.glacier_hip_allocation_allocate(gctx.h, C.byref(huge), C.byref(tok))
    if rc == 0:  # the device had it all free: the lease is ordinary
        assert _count(gh, gctx) == base + 1
        assert L.glacier_hip_allocation_free(gctx.h, C.byref(tok)) == 0
    else:
        assert rc == gh.OUT_OF_MEMORY
    assert _count(gh, gctx) == base
    # allocate -> info -> free
    assert L.glacier_hip_allocation_allocate(gctx.h, C.byref(q1), C.byref(tok)) == 0
    assert _count(gh, gctx) == base + 1 and tok.charged_bytes == q1.charged_bytes
    info = gh.BufferInfo()
    assert L.glacier_hip_buffer_info(gctx.h, C.byref(tok), C.byref(info)) == 0
    assert info.device_address != 0 and info.requested_bytes == 3 << 20
    assert L.glacier_hip_allocation_free(gctx.h, C.byref(tok)) == 0
    assert L.glacier_hip_allocation_free(gctx.h, C.byref(tok)) == gh.INVALID_HANDLE
    assert _count(gh, gctx) == base


def _buffers(gh, gctx, sizes):
    toks = []
    for n in sizes:
        t = gh.BufferToken()
        assert gh.lib().glacier_hip_buffer_create(gctx.h, n, C.byref(t)) == 0
        toks.append(t)
    return toks


def test_async_registered_dispatch(gh, gctx, ora):
    L = gh.lib()
    out_f, in_f = 4096, 3584
    packed = gh.synth_int4(77, 1, out_f * in_f // 2)
    scales = gh.synth_scales_f16(77, 2, out_f * in_f // 32).view(np.float16).astype(np.float32)
    x = np.random.default_rng(5).standard_normal(in_f).astype(np.float32)
    toks = _buffers(gh, gctx, [out_f * in_f // 2, scales.size * 4, in_f * 4, out_f * 4])
    binding = (C.c_uint8 * 32)(*range(1, 33))
    sub = gh.AsyncSubmission()
    rc = L.glacier_hip_int4_registered_buffers_submit_async(
        gctx.h, C.byref(toks[0]), C.byref(toks[1]), C.byref(toks[2]), C.byref(toks[3]),
        packed.ctypes.data, packed.size, scales.ctypes.data, scales.size, x.ctypes.data, in_f, 32,
        in_f, out_f, binding, C.byref(sub))
    assert rc == 0 and sub.disposition == 1 and sub.token.generation != 0
    n = C.c_uint64()
    assert L.glacier_hip_live_command_count(gctx.h, C.byref(n)) == 0 and n.value == 1
    comp = gh.AsyncCompletion()
    assert L.glacier_hip_registered_dispatch_poll(gctx.h, C.byref(sub.token), binding,
                                                 C.byref(comp)) == 0
    assert comp.state in (gh.COMMAND_PENDING, gh.COMMAND_COMPLETED)
    # a live command pins its buffers
    assert L.glacier_hip_buffer_release(gctx.h, C.byref(toks[3])) == gh.BUSY
    # a different binding names no command
    other = (C.c_uint8 * 32)(*([7] * 32))
    assert L.glacier_hip_registered_dispatch_wait(gctx.h, C.byref(sub.token), other,
                                                 C.byref(comp)) == gh.INVALID_HANDLE
    assert L.glacier_hip_registered_dispatch_wait(gctx.h, C.byref(sub.token), binding,
                                                 C.byref(comp)) == 0
    assert comp.state == gh.COMMAND_COMPLETED and comp.gpu_end_time >= comp.gpu_start_time > 0
    again = gh.AsyncCompletion()
    assert L.glacier_hip_registered_dispatch_poll(gctx.h, C.byref(sub.token), binding,
                                                 C.byref(again)) == 0
    assert bytes(again) == bytes(comp)  # the completion record is fixed once observed
    y = np.empty(out_f, np.float32)
    assert L.glacier_hip_int4_registered_output_read(gctx.h, C.byref(sub.token), binding,
                                                    C.byref(comp), C.byref(toks[2]),
                                                    y.ctypes.data, out_f) == gh.SHAPE_MISMATCH
    assert L.glacier_hip_int4_registered_output_read(gctx.h, C.byref(sub.token), binding,
                                                    C.byref(comp), C.byref(toks[3]),
                                                    y.ctypes.data, out_f) == 0
    want = ora.linear_int4_f32(x, packed, scales, out_f, in_f, 32)[0]
    assert np.max(np.abs(y - want)) / np.max(np.abs(want)) < 1e-5
    # finalize needs the exact completion record
    wrong = gh.AsyncCompletion.from_buffer_copy(bytes(comp))
    wrong.gpu_end_time += 1.0
    assert L.glacier_hip_registered_dispatch_finalize(gctx.h, C.byref(sub.token), binding,
                                                     C.byref(wrong)) == gh.INVALID_TRANSACTION
    assert L.glacier_hip_registered_dispatch_finalize(gctx.h, C.byref(sub.token), binding,
                                                     C.byref(comp)) == 0
    assert L.glacier_hip_live_command_count(gctx.h, C.byref(n)) == 0 and n.value == 0
    assert L.glacier_hip_registered_dispatch_poll(gctx.h, C.byref(sub.token), binding,
                                                 C.byref(comp)) == gh.INVALID_HANDLE
    for t in toks:
        assert L.glacier_hip_buffer_release(gctx.h, C.byref(t)) == 0


TINY = dict(num_layers=2, dim=256, hidden_dim=512, num_heads=4, num_kv_heads=2, head_dim=64,
            vocab_size=4096, group_size=32, rms_eps=1e-6, rope_theta=1e6)


def _dev(gh, gctx):
    r, c = C.c_uint64(), C.c_uint64()
    assert gh.lib().glacier_hip_live_device_bytes(gctx.h, C.byref(r), C.byref(c)) == 0
    return r.value, c.value


def test_model_and_session_quotes_are_their_exact_charge(gh, gctx):
    """Weights and KV pools go through the lease accounting too: the model's
    and the session's side-effect-free quotes equal the device bytes their
    creation takes, and destroying them returns the bytes."""
    L = gh.lib()
    base = _dev(gh, gctx)
    mq = gh.AllocationQuote()
    cfg = gh.ModelConfig(**{k: TINY[k] for k, _ in gh.ModelConfig._fields_})
    assert L.glacier_hip_model_quote(gctx.h, C.byref(cfg), 0, C.byref(mq)) == 0
    assert _dev(gh, gctx) == base  # quoting allocates nothing
    m = gh.Model(gctx, TINY)
    m.set_from_host(gh.random_model_host(TINY, 1))
    after_model = _dev(gh, gctx)
    assert (after_model[0] - base[0], after_model[1] - base[1]) == (mq.requested_bytes,
                                                                    mq.charged_bytes)
    for kv in (gh.F32, gh.F16):
        opts = gh.SessionOptions(max_lanes=4, max_positions=300, total_pages=0, kv_dtype=kv,
                                 layer_activation=gh.ACT_AUTO, head_activation=gh.ACT_AUTO,
                                 use_graph=1, prefill_chunk=0)
        sq = gh.AllocationQuote()
        assert L.glacier_hip_session_quote(m.h, C.byref(opts), C.byref(sq)) == 0
        assert _dev(gh, gctx) == after_model
        s = gh.Session(m, max_lanes=4, max_positions=300, kv_dtype=kv)
        got = _dev(gh, gctx)
        assert (got[0] - after_model[0], got[1] - after_model[1]) == (sq.requested_bytes,
                                                                      sq.charged_bytes)
        s.close()
        assert _dev(gh, gctx) == after_model
    bad = gh.SessionOptions(max_lanes=0, max_positions=300)
    assert L.glacier_hip_session_quote(m.h, C.byref(bad), C.byref(gh.AllocationQuote())) == \
        gh.INVALID_ARGUMENT
    m.close()
    assert _dev(gh, gctx) == base
