"""Resource accounting and limits of the HIP backend.

The report counts physical bytes the way the reference's wgpu backend does
(crates/backend-wgpu/src/lib.rs:340-370, tests.rs:75-129): every device
block the context holds, including the backend-private tile copies of
packed weights and idle pooled blocks, plus pending readback staging.  The
limits of `ResourceLimits` (crates/engine-api/src/resources.rs:27-43) apply
to all of it, and mfh_prepare_packed moves the cost of the private copies
(and any ResourceLimit) to load time, as the reference's LUT2 repack is
funded at construction (executor-core/src/lfm2/executor/construction.rs:
404-424).
"""
from __future__ import annotations

import ctypes
import sys

import numpy as np
import pytest

from runtime_amd import convert
from runtime_amd.backend import WEIGHT, ExecutorError, HipBackend, Limits

pytestmark = pytest.mark.gpu
MIB = 1 << 20


def say(*parts):
    print("[case]", *parts, flush=True)
    sys.stdout.flush()


def total(report) -> int:
    return (report.resident_weight_bytes + report.cache_bytes + report.scratch_bytes +
            report.staged_branch_bytes + report.pending_operation_bytes)


def device_free() -> int:
    """Free device memory of the current HIP device (hipMemGetInfo)."""
    hip = ctypes.CDLL("libamdhip64.so")
    free, whole = ctypes.c_size_t(0), ctypes.c_size_t(0)
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(whole)) == 0
    return free.value


def packed(n, k, scheme, seed=0x5EED0900):
    codes, scales16 = convert.packed_weights(n, k, scheme, seed)
    return codes, convert.f16_to_f32(scales16)


def upload(backend, codes, scales):
    return (backend.upload_u8_classified(codes.shape, codes, WEIGHT),
            backend.upload_f32_classified(scales.shape, scales, WEIGHT))


def test_report_matches_the_device_footprint():
    """The private copies (repacked tiles, tiled scales, binary16 shadow) are
    weight bytes, and the report's total tracks the device memory the
    context takes from the driver."""
    say("footprint int8 65536x2048")
    backend = HipBackend(0)
    try:
        # Load the code objects first so that module loading is not counted.
        warm = backend.upload_f32((4, 4), np.ones((4, 4), np.float32))
        backend.copy(backend.allocate_f32((4, 4)), warm)
        backend.synchronize()
        free0, report0 = device_free(), total(backend.resource_report())
        codes, scales = packed(65536, 2048, "int8")
        cb, sb = upload(backend, codes, scales)
        before = backend.resource_report()
        assert before.resident_weight_bytes >= codes.nbytes + scales.nbytes
        assert not backend.packed_prepared(cb, sb)
        backend.prepare_packed(cb, sb)
        backend.synchronize()
        assert backend.packed_prepared(cb, sb)
        after = backend.resource_report()
        # Repacked codes (the same bytes, padded) and tiled binary16 scales.
        grown = after.resident_weight_bytes - before.resident_weight_bytes
        assert codes.nbytes <= grown <= codes.nbytes + scales.nbytes + 4 * MIB
        # Classes are charged byte extents; the pool's bucket slack is scratch.
        assert 0 <= after.scratch_bytes - before.scratch_bytes <= grown // 8 + MIB
        used = free0 - device_free()
        reported = total(after) - report0
        assert 0.97 * reported <= used <= reported + 32 * MIB, (used, reported)
        assert backend.peak_accounted_bytes() >= total(after)
        # Preparing again changes nothing.
        backend.prepare_packed(cb, sb)
        assert total(backend.resource_report()) == total(after)
    finally:
        backend.close()


class Ballast:
    """Cache-class fillers that leave the context between 0 and `room` bytes
    under `limit`.  (A limit can never be tighter than the uploads
    themselves: the capability rule allows max_total_bytes / 4 elements of
    any dtype, storage.rs:183.)  Pieces are powers of two above 1 MiB and
    256-byte multiples below, sizes the pool serves exactly."""

    def __init__(self, backend, limit, room):
        self.pieces = []
        while True:
            want = limit - total(backend.resource_report()) - room // 2
            if want < 1024:
                break
            size = 1 << (want.bit_length() - 1) if want > MIB else want // 256 * 256
            self.pieces.append(backend.allocate_f32_classified((size // 4,), 1))
        left = limit - total(backend.resource_report())
        assert 0 <= left < room, (left, room)

    def release(self):
        for piece in self.pieces:
            piece.release()
        self.pieces = []


def test_tight_limit_fails_at_prepare_and_leaves_outputs_untouched():
    say("tight limit prepare")
    n, k, m = 8192, 2048, 2
    codes, scales = packed(n, k, "ternary")
    x = convert.normal((m, k), 0xAC70900)
    sentinel = np.full((m, n), 5.0, np.float32)
    limit = 4 * codes.size + 8 * MIB

    def loaded(backend):
        cb, sb = upload(backend, codes, scales)
        xb = backend.upload_f32(x.shape, x)
        out = backend.upload_f32(sentinel.shape, sentinel)
        return cb, sb, xb, out

    roomy = HipBackend(0, limits=Limits(max_total_bytes=limit))
    try:
        cb, sb, xb, out = loaded(roomy)
        need = total(roomy.resource_report())
        roomy.prepare_packed(cb, sb)
        copies = total(roomy.resource_report()) - need
        assert copies >= codes.nbytes
        roomy.packed_linear(out, xb, cb, sb)
        want = roomy.read(out)
        assert roomy.peak_accounted_bytes() <= limit
    finally:
        roomy.close()

    # Room for every upload, not for the private copies.
    tight = HipBackend(0, limits=Limits(max_total_bytes=limit))
    try:
        cb, sb, xb, out = loaded(tight)
        fill = Ballast(tight, limit, copies)
        before = total(tight.resource_report())
        with pytest.raises(ExecutorError) as e:
            tight.prepare_packed(cb, sb)
        assert e.value.variant == "ResourceLimit"
        assert e.value.message == "allocation exceeds configured total resource limit"
        assert total(tight.resource_report()) == before
        assert not tight.packed_prepared(cb, sb)
        # Without prepare, the first product meets the same limit before it
        # enqueues anything.
        with pytest.raises(ExecutorError) as e:
            tight.packed_linear(out, xb, cb, sb)
        assert e.value.variant == "ResourceLimit"
        assert np.array_equal(tight.read(out), sentinel)
        assert tight.peak_accounted_bytes() <= limit
        # Releasing the filler makes room; the product then matches.
        fill.release()
        tight.prepare_packed(cb, sb)
        tight.packed_linear(out, xb, cb, sb)
        assert tight.read(out).tobytes() == want.tobytes()
    finally:
        tight.close()


def test_model_attach_fails_at_load_under_a_tight_limit():
    from runtime_amd.lfm2 import ATTENTION, CONV, CONV_IN, Lfm2Config, Lfm2Model
    say("tight limit model attach")
    cfg = Lfm2Config(hidden=256, intermediate=512, attention_heads=4, key_value_heads=2,
                     vocab=1000, layers=[CONV, ATTENTION], max_tokens=64,
                     formats={"embedding": "int8", "conv": "nf4", "attention": "nf4",
                              "ffn": "ternary"})
    codes, scales = packed(3 * 256, 256, "nf4")
    limit = 4 * codes.size + 4 * MIB
    backend = HipBackend(0, limits=Limits(max_total_bytes=limit))
    try:
        model = Lfm2Model(backend, cfg)
        cb, sb = upload(backend, codes, scales)
        fill = Ballast(backend, limit, codes.nbytes)
        with pytest.raises(ExecutorError) as e:
            model.set_weight(CONV_IN, 0, cb, sb)
        assert e.value.variant == "ResourceLimit"
        fill.release()
        model.set_weight(CONV_IN, 0, cb, sb)
        assert backend.packed_prepared(cb, sb)
        model.close()
    finally:
        backend.close()


def test_idle_blocks_stay_charged_until_evicted():
    """backend-wgpu/src/tests.rs:75-129: a released block stays charged
    while pooled; an allocation that would exceed the limit first returns
    idle blocks to the driver."""
    say("pool eviction")
    backend = HipBackend(0, limits=Limits(max_total_bytes=24 * MIB))
    try:
        base = total(backend.resource_report())
        big = backend.allocate_f32((4 * MIB,))          # 16 MiB
        charged = total(backend.resource_report())
        assert charged - base == 16 * MIB
        assert backend.peak_accounted_bytes() == charged
        big.release()
        assert total(backend.resource_report()) == charged  # pooled, still charged
        other = backend.allocate_f32((2 * MIB + 1024,))      # different bucket, 8+ MiB
        now = total(backend.resource_report())
        assert now < charged
        assert backend.peak_accounted_bytes() == charged
        with pytest.raises(ExecutorError) as e:
            backend.allocate_f32((4 * MIB,))
        assert e.value.variant == "ResourceLimit"
        other.release()
    finally:
        backend.close()


def test_readback_staging_counts_against_the_limit():
    say("readback staging limit")
    backend = HipBackend(0, limits=Limits(max_total_bytes=20 * MIB))
    try:
        buf = backend.allocate_f32((3 * MIB,))  # 12 MiB
        with pytest.raises(ExecutorError) as e:
            backend.read_f32_async(buf)
        assert e.value.variant == "ResourceLimit"
        small = backend.allocate_f32((1024,))
        rb = backend.read_f32_async(small)
        report = backend.resource_report()
        assert report.pending_operation_bytes == 4096
        while rb.poll_step() is None:
            pass
        assert backend.resource_report().pending_operation_bytes == 0
    finally:
        backend.close()


def test_readback_evicts_idle_blocks_before_refusing():
    """A released block stays pooled (and charged); a readback that fits
    once the idle blocks are returned to the driver succeeds, as device
    allocations do (backend-wgpu/src/device.rs:657-676)."""
    say("readback eviction")
    backend = HipBackend(0, limits=Limits(max_total_bytes=28 * MIB))
    try:
        values = convert.normal((1, 2 * MIB), 0xAC70900).reshape(-1)
        buf = backend.upload_f32((2 * MIB,), values)     # 8 MiB
        big = backend.allocate_f32((4 * MIB,))          # 16 MiB: 24 MiB held
        big.release()                                    # idle, still charged
        assert total(backend.resource_report()) >= 24 * MIB
        rb = backend.read_f32_async(buf)                 # 32 MiB with staging, 16 once evicted
        got = None
        while got is None:
            got = rb.poll_step()
        assert got.tobytes() == values.tobytes()
        assert backend.resource_report().pending_operation_bytes == 0
    finally:
        backend.close()
