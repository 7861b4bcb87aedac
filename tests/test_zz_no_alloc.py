"""mfh_packed_linear_noalloc against mfh_packed_linear.

The allocation-free entry point runs the same decode GEMV with a fixed
device scratch array in place of pooled scratch, so its outputs must equal
packed_linear's bit for bit, call after call (the array keeps the previous
call's contents), and it must take no device memory from the context.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

import oracle
from runtime_amd import convert
from runtime_amd.backend import WEIGHT, ExecutorError, HipBackend
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu
SCHEMES = ["ternary", "nf4", "int8"]


def say(*parts):
    print("[case]", *parts, flush=True)
    sys.stdout.flush()


def total(report) -> int:
    return (report.resident_weight_bytes + report.cache_bytes + report.scratch_bytes +
            report.staged_branch_bytes + report.pending_operation_bytes)


@pytest.fixture(scope="module")
def be():
    b = HipBackend(0)
    yield b
    b.close()


def weights(backend, n, k, scheme, seed):
    codes, scales16 = convert.packed_weights(n, k, scheme, seed)
    scales = convert.f16_to_f32(scales16)
    cb = backend.upload_u8_classified(codes.shape, codes, WEIGHT)
    sb = backend.upload_f32_classified(scales.shape, scales, WEIGHT)
    return codes, scales, cb, sb


@pytest.mark.parametrize("scheme", SCHEMES)
def test_noalloc_equals_packed_linear_twice(be, scheme):
    # The second call is smaller in every dimension, so it reads less of the
    # shared scratch than the first one wrote.
    for call, (m, n, k) in enumerate([(8, 8192, 2048), (3, 1024, 1024), (1, 4608, 1024)]):
        say("noalloc", scheme, call, m, n, k)
        codes, scales, cb, sb = weights(be, n, k, scheme, 0x5EED0A00 + call)
        x = convert.normal((m, k), 0xAC70A00 + call)
        xb = be.upload_f32(x.shape, x)
        want_buf = be.allocate_f32((m, n))
        got_buf = be.allocate_f32((m, n))
        with pytest.raises(ExecutorError) as e:
            be.packed_linear_noalloc(got_buf, xb, cb, sb)
        assert e.value.variant == "Unsupported"
        be.prepare_packed(cb, sb)
        be.packed_linear(want_buf, xb, cb, sb)   # also grows the pooled scratch
        be.synchronize()
        before = total(be.resource_report())
        be.packed_linear_noalloc(got_buf, xb, cb, sb)
        got = be.read(got_buf)
        assert total(be.resource_report()) == before
        want = be.read(want_buf)
        assert got.tobytes() == want.tobytes()
        assert_close(got, oracle.packed_linear_threaded(x, codes, scales))


@pytest.mark.parametrize("scheme", SCHEMES)
def test_noalloc_first_on_a_fresh_context_takes_no_memory(scheme):
    """On a context whose pooled GEMV scratch has never been grown, the
    allocation-free call leaves the footprint (and its scratch part)
    unchanged; packed_linear afterwards gives the same bits."""
    say("noalloc fresh", scheme)
    fresh = HipBackend(0)
    try:
        m, n, k = 8, 8192, 2048
        codes, scales, cb, sb = weights(fresh, n, k, scheme, 0x5EED0A20)
        x = convert.normal((m, k), 0xAC70A20)
        xb = fresh.upload_f32(x.shape, x)
        got_buf = fresh.allocate_f32((m, n))
        want_buf = fresh.allocate_f32((m, n))
        fresh.prepare_packed(cb, sb)
        fresh.synchronize()
        before = fresh.resource_report()
        fresh.packed_linear_noalloc(got_buf, xb, cb, sb)
        fresh.synchronize()
        after = fresh.resource_report()
        assert total(after) == total(before)
        assert after.scratch_bytes == before.scratch_bytes
        got = fresh.read(got_buf)
        fresh.packed_linear(want_buf, xb, cb, sb)
        assert got.tobytes() == fresh.read(want_buf).tobytes()
    finally:
        fresh.close()


def test_noalloc_rejects_what_it_cannot_serve(be):
    say("noalloc rejects")
    codes, scales, cb, sb = weights(be, 64, 16512, "int8", 0x5EED0A10)
    be.prepare_packed(cb, sb)
    x = be.upload_f32((1, 16512), convert.normal((1, 16512), 1))
    out = be.allocate_f32((1, 64))
    with pytest.raises(ExecutorError) as e:
        be.packed_linear_noalloc(out, x, cb, sb)
    assert e.value.variant == "ResourceLimit"
    codes, scales, cb, sb = weights(be, 64, 1024, "int8", 0x5EED0A11)
    be.prepare_packed(cb, sb)
    x9 = be.upload_f32((9, 1024), convert.normal((9, 1024), 2))
    out9 = be.allocate_f32((9, 64))
    with pytest.raises(ExecutorError) as e:
        be.packed_linear_noalloc(out9, x9, cb, sb)
    assert e.value.variant == "Unsupported"
    # Admission is packed_linear's: a wrong output shape is InvalidShape.
    x1 = be.upload_f32((1, 1024), convert.normal((1, 1024), 3))
    with pytest.raises(ExecutorError) as e:
        be.packed_linear_noalloc(be.allocate_f32((1, 65)), x1, cb, sb)
    assert e.value.variant == "InvalidShape"
