"""rq_device_delay: the bounded device-side wait that benchmark drivers put in
front of a batch of direct launches (no reference counterpart)."""
import pytest

from rusty_amd import _lib
from rusty_amd.hiprt import Event

pytestmark = pytest.mark.gpu


def test_device_delay_holds_the_stream(ctx):
    a, b = Event(), Event()
    a.record(ctx.stream)
    _lib.call("rq_device_delay", ctx.handle, 2000, None)
    b.record(ctx.stream)
    b.synchronize()
    ms = a.elapsed_ms(b)
    assert 1.9 <= ms <= 50.0, ms


def test_device_delay_limits(ctx):
    lib = _lib.lib()
    assert lib.rq_device_delay(ctx.handle, 0, None) == _lib.RQ_OK
    assert lib.rq_device_delay(ctx.handle, 100001, None) == _lib.RQ_ERR_INVALID_ARGUMENT
    assert b"100000" in lib.rq_last_error()
    ctx.sync()
