"""GPU: the measurement hooks bench.py builds its floors and synchronisation
figures on (cq_time_stream, cq_time_grid_barrier; no counterpart in the
reference).  They must return plausible times, finish every barrier (no
bounded wait gives up) and reject arguments they cannot run."""
import ctypes

import pytest

import cuqwen_amd as cq

pytestmark = pytest.mark.gpu


def test_time_stream_empty_and_small_read():
    us = ctypes.c_double()
    cq.check(cq.lib.cq_time_stream(0, 1, None, 16, ctypes.byref(us)))
    assert 0.1 < us.value < 50.0
    n = 1 << 20
    bufs = [cq.DeviceBuffer(n) for _ in range(2)]
    for b in bufs:
        b.zero()
    arr = (ctypes.c_void_p * 2)(*[b.value for b in bufs])
    cq.check(cq.lib.cq_time_stream(n, 2, arr, 16, ctypes.byref(us)))
    assert 0.1 < us.value < 200.0
    for b in bufs:
        b.free()


@pytest.mark.parametrize("kind", [0, 1, 2, 3])
@pytest.mark.parametrize("blocks", [1, 64, 256])
def test_grid_barrier_every_kind_completes(kind, blocks):
    print(f"grid barrier kind={kind} blocks={blocks}", flush=True)
    t, to = ctypes.c_double(), ctypes.c_int32(-1)
    cq.check(cq.lib.cq_time_grid_barrier(kind, blocks, 20, ctypes.byref(t), ctypes.byref(to)))
    assert to.value == 0
    assert -5.0 < t.value < 1000.0


def test_grid_barrier_rejects_bad_arguments():
    t, to = ctypes.c_double(), ctypes.c_int32()
    for kind, blocks, rounds in ((4, 64, 10), (0, 0, 10), (0, 100000, 10), (1, 64, 0)):
        with pytest.raises(cq.CuQwenError):
            cq.check(cq.lib.cq_time_grid_barrier(kind, blocks, rounds, ctypes.byref(t), ctypes.byref(to)))
