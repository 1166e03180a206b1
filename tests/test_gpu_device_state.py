"""The tripped device state on the GPU: a tripped device refuses operator calls (MoaError, code
MOA_ERROR_DEVICE_STATE) and moa_init; after moa_clear_device_state the same call computes the
same bits as before; checked mode passes a clean call."""
import numpy as np
import pytest

from gpu_util import need_gpu, say
from moa_amd import _lib, synth
from test_gpu_ffn import gpu_fp8

pytestmark = pytest.mark.gpu


def test_trip_refuse_clear():
    need_gpu()
    from moa_amd import ops
    say("device state: trip, refuse, clear")
    d = synth.cfg_ffn_fp8(3)
    want = gpu_fp8(d)
    lib = _lib.load()
    assert lib.moa_test_trip_device_state(0) == 0
    try:
        with pytest.raises(_lib.MoaError) as e:
            gpu_fp8(d)
        assert e.value.code == -5
        assert lib.moa_init(0) == -5
    finally:
        ops.clear_device_state(0)
    assert np.array_equal(gpu_fp8(d), want)
    ops.set_checked(True)
    try:
        assert np.array_equal(gpu_fp8(d), want)
    finally:
        ops.set_checked(False)
    assert ops.device_errors() == 0
