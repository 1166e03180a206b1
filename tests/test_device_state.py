"""The tripped device state (no GPU needed): after an expired cross-workgroup wait has been read
back (MOA_DEVERR_SPIN_TIMEOUT), every call that computes on the device and moa_init refuse with
MOA_ERROR_DEVICE_STATE until moa_clear_device_state; and the Python binding's checked mode turns
device error bits read after a call into MoaError. The trip hook sets the state as the read-back
does, so nothing here launches: the refused calls return before touching their pointers (fake,
aligned, never dereferenced)."""
import ctypes as C

import pytest

from moa_amd import _lib

FAKE = 0x100000  # aligned, never dereferenced (the refusal comes before any launch)

CALLS = [
    ("moa_sliding_project_qkv", 17),
    ("moa_sliding_attention_output", 5),
    ("moa_decoder_feedforward", 13),
    ("moa_decoder_feedforward_fp8", 10),
    ("moa_decoder_feedforward_mxfp4", 10),
    ("moa_decoder_feedforward_fp8_noalloc", 10),
    ("moa_sliding_attention_output_feedforward_fp8", 14),
    ("moa_sliding_attention", 5),
    ("moa_final_norm_and_logits", 4),
    ("moa_full_project_qkv", 15),
    ("moa_full_attention_output", 6),
]


@pytest.fixture
def tripped():
    lib = _lib.load()
    assert lib.moa_test_trip_device_state(0) == 0
    yield lib
    assert lib.moa_clear_device_state(0) == 0


@pytest.mark.parametrize("fn,nptr", CALLS)
def test_tripped_device_refuses_calls(tripped, fn, nptr):
    rc = getattr(tripped, fn)(*([FAKE] * nptr), 1, None)
    assert rc == -5, (fn, rc)
    msg = tripped.moa_last_error_string().decode()
    assert "expired" in msg and "moa_clear_device_state(0)" in msg


def test_tripped_device_refuses_init(tripped):
    assert tripped.moa_init(0) == -5


def test_argument_errors_still_come_first(tripped):
    """A call with a NULL pointer is rejected for it, tripped state or not."""
    rc = tripped.moa_decoder_feedforward_fp8(*([None] * 10), 1, None)
    assert rc == -1


def test_clear_restores_calls():
    lib = _lib.load()
    assert lib.moa_test_trip_device_state(0) == 0
    assert lib.moa_clear_device_state(0) == 0
    # the call now goes on to the device (which this machine may lack): any code but the refusal
    rc = lib.moa_decoder_feedforward_fp8(*([FAKE] * 10), 1, None) if _no_device() else None
    if rc is not None:
        assert rc != -5
    assert lib.moa_clear_device_state(-1) == -1
    assert lib.moa_test_trip_device_state(64) == -1


def _no_device() -> bool:
    import torch
    return not torch.cuda.is_available()


def test_checked_mode_raises_on_device_error_bits(monkeypatch):
    """ops._call runs the entry point, then (checked mode) device_errors(); a bit raises."""
    from moa_amd import ops
    calls = []
    monkeypatch.setattr(_lib, "call", lambda name, *a: calls.append(name))
    monkeypatch.setattr(ops, "device_errors", lambda device=None: _lib.DEVERR_SPIN_TIMEOUT)
    ops.set_checked(False)
    ops._call("moa_x")  # unchecked: no read-back
    ops.set_checked(True)
    try:
        with pytest.raises(_lib.MoaError) as e:
            ops._call("moa_y")
        assert e.value.code == -5 and "0x4" in str(e.value)
        monkeypatch.setattr(ops, "device_errors", lambda device=None: 0)
        ops._call("moa_z")  # no bits: no error
    finally:
        ops.set_checked(False)
    assert calls == ["moa_x", "moa_y", "moa_z"]
