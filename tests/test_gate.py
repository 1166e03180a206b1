"""CPU checks of the parity gates themselves: the plain atol/rtol gate and the addend-aware
gate used where an output is bf16(r + bf16(d)) with no normalisation after d's rounding."""
import numpy as np
import pytest

from gpu_util import bf16_ulp, gate, gate_addend
from kat_inputs import unbf
from moa_amd import prng


def bf(x):
    return prng.f32_to_bf16_bits(np.asarray(x, np.float32))


def test_bf16_ulp_matches_bit_steps():
    x = np.array([1.0, 1.5, 3.0, 5.0, 0.01, -6.0], np.float32)
    bits = bf(x)
    step = np.abs(unbf((bits + 1).astype(np.uint16)).astype(np.float64) - unbf(bits))
    assert np.array_equal(bf16_ulp(x), step)


def _cancelling_case(shift_ulps):
    # r = -d exactly cancels; the "device" rounded d one (or two) bf16 ulps away.
    d = np.array([5.0, -6.5, 3.25, 0.75], np.float32)
    r = bf(-d + np.array([0.0, 0.0, 0.0, 0.5], np.float32))
    e = bf(unbf(r) + d)
    d_dev = d + shift_ulps * bf16_ulp(d).astype(np.float32) * np.array([1, 0, 0, 0], np.float32)
    a = bf(unbf(r) + d_dev)
    big = np.zeros(4000, np.uint16)  # exact elements, so one allowance fits in 1/1000
    return np.concatenate([e, big]), np.concatenate([a, big]), np.concatenate([r, big])


def test_plain_gate_rejects_one_addend_ulp_at_cancellation():
    e, a, _ = _cancelling_case(1)
    with pytest.raises(AssertionError):
        gate(e, a, "cancel 1ulp")


def test_addend_gate_takes_one_ulp_and_rejects_two():
    e, a, r = _cancelling_case(1)
    gate_addend(e, a, r, "cancel 1ulp")
    e, a, r = _cancelling_case(2)
    with pytest.raises(AssertionError):
        gate_addend(e, a, r, "cancel 2ulp")


def test_addend_gate_bounds_how_often_the_allowance_is_used():
    e, a, r = _cancelling_case(1)
    with pytest.raises(AssertionError):
        gate_addend(e[:4], a[:4], r[:4], "cancel 1ulp, too often")
