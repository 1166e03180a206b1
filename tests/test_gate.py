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


def test_sign_rule_rejects_a_flip_the_bound_alone_allows():
    """|e| = 1.005 atol, a = -2e-5: |a - e| = 1.007 atol <= atol + rtol |e| = 1.01005 atol, so
    the atol/rtol bound passes; the output has the wrong sign where |e| >= atol, so the gate fails."""
    from kat_inputs import compare, sign_failures
    atol = 1e-2
    e = np.array([1.005 * atol, 0.5, -0.25], np.float32)
    a_bits = bf([-2e-5, 0.5, -0.25])
    diff = np.abs(unbf(a_bits) - e)
    assert np.all(diff <= atol + 1e-2 * np.abs(e))  # the bound alone passes
    assert sign_failures(e, unbf(a_bits), atol).tolist() == [True, False, False]
    ok, _, _, nfail = compare(e, a_bits, atol)
    assert not ok and nfail == 1


def test_sign_rule_allows_sign_noise_below_atol():
    from kat_inputs import compare
    e = np.array([0.5 * 1e-2, -1e-5, 0.0], np.float32)
    ok, _, _, _ = compare(e, bf([-1e-3, 1e-5, -0.0]), 1e-2)
    assert ok


def _rope_case(shift_ulps):
    """Heads of 256 whose element 0 is a near-cancelling rotation: y_0 = bf16(bf16(n_0 c) + bf16(n_128 s))
    with n_0 c ~ -n_128 s; the "device" rounded n_0 `shift_ulps` bf16 ulps away. Every other element is
    exact."""
    from gpu_util import gate_rope  # noqa: F401
    c, s = np.float32(0.6), np.float32(0.8)
    n0, n1 = np.float32(3.0), np.float32(-2.2265625)  # 3 * 0.6 = 1.8, -2.2265625 * 0.8 = -1.78125
    rot = lambda a, b: unbf(bf([unbf(bf([a * c]))[0] + unbf(bf([b * s]))[0]]))[0]
    e_heads = np.zeros((1000, 256), np.float32)
    a_heads = e_heads.copy()
    e_heads[0, 0] = rot(n0, n1)
    a_heads[0, 0] = rot(n0 + shift_ulps * np.float32(bf16_ulp(n0)), n1)
    # the partner element holds the other rotated output, so the pair's norm bounds |n|
    e_heads[0, 128] = a_heads[0, 128] = unbf(bf([n1 * c - n0 * s]))[0]
    return bf(e_heads), bf(a_heads)


def test_rope_gate_takes_one_rotation_ulp_and_rejects_three():
    """One ulp of n_0 (times cos 0.6) passes with the allowance; three ulps exceed atol + one ulp of
    the pair's norm (same binade as n_0 here) and fail."""
    from gpu_util import gate_rope
    e, a = _rope_case(1)
    e0, a0 = float(unbf(e)[0, 0]), float(unbf(a)[0, 0])
    assert abs(a0 - e0) > 1e-2 + 1e-2 * abs(e0)  # the plain gate fails
    with pytest.raises(AssertionError):
        gate(e, a, "rope 1ulp plain")
    gate_rope(e, a, "rope 1ulp", 256)
    e, a = _rope_case(3)
    with pytest.raises(AssertionError):
        gate_rope(e, a, "rope 3ulp", 256)


def test_rope_gate_bounds_how_often_the_allowance_is_used():
    from gpu_util import gate_rope
    e, a = _rope_case(1)
    with pytest.raises(AssertionError):
        gate_rope(e[:1], a[:1], "rope 1ulp, too often", 256)
