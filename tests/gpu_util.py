"""Helpers for the GPU parity tests: upload numpy inputs, call the C ABI through moa_amd.ops,
and compare against the CPU oracle with the reference's gate."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from kat_inputs import compare, sign_failures, unbf

torch = pytest.importorskip("torch")

# bf16 outputs within rtol 1e-2 / atol 1e-2 (the reference itself uses atol
# 0.04 QKV, 0.05 O, 0.01 FFN: FO/src/bin/test_kernels.rs:447-465).
RTOL, ATOL = 1e-2, 1e-2


def bf16_ulp(x: np.ndarray) -> np.ndarray:
    """Spacing of bf16 numbers at |x| (8 significant bits); 2^-133 at zero."""
    ax = np.maximum(np.abs(np.asarray(x, np.float64)), 2.0 ** -126)
    return np.exp2(np.floor(np.log2(ax)) - 7)


def gate_addend(expected_bits, actual_bits, residual_bits, label: str, atol=ATOL, rtol=RTOL):
    """The gate for outputs of the form bf16(r + bf16(d)) with no normalisation after the
    rounding of d (the FFN with its post-norm and layer scalar switched off, a mode the
    reference operator does not have: FO/src/ops.rs:235-237 always applies both). d is an f32
    sum of 15360 products; any two f32 summation orders round it to bf16 differently when it
    lies within a few f32 ulps of a bf16 rounding midpoint, and that one-ulp step of d passes
    to the output unscaled, where r + d can cancel. Such an element passes if it is within
    atol + rtol |e| plus one bf16 ulp of the addend and one of the sum; at most 1 in 1000
    elements may need that allowance, every other one meets the plain gate."""
    e = unbf(np.asarray(expected_bits).reshape(-1)).astype(np.float64)
    a = unbf(np.asarray(actual_bits).reshape(-1)).astype(np.float64)
    r = unbf(np.asarray(residual_bits).reshape(-1)).astype(np.float64)
    assert np.all(np.isfinite(a)), f"{label}: non-finite output"
    diff = np.abs(a - e)
    plain = atol + rtol * np.abs(e)
    addend = np.maximum(np.abs(e - r), np.abs(a - r))
    allow = plain + bf16_ulp(addend) + bf16_ulp(np.maximum(np.abs(e), np.abs(a)))
    n = e.size
    n_step = int(np.count_nonzero(diff > plain))
    n_fail = int(np.count_nonzero(diff > allow))
    say(f"[{label:40}] max|d|={diff.max(initial=0.0):.5f} exact={int(np.count_nonzero(diff == 0))}/{n} "
        f"one-ulp-addend={n_step} fail={n_fail}")
    assert n_fail == 0, f"{label}: {n_fail} of {n} outside the gate plus one addend ulp"
    assert n_step <= n // 1000, f"{label}: {n_step} of {n} need the addend allowance"


def need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")


def dev(a: np.ndarray) -> "torch.Tensor":
    """Upload; bf16 bit arrays (uint16) travel as int16 views (torch's uint16 support is partial)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a.copy()).cuda()


def dev_zeros(n: int) -> "torch.Tensor":
    return torch.zeros(n, dtype=torch.int16, device="cuda")


def host(t: "torch.Tensor") -> np.ndarray:
    torch.cuda.synchronize()
    a = t.cpu().numpy()
    return a.view(np.uint16) if a.dtype == np.int16 else a


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _show_failures(e: np.ndarray, a: np.ndarray, bad: np.ndarray, label: str, limit: int = 8) -> None:
    for i in np.nonzero(bad)[0][:limit]:
        say(f"    {label}: element {int(i)} expected {e[i]!r} got {a[i]!r} |d|={abs(float(a[i]) - float(e[i])):.6g}")


def gate(expected_bits: np.ndarray, actual_bits: np.ndarray, label: str, atol=ATOL, rtol=RTOL):
    """Assert the reference gate on bf16 outputs; print the comparison line the reference prints
    (and each failing element)."""
    ok, maxd, exact, nfail = compare(unbf(expected_bits), actual_bits, atol, rtol)
    n = expected_bits.size
    say(f"[{label:40}] max|d|={maxd:.5f} exact={exact}/{n} fail={nfail}")
    if not ok:
        e = unbf(np.asarray(expected_bits).reshape(-1))
        a = unbf(np.asarray(actual_bits).reshape(-1))
        bad = ~np.isfinite(a) | (np.abs(a - e) > atol + rtol * np.abs(e)) | sign_failures(e, a, atol)
        _show_failures(e, a, bad, label)
    assert ok, f"{label}: {nfail} of {n} outside atol {atol} + rtol {rtol}; max |d| {maxd}"
    return exact / n


def gate_rope(expected_bits, actual_bits, label: str, head_dim: int, atol=ATOL, rtol=RTOL):
    """The gate for rotated head outputs y_i = bf16(bf16(n_i cos) + bf16(n_j sin)), j = i ^ (D/2),
    n the normalised head (sliding/rope.rs, generate_references.py:213-220). n comes out of an f32
    projection whose summation order the reference leaves unspecified, so two correct orders can
    round an element of n to bf16 values one ulp apart; that step reaches y unscaled by the
    rotation, and where the two terms cancel it can exceed atol + rtol |y| and even flip y's sign.
    |n_i| and |n_j| are at most the norm of the rotated pair (y_i, y_j) (a rotation keeps it), so an
    element passes if it is within atol + rtol |e| plus one bf16 ulp of that norm (with 2^-6
    relative slack for the roundings) and one ulp of the output; at most 1 in 1000 elements may use
    the allowance (exempt from the sign rule: it is the cancellation), every other one meets the
    plain gate and the sign rule. Each element that uses the allowance is printed."""
    e = unbf(np.asarray(expected_bits).reshape(-1, head_dim)).astype(np.float64)
    a = unbf(np.asarray(actual_bits).reshape(-1, head_dim)).astype(np.float64)
    assert np.all(np.isfinite(a)), f"{label}: non-finite output"
    h = head_dim // 2
    partner = np.concatenate([e[:, h:], e[:, :h]], axis=1)
    pair = np.hypot(e, partner) * (1.0 + 2.0 ** -6)
    diff = np.abs(a - e)
    plain = atol + rtol * np.abs(e)
    allow = plain + bf16_ulp(pair) + bf16_ulp(np.maximum(np.abs(e), np.abs(a)))
    step = diff > plain
    sign = sign_failures(e.reshape(-1), a.reshape(-1), atol).reshape(e.shape) & ~step
    n_fail = int(np.count_nonzero(diff > allow)) + int(np.count_nonzero(sign))
    n_step = int(np.count_nonzero(step))
    say(f"[{label:40}] max|d|={diff.max(initial=0.0):.5f} exact={int(np.count_nonzero(diff == 0))}/{e.size} "
        f"one-ulp-rotation={n_step} fail={n_fail}")
    if n_step or n_fail:
        _show_failures(e.reshape(-1), a.reshape(-1), (step | sign).reshape(-1), label)
    assert n_fail == 0, f"{label}: {n_fail} of {e.size} outside the gate plus one ulp of the rotated pair"
    assert n_step <= e.size // 1000, f"{label}: {n_step} of {e.size} need the rotation allowance"
