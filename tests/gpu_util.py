"""Helpers for the GPU parity tests: upload numpy inputs, call the C ABI through moa_amd.ops,
and compare against the CPU oracle with the reference's gate."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from kat_inputs import compare, unbf

torch = pytest.importorskip("torch")

# bf16 outputs within rtol 1e-2 / atol 1e-2 (the reference itself uses atol
# 0.04 QKV, 0.05 O, 0.01 FFN: FO/src/bin/test_kernels.rs:447-465).
RTOL, ATOL = 1e-2, 1e-2


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


def gate(expected_bits: np.ndarray, actual_bits: np.ndarray, label: str, atol=ATOL, rtol=RTOL):
    """Assert the reference gate on bf16 outputs; print the comparison line the reference prints."""
    ok, maxd, exact, nfail = compare(unbf(expected_bits), actual_bits, atol, rtol)
    n = expected_bits.size
    say(f"[{label:40}] max|d|={maxd:.5f} exact={exact}/{n} fail={nfail}")
    assert ok, f"{label}: {nfail} of {n} outside atol {atol} + rtol {rtol}; max |d| {maxd}"
    return exact / n
