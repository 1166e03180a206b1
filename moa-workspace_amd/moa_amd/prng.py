"""Name-addressed input synthesis of the reference harness, restated in numpy.

Same recipes as FO/scripts/fixture_prng.py:44-198 (== FO/src/bin/test_kernels.rs:34-145):
an element's value depends only on its tensor's name and its index -- FNV-1a of the
name, then splitmix64's finaliser over (hash ^ index) + golden. Inputs built here are
byte-identical to the reference's, so its checksums apply to them.
"""
from __future__ import annotations

import numpy as np

_M64 = (1 << 64) - 1
_FNV_OFFSET = 0xCBF29CE484222325
_FNV_PRIME = 0x100000001B3
_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_MIX_A = np.uint64(0xBF58476D1CE4E5B9)
_MIX_B = np.uint64(0x94D049BB133111EB)
_BLOCK = 1 << 22  # elements generated per step (bounds temporary memory)


def name_hash(name: str) -> int:
    """FNV-1a (64-bit) of the UTF-8 name (fixture_prng.py:44-54)."""
    h = _FNV_OFFSET
    for b in name.encode("utf-8"):
        h = ((h ^ b) * _FNV_PRIME) & _M64
    return h


def _mix(x: np.ndarray) -> np.ndarray:
    x = x + _GOLDEN
    x = (x ^ (x >> np.uint64(30))) * _MIX_A
    x = (x ^ (x >> np.uint64(27))) * _MIX_B
    return x ^ (x >> np.uint64(31))


def words(name: str, count: int, offset: int = 0) -> np.ndarray:
    """`count` 64-bit words of tensor `name` starting at element `offset` (fixture_prng.py:57-67)."""
    seed = np.uint64(name_hash(name))
    idx = np.arange(offset, offset + count, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix(seed ^ idx)


def _blocks(count: int):
    for start in range(0, count, _BLOCK):
        yield start, min(count, start + _BLOCK)


def u01(w: np.ndarray) -> np.ndarray:
    """Top 24 bits as an exact f32 in [0, 1) (fixture_prng.py:71-77)."""
    return (w >> np.uint64(40)).astype(np.uint32).astype(np.float32) / np.float32(16777216.0)


def f32_to_bf16_bits(v) -> np.ndarray:
    """Round-half-to-even f32 -> bf16 bits (fixture_prng.py:80-90); NaN -> 0x7fc0."""
    b = np.ascontiguousarray(v, dtype=np.float32).view(np.uint32)
    out = ((b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    nan = (b & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    if nan.any():
        out[nan] = 0x7FC0
    return out


def bf16_bits_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def bf16_uniform(name: str, count: int, lo: float, hi: float) -> np.ndarray:
    """bf16 bits uniform in [lo, hi): lo + (hi - lo) * u in f32, then RNE (fixture_prng.py:94-103)."""
    out = np.empty(count, np.uint16)
    lo32, span = np.float32(lo), np.float32(hi) - np.float32(lo)
    for a, b in _blocks(count):
        out[a:b] = f32_to_bf16_bits(lo32 + span * u01(words(name, b - a, a)))
    return out


def f32_uniform(name: str, count: int, lo: float, hi: float) -> np.ndarray:
    lo32, span = np.float32(lo), np.float32(hi) - np.float32(lo)
    return (lo32 + span * u01(words(name, count))).astype(np.float32)


def bf16_signs(name: str, count: int, scale: float = 1.0) -> np.ndarray:
    """+-scale as bf16 bits, sign from the word's top bit (fixture_prng.py:115-125)."""
    mag = f32_to_bf16_bits(np.array([abs(scale)], np.float32))[0]
    neg = (words(name, count) >> np.uint64(63)).astype(bool)
    return np.where(neg, mag | np.uint16(0x8000), mag).astype(np.uint16)


def f8_banded(name: str, count: int, exp_min: int, exp_max: int, signed: bool = True) -> np.ndarray:
    """E4M3 codes with the exponent field drawn from [exp_min, exp_max] (fixture_prng.py:128-148)."""
    assert 0 <= exp_min <= exp_max <= 14
    out = np.empty(count, np.uint8)
    span = np.uint64(exp_max - exp_min + 1)
    for a, b in _blocks(count):
        w = words(name, b - a, a)
        e = (np.uint64(exp_min) + (w >> np.uint64(32)) % span).astype(np.uint8)
        m = ((w >> np.uint64(56)) & np.uint64(7)).astype(np.uint8)
        s = ((w >> np.uint64(63)).astype(np.uint8) << np.uint8(7)) if signed else np.uint8(0)
        out[a:b] = s | (e << np.uint8(3)) | m
    return out


def f4_nibbles(name: str, count: int) -> np.ndarray:
    """`count` E2M1 codes packed two per byte, low nibble first (fixture_prng.py:151-166)."""
    assert count % 2 == 0
    out = np.empty(count // 2, np.uint8)
    for a, b in _blocks(count):
        c = ((words(name, b - a, a) >> np.uint64(60)) & np.uint64(0xF)).astype(np.uint8)
        out[a // 2:b // 2] = c[0::2] | (c[1::2] << np.uint8(4))
    return out


def checksum(storage) -> int:
    """Position-weighted u32 checksum over the storage bytes (fixture_prng.py:170-198)."""
    data = np.ascontiguousarray(storage).reshape(-1).view(np.uint8)
    pad = (-data.size) % 4
    if pad:
        data = np.concatenate([data, np.zeros(pad, np.uint8)])
    w = data.view(np.uint32)
    total = 0
    for a in range(0, w.size, _BLOCK):
        blk = w[a:a + _BLOCK]
        idx = np.arange(a, a + blk.size, dtype=np.uint32)
        with np.errstate(over="ignore"):
            total += int((blk * (idx * np.uint32(2) + np.uint32(1))).sum(dtype=np.uint32))
    return total & 0xFFFFFFFF


def run_pos(run: int) -> int:
    """The harness's RoPE/cache position for run `run` (generate_references.py:79-90)."""
    return 1 + int(words(f"run{run}.global.pos", 1)[0] % np.uint64(2047))
