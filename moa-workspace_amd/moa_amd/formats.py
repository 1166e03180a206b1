"""Weight formats: decode tables and round-to-nearest-even quantisers (numpy).

E4M3FN (OCP): bias 7, S.1111.111 = NaN, max 448, subnormals m * 2^-9 -- the code type the
reference's FP8 weights use (torch.float8_e4m3fn, FO/scripts/generate_references.py:152).
E2M1: {0,.5,1,1.5,2,3,4,6}, bit 3 = sign, packed two per byte low nibble first
(generate_references.py:69,154-163). E8M0: 2^(e-127).
"""
from __future__ import annotations

import numpy as np

E2M1_MAGNITUDES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], np.float32)


def e4m3_decode_table() -> np.ndarray:
    c = np.arange(256)
    e = (c >> 3) & 15
    m = c & 7
    mag = np.where(e == 0, np.ldexp(m.astype(np.float64), -9), np.ldexp(1.0 + m / 8.0, e - 7))
    mag = np.where((e == 15) & (m == 7), np.nan, mag)
    return np.where(c & 0x80, -mag, mag).astype(np.float32)


def e2m1_decode_table() -> np.ndarray:
    c = np.arange(16)
    return np.where(c & 8, -E2M1_MAGNITUDES[c & 7], E2M1_MAGNITUDES[c & 7]).astype(np.float32)


def e4m3_encode(v) -> np.ndarray:
    """f32 -> E4M3FN code, round half to even, saturating at +-448 (inputs never exceed it)."""
    v = np.asarray(v, dtype=np.float32)
    sign = np.signbit(v).astype(np.uint8) << np.uint8(7)
    a = np.abs(v).astype(np.float32)
    _, e = np.frexp(a)  # a = f * 2^e, f in [0.5, 1)
    quantum = np.where(a < np.float32(2.0 ** -6), np.float32(2.0 ** -9), np.ldexp(np.float32(1.0), e - 4)).astype(np.float32)
    r = (np.rint(a / quantum) * quantum).astype(np.float32)  # scaling by 2^k is exact
    r = np.minimum(r, np.float32(448.0))
    _, er = np.frexp(r)
    exp_field = np.clip(er - 1 + 7, 1, 15)
    mant_n = np.rint((r / np.ldexp(np.float32(1.0), er - 1) - 1.0) * 8.0).astype(np.int64)
    normal = ((exp_field.astype(np.int64) << 3) | mant_n).astype(np.uint8)
    sub = np.rint(r / np.float32(2.0 ** -9)).astype(np.uint8)
    code = np.where(r >= np.float32(2.0 ** -6), normal, sub)
    code = np.where(np.isnan(v), np.uint8(0x7F), code | sign)
    return code.astype(np.uint8)


def e2m1_encode(v) -> np.ndarray:
    """f32 -> E2M1 nibble, round half to even onto {0,.5,1,1.5,2,3,4,6}, saturating at 6."""
    v = np.asarray(v, dtype=np.float32)
    a = np.abs(v)
    c = np.full(a.shape, 7, np.uint8)
    for code, hi, inclusive in ((0, 0.25, True), (1, 0.75, False), (2, 1.25, True), (3, 1.75, False),
                                (4, 2.5, True), (5, 3.5, False), (6, 5.0, True)):
        hit = (a <= hi) if inclusive else (a < hi)
        c = np.where(hit & (c == 7), np.uint8(code), c)
    return (c | (np.signbit(v).astype(np.uint8) << np.uint8(3))).astype(np.uint8)


def pack_nibbles(codes: np.ndarray) -> np.ndarray:
    """[..., K] nibbles -> [..., K/2] bytes, low nibble = even index."""
    return (codes[..., 0::2] | (codes[..., 1::2] << np.uint8(4))).astype(np.uint8)


def unpack_nibbles(packed: np.ndarray) -> np.ndarray:
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), np.uint8)
    out[..., 0::2] = packed & 0xF
    out[..., 1::2] = packed >> 4
    return out


def quantize_fp8_rows(w: np.ndarray):
    """Per-output-channel FP8: s = max|row| / 448 (f32), code = E4M3_RNE(w / s).

    The bulk conversion uses torch's float8_e4m3fn cast when torch is importable: it is the same
    round-half-to-even map as e4m3_encode (tests/test_formats.py checks the two agree) and much
    faster on 59M-element matrices."""
    w = np.asarray(w, dtype=np.float32)
    s = (np.abs(w).max(axis=1) / np.float32(448.0)).astype(np.float32)
    s = np.where(s == 0, np.float32(1.0), s).astype(np.float32)
    q = w / s[:, None]
    try:
        import torch
    except ImportError:
        return e4m3_encode(q), s
    codes = torch.from_numpy(np.ascontiguousarray(q)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    return codes, s


def quantize_mxfp4(w: np.ndarray):
    """OCP MXFP4 along K: per 32-block X = 2^(floor(log2 amax) - 2) as E8M0, codes E2M1_RNE(w/X)."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    blk = w.reshape(n, k // 32, 32)
    amax = np.abs(blk).max(axis=2)
    _, e = np.frexp(amax)  # amax = f * 2^e, floor(log2 amax) = e - 1
    x_exp = np.where(amax > 0, e - 1 - 2, -127).clip(-127, 127)
    scale_code = (x_exp + 127).astype(np.uint8)
    codes = e2m1_encode(blk / np.ldexp(np.float32(1.0), x_exp)[..., None].astype(np.float32))
    return pack_nibbles(codes.reshape(n, k)), scale_code


def dequantize_fp8_rows(codes: np.ndarray, s: np.ndarray) -> np.ndarray:
    return e4m3_decode_table()[codes] * s[:, None]
