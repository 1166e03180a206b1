"""Device number-format helpers (the ones every kernel uses) against the oracle's tables."""
import numpy as np
import pytest

from gpu_util import host, need_gpu, say, torch
from moa_amd import formats as F
from moa_amd import prng
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def test_device_decoders_and_gelu_exhaustive():
    need_gpu()
    from moa_amd import ops
    say("format selftest: E4M3 x256, E2M1 x512, E8M0 x256, GeLU x65536")
    out = host(ops.format_selftest()).view(np.uint32)
    f32 = out.view(np.float32)
    e4m3 = F.e4m3_decode_table()
    nan = np.isnan(e4m3)
    assert np.array_equal(np.isnan(f32[:256]), nan)
    assert np.array_equal(f32[:256][~nan], e4m3[~nan])
    nib = F.e2m1_decode_table()
    b = np.arange(256)
    want = np.stack([nib[b & 0xF], nib[b >> 4]], axis=1).reshape(-1)  # low nibble first
    assert np.array_equal(f32[256:768], want)
    e8 = np.ldexp(np.float64(1.0), np.arange(255) - 127).astype(np.float32)
    assert np.array_equal(f32[768:768 + 255], e8)
    # How v_cvt_scalef32_pk_f32_fp4 applies an f32 scale to 6.0 (scales 15, 2, 3, 0.75); the
    # kernels decode at scale 1 and multiply block scales themselves, so this is a record only.
    say(f"scaled fp4 decode of 6.0 at scales 15,2,3,0.75 -> {f32[66560:66564].tolist()}")
    # GeLU: device tanhf vs host libm may differ in the last f32 ulp
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    x = prng.bf16_bits_to_f32(bits)
    gl, rne = O.lib().orc_gelu_tanh, O.lib().orc_bf16_rne
    ref = np.array([rne(gl(float(v))) for v in x], np.uint16)
    got = out[1024:1024 + 65536].astype(np.uint16)
    keep = np.isfinite(x)
    mism = keep & (got != ref)
    say(f"gelu mismatches vs oracle: {int(mism.sum())}")
    assert mism.sum() <= 64
    d = np.abs(prng.bf16_bits_to_f32(got[mism]) - prng.bf16_bits_to_f32(ref[mism]))
    assert np.all(d <= np.maximum(np.abs(prng.bf16_bits_to_f32(ref[mism])) * 2.0 ** -7, 2.0 ** -20))


def test_device_bf16_rounding():
    """The kernels' f32 -> bf16 rounding (v_cvt_pk_bf16_f32) against the raw-bit rule of
    fixture_prng.py:80-90 (prng.f32_to_bf16_bits): every bf16 high half with eight low halves --
    zero, one, just below, at and just above the tie, a quarter, three quarters, all ones -- so
    ties to even, carries into the exponent, subnormals, overflow to infinity and NaN inputs are
    all covered; plus the packed pair helper on every high half."""
    need_gpu()
    from moa_amd import ops
    say("format selftest: f32 -> bf16 rounding x524288, packed pairs x65536")
    out = host(ops.format_selftest()).view(np.uint32)
    hi = np.arange(1 << 16, dtype=np.uint32) << np.uint32(16)
    lows = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0x4000, 0xC000, 0xFFFF], np.uint32)
    src = (hi[:, None] | lows[None, :]).reshape(-1)
    want = prng.f32_to_bf16_bits(src.view(np.float32))
    got = out[132100:132100 + src.size].astype(np.uint16)
    nan_in = np.isnan(src.view(np.float32))
    assert np.all(np.isnan(prng.bf16_bits_to_f32(got[nan_in]))), "a NaN input lost its NaN"
    bad = ~nan_in & (got != want)
    assert not bad.any(), f"{int(bad.sum())} roundings differ, first input {src[bad][0]:#010x}"
    pair = out[656388:656388 + (1 << 16)]
    lo_src, hi_src = (hi | np.uint32(0x8000)).view(np.float32), (hi | np.uint32(0x7FFF)).view(np.float32)
    want_lo, want_hi = prng.f32_to_bf16_bits(lo_src), prng.f32_to_bf16_bits(hi_src)
    fin = ~np.isnan(lo_src)
    assert np.array_equal((pair & 0xFFFF)[fin].astype(np.uint16), want_lo[fin])
    assert np.array_equal((pair >> 16)[fin].astype(np.uint16), want_hi[fin])
