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
