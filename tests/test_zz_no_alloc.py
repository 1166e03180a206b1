"""moa_decoder_feedforward_fp8_noalloc (static device scratch, no allocation) against
moa_decoder_feedforward_fp8 (the per-device hipMalloc'd scratch), both called through the C ABI:
the same kernels must give the same bits. Two calls in a row, the second with fewer rows (16 rows
on the matrix-core rows path, then one row on the single-launch kernel, then five), so the second
runs on the scratch the first left behind; then a call beyond the stated maximum is rejected."""
import ctypes as C

import numpy as np
import pytest

from gpu_util import dev, host, need_gpu, say, torch
from moa_amd import _lib, synth

pytestmark = pytest.mark.gpu


def _call(name, d, r):
    M = r.numel() // 3840
    args = [C.c_void_p(r.data_ptr())] + [C.c_void_p(d[k].data_ptr()) for k in (
        "pre_ff_rms_weight", "up_weight", "gate_weight", "down_weight", "up_weight_scale", "gate_weight_scale",
        "down_weight_scale", "post_ff_rms_weight", "layer_scalar")]
    return getattr(_lib.load(), name)(*args, M, C.c_void_p(torch.cuda.current_stream().cuda_stream))


def test_noalloc_matches_the_allocating_entry_point():
    need_gpu()
    from moa_amd import ops
    w = synth.cfg_ffn_fp8(12)
    d = {k: dev(v) for k, v in w.items() if k != "residual"}
    for M in (16, 1, 5):
        say(f"no-alloc fp8 ffn M{M} vs moa_decoder_feedforward_fp8")
        res = synth.bf16_normal(f"noalloc.M{M}.residual", (M, 3840))
        a, b = dev(res), dev(res)
        assert _call("moa_decoder_feedforward_fp8_noalloc", d, a) == 0, _lib.load().moa_last_error_string()
        assert _call("moa_decoder_feedforward_fp8", d, b) == 0, _lib.load().moa_last_error_string()
        ga, gb = host(a), host(b)
        assert np.array_equal(ga, gb), f"M{M}: {np.count_nonzero(ga != gb)} elements differ"
        assert not np.array_equal(ga, res.reshape(-1)), f"M{M}: the residual was not updated"
    assert ops.device_errors() == 0


def test_noalloc_rejects_more_rows_than_its_scratch_holds():
    need_gpu()
    lib = _lib.load()
    w = synth.cfg_ffn_fp8(12)
    d = {k: dev(v) for k, v in w.items() if k != "residual"}
    r = dev(np.zeros((17, 3840), np.uint16))
    assert _call("moa_decoder_feedforward_fp8_noalloc", d, r) == -1
    assert b"no-allocation" in lib.moa_last_error_string()
    assert np.all(host(r) == 0)
