"""One-token kernels whose grid is not all running at once. The single-launch QKV, O and FFN
kernels hand data between the workgroups of one launch; a wait that lasts the take-over threshold
computes the missing workgroup's share itself (moa_decode.hip, Stall). The test hook holds chosen
workgroups at entry -- before they read or write anything, as if the device had started them
late (another process holding CUs) -- and shortens the threshold. Every call must give the bits of
an undisturbed call, raise no device error, and (when the hold outlasts the threshold) count
take-overs; with a threshold longer than the hold, the waits simply last and nothing is taken
over. The held set includes post-norm leaders (0-7), which alone write their residual rows and
therefore find them unchanged when they start late."""
import ctypes as C

import numpy as np
import pytest

from gpu_util import need_gpu, say
from moa_amd import _lib, synth
from test_gpu_ffn import gpu_fp8, gpu_mxfp4, gpu_nvfp4
from test_gpu_full import out_gpu as full_o_gpu
from test_gpu_o import run_gpu as o_gpu
from test_gpu_o_ffn import gpu_fused as o_ffn_gpu
from test_gpu_qkv import run_gpu as qkv_gpu

pytestmark = pytest.mark.gpu

STEAL = 3000   # 30 us of the 100 MHz wall clock
HOLD = 40000   # 400 us


def set_stall(steal: int, hold_ticks: int = 0, hold=(-1, -1, -1, -1)) -> None:
    _lib.call("moa_test_set_stall", C.c_uint32(steal), C.c_uint32(hold_ticks), (C.c_int32 * 4)(*hold))


def take_overs() -> int:
    n = C.c_uint32(0)
    _lib.call("moa_test_take_overs", C.byref(n))
    return n.value


def noalloc_fp8(d):
    """moa_decoder_feedforward_fp8_noalloc (its hand-off and claim words live in the library's
    static device array) through the C ABI."""
    import torch
    from gpu_util import dev, host
    r = dev(d["residual"])
    t = {k: dev(d[k]) for k in ("pre_ff_rms_weight", "up_weight", "gate_weight", "down_weight", "up_weight_scale",
                                "gate_weight_scale", "down_weight_scale", "post_ff_rms_weight", "layer_scalar")}
    args = [C.c_void_p(r.data_ptr())] + [C.c_void_p(t[k].data_ptr()) for k in (
        "pre_ff_rms_weight", "up_weight", "gate_weight", "down_weight", "up_weight_scale", "gate_weight_scale",
        "down_weight_scale", "post_ff_rms_weight", "layer_scalar")]
    rc = _lib.load().moa_decoder_feedforward_fp8_noalloc(*args, 1, C.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, _lib.load().moa_last_error_string()
    return host(r)


@pytest.fixture(scope="module")
def calls():
    """One closure per single-launch kernel (and FFN mode): fixed inputs, host bits out."""
    need_gpu()
    f, m, n = synth.cfg_ffn_fp8(5), synth.cfg_ffn_mxfp4(5), synth.ref_ffn_inputs(1)
    o, fo, q, ro = synth.cfg_o(5), synth.cfg_full_o(5), synth.cfg_qkv(5), synth.ref_o_inputs(1)
    return {
        "ffn_fp8": lambda: gpu_fp8(f),
        "ffn_fp8_no_post_norm": lambda: gpu_fp8(f, post=False, ls=False),
        "ffn_fp8_noalloc": lambda: noalloc_fp8(f),
        "ffn_mxfp4": lambda: gpu_mxfp4(m),
        "ffn_nvfp4": lambda: gpu_nvfp4(n),
        "o": lambda: o_gpu(o),
        "o_ffn_fp8": lambda: o_ffn_gpu("fp8", o, f),
        "o_ffn_nvfp4": lambda: o_ffn_gpu("nvfp4", ro, n),
        "full_o": lambda: full_o_gpu(fo),
        "qkv": lambda: np.concatenate([a.reshape(-1) for a in qkv_gpu(q)]),
    }


# (label, steal ticks, held workgroups, take-overs expected). 2, 100, 239: an O/FFN leader, a
# middle and the last workgroup of the 240-workgroup grids (QKV, head b % 32: heads 2, 4 and 15);
# 255: QKV's last. 0, 1: two leaders; 130, 162: two workgroups of QKV head 2.
CASES = [
    ("take-over", STEAL, (2, 100, 239, 255), True),
    ("leaders late", STEAL, (0, 1, 130, 162), True),
    ("slow, no take-over", 10 * HOLD, (2, 100, 239, 255), False),
]


@pytest.mark.parametrize("label,steal,hold,expect", CASES, ids=[c[0] for c in CASES])
def test_late_workgroups_give_the_same_bits(calls, label, steal, hold, expect):
    from moa_amd import ops
    want = {k: fn() for k, fn in calls.items()}
    assert ops.device_errors() == 0
    assert take_overs() == 0, "an undisturbed call took work over"
    for k, fn in calls.items():
        say(f"residency {label}: {k}, workgroups {hold} held {HOLD / 100:.0f} us, threshold {steal / 100:.0f} us")
        set_stall(steal, HOLD, hold)
        try:
            got = fn()
            n = take_overs()
        finally:
            set_stall(0)
        assert np.array_equal(got, want[k]), f"{k}: {np.count_nonzero(got != want[k])} values differ"
        assert ops.device_errors() == 0, f"{k}: device error"
        if expect:
            assert n > 0, f"{k}: no wait took work over"
        else:
            assert n == 0, f"{k}: {n} take-overs with a threshold longer than the hold"
        assert np.array_equal(fn(), want[k]), f"{k}: the next undisturbed call differs"
    assert take_overs() == 0
