"""Launch epochs across their wrap points on the device. The epoch counters of the one-token
QKV, O and FFN kernels and of the 16-row FFN (and the sliding-attention tickets) are preset by the test hook as if
2^27 - 2, 2^28 - 2 or 2^32 - 3 launches had run; four launches of each operator then cross:
the 32-bit wrap of the attention tickets (2^27 launches x 32 arrivals), the 32-bit boundary of the
64-bit FFN / O counters (2^28 launches x 16 workgroups), and the wrap of the 32-bit tag itself
(2^32 - 1 launches). Every result must equal, bit for bit, the result of the same call before the
preset, with no device error raised (an expired wait would raise MOA_DEVERR_SPIN_TIMEOUT)."""
import ctypes as C

import numpy as np
import pytest

from gpu_util import dev, dev_zeros, host, need_gpu, say, torch
from moa_amd import synth

pytestmark = pytest.mark.gpu


def preset(launches: int) -> None:
    from moa_amd import _lib
    _lib.call("moa_test_preset_epochs", C.c_uint64(launches))


@pytest.fixture(scope="module")
def calls():
    """One closure per operator: runs the one-token call on fixed device inputs, returns host bits."""
    need_gpu()
    from moa_amd import ops
    f = synth.cfg_ffn_fp8(3)
    ft = {k: dev(v) for k, v in f.items() if isinstance(v, np.ndarray)}
    o = synth.cfg_o(3)
    ot = {k: dev(v) for k, v in o.items() if isinstance(v, np.ndarray)}
    q = synth.cfg_qkv(3)
    qt = {k: dev(v) for k, v in q.items() if isinstance(v, np.ndarray)}
    kv = torch.tensor([q["kv_offset"]], dtype=torch.int32, device="cuda")
    ro = torch.tensor([q["rope_offset"]], dtype=torch.int32, device="cuda")
    a = synth.cfg_attention(seed=3, M=1, pos=900)
    at = {k: dev(v) for k, v in a.items()}

    def ffn():
        r = ft["residual"].clone()
        ops.decoder_feedforward_fp8(r, ft["pre_ff_rms_weight"], ft["up_weight"], ft["gate_weight"], ft["down_weight"],
                                    ft["up_weight_scale"], ft["gate_weight_scale"], ft["down_weight_scale"],
                                    ft["post_ff_rms_weight"], ft["layer_scalar"])
        return host(r)

    r16 = dev(synth.bf16_normal("epochs.rows16", (16, 3840)))

    def ffn_rows():
        r = r16.clone()
        ops.decoder_feedforward_fp8(r, ft["pre_ff_rms_weight"], ft["up_weight"], ft["gate_weight"], ft["down_weight"],
                                    ft["up_weight_scale"], ft["gate_weight_scale"], ft["down_weight_scale"],
                                    ft["post_ff_rms_weight"], ft["layer_scalar"])
        return host(r)

    def o_proj():
        r = ot["residual"].clone()
        ops.sliding_attention_output(ot["x"], ot["post_attn_rms_weight"], ot["o_weight"], ot["o_weight_scale"], r)
        return host(r)

    def qkv():
        kc, vc, qo = qt["k_cache"].clone(), qt["v_cache"].clone(), dev_zeros(4096)
        ops.sliding_project_qkv(qt["x"], qt["q_weight"], qt["k_weight"], qt["v_weight"], qt["q_weight_scale"],
                                qt["k_weight_scale"], qt["v_weight_scale"], qt["input_rms_weight"], qt["q_rms_weight"],
                                qt["k_rms_weight"], kv, ro, qt["cos"], qt["sin"], kc, vc, qo)
        return np.concatenate([host(qo), host(kc).reshape(-1), host(vc).reshape(-1)])

    def attn():
        out = dev_zeros(4096)
        ops.sliding_attention(at["q"], at["k_cache"], at["v_cache"], at["mask"], out)
        return host(out)

    return {"ffn": ffn, "ffn_rows": ffn_rows, "o": o_proj, "qkv": qkv, "attention": attn}


@pytest.mark.parametrize("start", [2**27 - 2, 2**28 - 2, 2**32 - 3])
def test_results_unchanged_across_epoch_wraps(calls, start):
    from moa_amd import ops
    say(f"epochs: reference results, then preset {start:#x} and 4 launches of each operator")
    want = {k: fn() for k, fn in calls.items()}
    assert ops.device_errors() == 0
    preset(start)
    for i in range(4):
        for k, fn in calls.items():
            assert np.array_equal(fn(), want[k]), f"{k}: launch {i} after preset {start:#x} differs"
    assert ops.device_errors() == 0
