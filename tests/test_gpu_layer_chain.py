"""BASELINE config 4 as one decoder-layer chunk: QKV -> O -> FFN over M = 256 prefill rows at
positions 0..255, with the residual stream flowing through (the caller sequence of
FO/src/host/runtime.rs:401-460; the attention output that feeds O is a seeded bf16 input, as the
config says). The GPU chain runs on device buffers only -- the residual never leaves the device
between the operators -- and is compared with the oracle chain: q_out, every ring-cache slot
(slots 0..255 written, the other 768 bit-identical), the residual after O and after the FFN.
Each stage is also checked on its own input (the GPU's previous stage), so that a failure names
the operator."""
import numpy as np
import pytest

from gpu_util import dev, gate, gate_rope, host, need_gpu, say, torch
from kat_inputs import unbf
from moa_amd import synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu
M = 256


@pytest.mark.parametrize("seed", [0, 1])
def test_config4_layer_chain(seed):
    need_gpu()
    from moa_amd import ops
    say(f"config 4 chain seed {seed}: QKV -> O -> FFN, M={M}")
    c = synth.cfg_layer_chunk(seed, M=M)
    q = synth.cfg_qkv(seed)  # the configs' FP8 weights, norms and scales
    o = synth.cfg_o(seed)
    f = synth.cfg_ffn_fp8(seed)
    fw = O.ffn_weights(O.FFN_FP8, f["up_weight"], f["gate_weight"], f["down_weight"], f["up_weight_scale"],
                       f["gate_weight_scale"], f["down_weight_scale"])

    # GPU chain
    x = dev(c["x"])
    kc, vc = dev(c["k_cache"]), dev(c["v_cache"])
    qo = dev(np.zeros(M * 4096, np.uint16))
    kv = torch.zeros(1, dtype=torch.int32, device="cuda")
    ro = torch.zeros(1, dtype=torch.int32, device="cuda")
    ops.sliding_project_qkv(x, dev(q["q_weight"]), dev(q["k_weight"]), dev(q["v_weight"]), dev(q["q_weight_scale"]),
                            dev(q["k_weight_scale"]), dev(q["v_weight_scale"]), dev(q["input_rms_weight"]),
                            dev(q["q_rms_weight"]), dev(q["k_rms_weight"]), kv, ro, dev(c["cos"]), dev(c["sin"]),
                            kc, vc, qo)
    ops.sliding_attention_output(dev(c["attn"]), dev(o["post_attn_rms_weight"]), dev(o["o_weight"]),
                                 dev(o["o_weight_scale"]), x)
    after_o = host(x).reshape(M, 3840).copy()
    ops.decoder_feedforward_fp8(x, dev(f["pre_ff_rms_weight"]), dev(f["up_weight"]), dev(f["gate_weight"]),
                                dev(f["down_weight"]), dev(f["up_weight_scale"]), dev(f["gate_weight_scale"]),
                                dev(f["down_weight_scale"]), dev(f["post_ff_rms_weight"]), dev(f["layer_scalar"]))
    out = host(x).reshape(M, 3840)
    g_q, g_k, g_v = host(qo), host(kc), host(vc)
    assert ops.device_errors() == 0

    # oracle chain
    r = c["x"].copy()
    k_e, v_e, q_e = c["k_cache"].copy(), c["v_cache"].copy(), np.zeros(M * 4096, np.uint16)
    O.sliding_project_qkv(r, q["q_weight"], q["k_weight"], q["v_weight"], q["q_weight_scale"], q["k_weight_scale"],
                          q["v_weight_scale"], q["input_rms_weight"], q["q_rms_weight"], q["k_rms_weight"], 0, 0,
                          c["cos"], c["sin"], k_e, v_e, q_e)
    O.sliding_attention_output(c["attn"], o["post_attn_rms_weight"], o["o_weight"], o["o_weight_scale"], r)
    o_e = r.copy()
    O.decoder_feedforward(r, f["pre_ff_rms_weight"], fw, f["post_ff_rms_weight"], f["layer_scalar"])

    gate_rope(q_e, g_q, "chain q_out", 256)
    gate_rope(k_e[:M], g_k[:M], "chain k slots 0..255", 256)
    gate(v_e[:M], g_v[:M], "chain v slots 0..255")
    assert np.array_equal(g_k[M:], c["k_cache"][M:]) and np.array_equal(g_v[M:], c["v_cache"][M:])
    gate(o_e, after_o, "chain residual after O")
    gate(r, out, "chain residual after FFN (end to end)")
    # the FFN stage on the GPU's own O output
    r_stage = after_o.copy()
    O.decoder_feedforward(r_stage, f["pre_ff_rms_weight"], fw, f["post_ff_rms_weight"], f["layer_scalar"])
    gate(r_stage, out, "chain FFN stage")
