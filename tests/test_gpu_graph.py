"""The three operators captured in one HIP graph (as a decode loop would replay them) give the
eager results on every replay, with eager work and synchronisations between replays. The
library records no memset into the graph; its arrival counters reset themselves."""
import numpy as np
import pytest

from gpu_util import dev, host, need_gpu, say, torch
from moa_amd import synth

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager():
    need_gpu()
    from moa_amd import ops
    ops.init(0)
    f = synth.cfg_ffn_fp8(2)
    o = synth.cfg_o(2)
    q = synth.cfg_qkv(2)
    Fw = {k: dev(f[k]) for k in ("up_weight", "gate_weight", "down_weight", "up_weight_scale", "gate_weight_scale",
                                 "down_weight_scale", "pre_ff_rms_weight", "post_ff_rms_weight", "layer_scalar")}
    Ow = {k: dev(o[k]) for k in ("o_weight", "o_weight_scale", "post_attn_rms_weight", "x")}
    Qw = {k: dev(q[k]) for k in ("x", "q_weight", "k_weight", "v_weight", "q_weight_scale", "k_weight_scale",
                                 "v_weight_scale", "input_rms_weight", "q_rms_weight", "k_rms_weight", "cos", "sin")}
    kv = torch.tensor([q["kv_offset"]], dtype=torch.int32, device="cuda")
    ro = torch.tensor([q["rope_offset"]], dtype=torch.int32, device="cuda")
    res0, kc0, vc0 = dev(o["residual"]), dev(q["k_cache"]), dev(q["v_cache"])
    res, kc, vc = res0.clone(), kc0.clone(), vc0.clone()
    q_out = torch.zeros(4096, dtype=torch.int16, device="cuda")

    def step():
        res.copy_(res0)
        kc.copy_(kc0)
        vc.copy_(vc0)
        ops.sliding_project_qkv(Qw["x"], Qw["q_weight"], Qw["k_weight"], Qw["v_weight"], Qw["q_weight_scale"],
                                Qw["k_weight_scale"], Qw["v_weight_scale"], Qw["input_rms_weight"],
                                Qw["q_rms_weight"], Qw["k_rms_weight"], kv, ro, Qw["cos"], Qw["sin"], kc, vc, q_out)
        ops.sliding_attention_output(Ow["x"], Ow["post_attn_rms_weight"], Ow["o_weight"], Ow["o_weight_scale"], res)
        ops.decoder_feedforward_fp8(res, Fw["pre_ff_rms_weight"], Fw["up_weight"], Fw["gate_weight"],
                                    Fw["down_weight"], Fw["up_weight_scale"], Fw["gate_weight_scale"],
                                    Fw["down_weight_scale"], Fw["post_ff_rms_weight"], Fw["layer_scalar"])

    step()
    want = [host(t).copy() for t in (res, kc, vc, q_out)]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for replay in range(4):
        say(f"graph replay {replay}")
        res.fill_(0)  # eager work between replays
        q_out.fill_(0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = [host(t) for t in (res, kc, vc, q_out)]
        for w, x, name in zip(want, got, ("residual", "k_cache", "v_cache", "q_out")):
            assert np.array_equal(w, x), f"replay {replay}: {name} differs from the eager result"
        step()  # eager again, then compare once more
        torch.cuda.synchronize()
        assert np.array_equal(host(res), want[0])
    assert ops.device_errors() == 0
