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


def test_graph_replays_of_the_next_row_operators_match_eager():
    """sliding_attention, the full-attention layer (QKV, pages per call and fused, output) and
    final_norm_and_logits captured in one graph: every replay gives the eager bits."""
    need_gpu()
    from moa_amd import ops
    ops.init(0)
    at = synth.cfg_attention(3, M=1, pos=700)
    A = {k: dev(at[k]) for k in ("q", "k_cache", "v_cache", "mask")}
    a_out = torch.zeros(4096, dtype=torch.int16, device="cuda")
    fq = synth.cfg_full_qkv(3, pos=1500)
    F = {k: dev(fq[k]) for k in ("x", "q_weight", "k_weight", "q_weight_scale", "k_weight_scale", "input_rms_weight",
                                 "q_rms_weight", "k_rms_weight", "cos", "sin")}
    kv = torch.tensor([fq["kv_offset"]], dtype=torch.int32, device="cuda")
    ro = torch.tensor([fq["rope_offset"]], dtype=torch.int32, device="cuda")
    fa = synth.cfg_full_attention(3, M=1, P=12, q_std=0.3)
    kp0, vp0 = dev(fa["k_pages"]), dev(fa["v_pages"])
    kp, vp = kp0.clone(), vp0.clone()
    masks = dev(fa["masks"])
    q_f = torch.zeros(8192, dtype=torch.int16, device="cuda")
    mx1, sm1, out1 = (torch.zeros(16, device="cuda"), torch.zeros(16, device="cuda"),
                      torch.zeros(8192, dtype=torch.int16, device="cuda"))
    mx2, sm2, out2 = (torch.zeros(16, device="cuda"), torch.zeros(16, device="cuda"),
                      torch.zeros(8192, dtype=torch.int16, device="cuda"))
    fo = synth.cfg_full_o(3)
    O = {k: dev(fo[k]) for k in ("o_weight", "o_weight_scale", "post_attn_rms_weight")}
    res0 = dev(fo["residual"])
    res = res0.clone()
    lg = synth.cfg_logits(3)
    L = {k: dev(lg[k]) for k in ("input", "rms_weight")}
    lm = synth.lm_head_device(3)
    logits = torch.zeros(synth.W, dtype=torch.int16, device="cuda")

    def step():
        kp.copy_(kp0)
        vp.copy_(vp0)
        res.copy_(res0)
        ops.sliding_attention(A["q"], A["k_cache"], A["v_cache"], A["mask"], a_out)
        page = 1500 // 512
        ops.full_project_qkv(F["x"], F["q_weight"], F["k_weight"], F["q_weight_scale"], F["k_weight_scale"],
                             F["input_rms_weight"], F["q_rms_weight"], F["k_rms_weight"], kv, ro, F["cos"], F["sin"],
                             kp[page], vp[page], q_f)
        for p in range(12):
            fn = ops.full_attention_first_page if p == 0 else ops.full_attention_page
            fn(q_f, kp[p], vp[p], masks[p], mx1, sm1, out1)
        ops.full_attention(q_f, kp, vp, masks, mx2, sm2, out2)
        ops.full_attention_output(out2, sm2, O["post_attn_rms_weight"], O["o_weight"], O["o_weight_scale"], res)
        ops.final_norm_and_logits(L["input"], L["rms_weight"], lm, logits)

    outs = (a_out, kp, vp, q_f, mx1, sm1, out1, mx2, sm2, out2, res, logits)
    names = ("attn", "k_pages", "v_pages", "q_f", "max", "sum", "out", "fused max", "fused sum", "fused out",
             "residual", "logits")
    step()
    torch.cuda.synchronize()
    assert ops.device_errors() == 0
    want = [host(t).copy() for t in outs]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for replay in range(3):
        say(f"next-row graph replay {replay}")
        for t in (a_out, q_f, out1, out2, logits):
            t.fill_(0)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for w, t, name in zip(want, outs, names):
            assert np.array_equal(w, host(t)), f"replay {replay}: {name} differs from the eager result"
    assert ops.device_errors() == 0


def test_graph_replays_of_the_16_row_operators_match_eager():
    """16 token rows: the one-launch rows FFN (MXFP4 and FP8: pre-norm, contractions and post step
    in one kernel with tagged flags), O then the FFN through one entry point (O's post rows on the
    FFN kernel's service workgroups), and the rows-path QKV and O, captured in one graph: every
    replay gives the eager bits (the hand-off tags come from device-side epoch counters, so a
    replayed launch never meets a flag of an earlier replay)."""
    need_gpu()
    from moa_amd import ops
    ops.init(0)
    mx = synth.cfg_ffn_mxfp4(4)
    f = synth.cfg_ffn_fp8(4)
    o = synth.cfg_o(4, M=16)
    q = synth.cfg_qkv(4, M=16, pos=600)
    MXK = ("up_weight_packed", "gate_weight_packed", "down_weight_packed", "up_weight_scale", "gate_weight_scale",
           "down_weight_scale")
    FK = ("up_weight", "gate_weight", "down_weight", "up_weight_scale", "gate_weight_scale", "down_weight_scale")
    M_ = {k: dev(mx[k]) for k in MXK}
    F_ = {k: dev(f[k]) for k in FK}
    pre, post, ls = (dev(f[k]) for k in ("pre_ff_rms_weight", "post_ff_rms_weight", "layer_scalar"))
    O_ = {k: dev(o[k]) for k in ("x", "o_weight", "o_weight_scale", "post_attn_rms_weight")}
    Q_ = {k: dev(q[k]) for k in ("x", "q_weight", "k_weight", "v_weight", "q_weight_scale", "k_weight_scale",
                                 "v_weight_scale", "input_rms_weight", "q_rms_weight", "k_rms_weight", "cos", "sin")}
    kv = torch.tensor([q["kv_offset"]], dtype=torch.int32, device="cuda")
    ro = torch.tensor([q["rope_offset"]], dtype=torch.int32, device="cuda")
    kc0, vc0 = dev(q["k_cache"]), dev(q["v_cache"])
    kc, vc = kc0.clone(), vc0.clone()
    q_out = torch.zeros(16 * 4096, dtype=torch.int16, device="cuda")
    r0 = dev(synth.bf16_normal("graph16.residual", (16, 3840)))
    r_mx, r_f8, r_of, r_o = r0.clone(), r0.clone(), r0.clone(), r0.clone()

    def step():
        for t in (r_mx, r_f8, r_of, r_o):
            t.copy_(r0)
        kc.copy_(kc0)
        vc.copy_(vc0)
        ops.decoder_feedforward_mxfp4(r_mx, pre, *[M_[k] for k in MXK], post, ls)
        ops.decoder_feedforward_fp8(r_f8, pre, *[F_[k] for k in FK], post, ls)
        ops.sliding_attention_output_feedforward_mxfp4(O_["x"], O_["post_attn_rms_weight"], O_["o_weight"],
                                                       O_["o_weight_scale"], r_of, pre, *[M_[k] for k in MXK], post,
                                                       ls)
        ops.sliding_attention_output(O_["x"], O_["post_attn_rms_weight"], O_["o_weight"], O_["o_weight_scale"], r_o)
        ops.sliding_project_qkv(Q_["x"], Q_["q_weight"], Q_["k_weight"], Q_["v_weight"], Q_["q_weight_scale"],
                                Q_["k_weight_scale"], Q_["v_weight_scale"], Q_["input_rms_weight"],
                                Q_["q_rms_weight"], Q_["k_rms_weight"], kv, ro, Q_["cos"], Q_["sin"], kc, vc, q_out)

    outs = (r_mx, r_f8, r_of, r_o, kc, vc, q_out)
    names = ("ffn mxfp4", "ffn fp8", "o -> ffn", "o", "k_cache", "v_cache", "q_out")
    step()
    torch.cuda.synchronize()
    assert ops.device_errors() == 0
    want = [host(t).copy() for t in outs]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for replay in range(3):
        say(f"16-row graph replay {replay}")
        for t in (r_mx, r_f8, r_of, q_out):
            t.fill_(0)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for w, t, name in zip(want, outs, names):
            assert np.array_equal(w, host(t)), f"replay {replay}: {name} differs from the eager result"
        step()  # eager again
        torch.cuda.synchronize()
        assert np.array_equal(host(r_mx), want[0])
    assert ops.device_errors() == 0
