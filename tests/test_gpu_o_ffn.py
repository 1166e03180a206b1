"""The O -> FFN entry points (the tail of the reference's sliding-layer decode step,
FO/src/host/runtime.rs:440-459 then 543-571) on the GPU. The residual afterwards must have the same
bits as sliding_attention_output followed by decoder_feedforward through their own entry points,
and meet the gate against the oracle's chain of the two operators; one token row runs as one
launch (o_ffn_fused_kernel); from three rows on O's post rows also write the FFN's normalised
input (one kernel fewer), and two rows run the two operators in turn."""
import numpy as np
import pytest

from gpu_util import dev, gate, gate_addend, host, need_gpu, say
from kat_inputs import ffn_stress_inputs, unbf
from moa_amd import prng, synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu

FFN_ATOL = 1e-2  # the reference's FFN atol (test_kernels.rs:461-464), BASELINE's as well

FP8_KEYS = ("pre_ff_rms_weight", "up_weight", "gate_weight", "down_weight", "up_weight_scale", "gate_weight_scale",
            "down_weight_scale")
FP4_KEYS = ("pre_ff_rms_weight", "up_weight_packed", "gate_weight_packed", "down_weight_packed", "up_weight_scale",
            "gate_weight_scale", "down_weight_scale")
NV_GLOBALS = ("up_global_scale", "gate_global_scale", "down_global_scale")


def o_scale(o, bf16):
    s = o["o_weight_scale"]
    if bf16:
        return s if s.dtype == np.uint16 else prng.f32_to_bf16_bits(s)
    return s if s.dtype == np.float32 else unbf(s)


def opt(f, key, on):
    return dev(f[key]) if on else None


def gpu_fused(fmt, o, f, post=True, ls=True):
    """One call of the O -> FFN entry point of `fmt` on O's residual."""
    from moa_amd import ops
    r = dev(o["residual"])
    oa = [dev(o["x"]), dev(o["post_attn_rms_weight"]), dev(o["o_weight"]), dev(o_scale(o, fmt == "nvfp4")), r]
    if fmt == "fp8":
        ops.sliding_attention_output_feedforward_fp8(*oa, *[dev(f[k]) for k in FP8_KEYS],
                                                     opt(f, "post_ff_rms_weight", post), opt(f, "layer_scalar", ls))
    elif fmt == "mxfp4":
        ops.sliding_attention_output_feedforward_mxfp4(*oa, *[dev(f[k]) for k in FP4_KEYS],
                                                       opt(f, "post_ff_rms_weight", post), opt(f, "layer_scalar", ls))
    else:
        ops.sliding_attention_output_feedforward(*oa, *[dev(f[k]) for k in FP4_KEYS + NV_GLOBALS],
                                                 dev(f["post_ff_rms_weight"]), dev(f["layer_scalar"]))
    return host(r)


def gpu_two_calls(fmt, o, f, post=True, ls=True):
    """sliding_attention_output, then the FFN entry point of `fmt`, on O's residual."""
    from moa_amd import ops
    r = dev(o["residual"])
    ops.sliding_attention_output(dev(o["x"]), dev(o["post_attn_rms_weight"]), dev(o["o_weight"]),
                                 dev(o_scale(o, fmt == "nvfp4")), r)
    if fmt == "fp8":
        ops.decoder_feedforward_fp8(r, *[dev(f[k]) for k in FP8_KEYS], opt(f, "post_ff_rms_weight", post),
                                    opt(f, "layer_scalar", ls))
    elif fmt == "mxfp4":
        ops.decoder_feedforward_mxfp4(r, *[dev(f[k]) for k in FP4_KEYS], opt(f, "post_ff_rms_weight", post),
                                      opt(f, "layer_scalar", ls))
    else:
        ops.decoder_feedforward(r, *[dev(f[k]) for k in FP4_KEYS + NV_GLOBALS], dev(f["post_ff_rms_weight"]),
                                dev(f["layer_scalar"]))
    return host(r)


def oracle_chain(fmt, o, f, post=True, ls=True):
    """The oracle's sliding_attention_output, then its decoder_feedforward."""
    r = o["residual"].copy()
    O.sliding_attention_output(o["x"], o["post_attn_rms_weight"], o["o_weight"], unbf(o_scale(o, True))
                               if fmt == "nvfp4" else o_scale(o, False), r)
    if fmt == "fp8":
        w = O.ffn_weights(O.FFN_FP8, *[f[k] for k in FP8_KEYS[1:]])
    elif fmt == "mxfp4":
        w = O.ffn_weights(O.FFN_MXFP4, *[f[k] for k in FP4_KEYS[1:]])
    else:
        w = O.ffn_weights(O.FFN_NVFP4, *[f[k] for k in FP4_KEYS[1:]], tuple(f[k][0] for k in NV_GLOBALS))
    O.decoder_feedforward(r, f["pre_ff_rms_weight"], w, f["post_ff_rms_weight"] if post else None,
                          f["layer_scalar"] if ls else None)
    return r


def check(fmt, o, f, label, post=True, ls=True):
    got = gpu_fused(fmt, o, f, post, ls)
    two = gpu_two_calls(fmt, o, f, post, ls)
    diff = np.count_nonzero(got.reshape(-1) != two.reshape(-1))
    say(f"[{label:40}] fused vs two calls: {diff} of {got.size} differ")
    assert diff == 0
    gate(oracle_chain(fmt, o, f, post, ls), got, label, atol=FFN_ATOL)
    return got


@pytest.mark.parametrize("seed", range(3))
def test_fp8_configs_1_then_0(seed):
    """BASELINE config 1 (O) feeding config 0 (FP8 FFN) at M = 1, three seeds."""
    need_gpu()
    say(f"o->ffn fp8 seed{seed}")
    check("fp8", synth.cfg_o(seed), synth.cfg_ffn_fp8(seed), f"o->ffn fp8 seed{seed}")


def test_fp8_without_post_norm_and_scalar():
    need_gpu()
    say("o->ffn fp8 without post-norm and layer scalar")
    check("fp8", synth.cfg_o(1), synth.cfg_ffn_fp8(1), "o->ffn fp8 literal", post=False, ls=False)


@pytest.mark.parametrize("run", range(3))
def test_nvfp4_reference_runs(run):
    """The reference harness's O and FFN inputs of runs 0-2 (test_kernels.rs:548-624), chained as
    the runtime chains them: bf16 O scales, NVFP4 FFN."""
    need_gpu()
    say(f"o->ffn nvfp4 run{run}")
    check("nvfp4", synth.ref_o_inputs(run), synth.ref_ffn_inputs(run), f"o->ffn nvfp4 run{run}")


def test_mxfp4_config3():
    need_gpu()
    say("o->ffn mxfp4")
    check("mxfp4", synth.cfg_o(2), synth.cfg_ffn_mxfp4(0), "o->ffn mxfp4")


def test_zero_attention_row_then_ffn_stress_known_answer():
    """A zero attention row leaves the residual unchanged through O (d = 0, so RMSNorm(d) = 0
    whatever the weights: output-boundary-probe-e47 case 0), so the chain on full-ffn-stress's
    residual and NVFP4 weights must give that fixture's closed form, 3840 x 0x3ecf."""
    need_gpu()
    say("o->ffn zero row + nvfp4 stress")
    f = ffn_stress_inputs()
    o = synth.ref_o_inputs(0)
    o["x"] = np.zeros_like(o["x"])
    o["residual"] = f["residual"].copy()
    got = gpu_fused("nvfp4", o, f)
    assert np.all(got == 0x3ECF), np.unique(got)


def test_two_rows_run_the_two_operators():
    """Two token rows: the entry point runs the operators in turn (the same bits as the two calls)."""
    need_gpu()
    say("o->ffn fp8 M2")
    check("fp8", synth.cfg_o(0, M=2), synth.cfg_ffn_fp8(0, M=2), "o->ffn fp8 M2")


# 3..16 rows: the rows path, where O's post rows write the FFN's row-major normalised input
# (chunk_post_pre_rows_kernel<.., false>) and the FFN starts at its up/gate contraction
@pytest.mark.parametrize("fmt,M", [("fp8", 3), ("fp8", 7), ("fp8", 16), ("mxfp4", 16), ("nvfp4", 5)])
def test_rows_path_writes_the_ffn_input_with_the_o_post_norm(fmt, M):
    need_gpu()
    say(f"o->ffn {fmt} M{M} (rows path)")
    o, f = chunk_inputs(fmt, M)
    check(fmt, o, f, f"o->ffn {fmt} M{M} rows")


def test_rows_path_without_post_norm_and_scalar():
    """Without the FFN's post-norm (a mode the reference operator does not have) d is added to the
    residual unnormalised: the same bits as the two calls, and the oracle's chain within the gate
    for such sums (gate_addend: an f32 sum in the matrix cores' order may round d one bf16 ulp
    away from the oracle's, and that step reaches the output where r + d cancels)."""
    need_gpu()
    say("o->ffn fp8 M4 (rows path) without post-norm and layer scalar")
    o, f = chunk_inputs("fp8", 4)
    got = gpu_fused("fp8", o, f, False, False)
    two = gpu_two_calls("fp8", o, f, False, False)
    assert np.array_equal(got, two), f"{np.count_nonzero(got != two)} elements differ from the two calls"
    mid = o["residual"].copy()
    O.sliding_attention_output(o["x"], o["post_attn_rms_weight"], o["o_weight"], o_scale(o, False), mid)
    gate_addend(oracle_chain("fp8", o, f, False, False), got, mid, "o->ffn fp8 M4 rows literal", atol=FFN_ATOL)


def test_rows_path_bf16_o_scales():
    """The bf16-scale O entry point's rows path (the NVFP4 entry point takes bf16 O scales)
    feeding the FFN: O's scales read as bf16 by the shared row kernel."""
    need_gpu()
    say("o->ffn nvfp4 M16 (rows path, bf16 O scales)")
    o, f = chunk_inputs("nvfp4", 16)
    check("nvfp4", o, f, "o->ffn nvfp4 M16 rows")


def test_interleaved_with_the_ffn_entry_point():
    """The FFN half shares its hand-off words with decoder_feedforward_fp8 (tags from the same
    epoch counters): calls alternating between the two entry points keep giving the same bits."""
    need_gpu()
    o, f = synth.cfg_o(0), synth.cfg_ffn_fp8(0)
    want = gpu_fused("fp8", o, f)
    from test_gpu_ffn import gpu_fp8
    ffn_want = gpu_fp8(f)
    for i in range(3):
        assert np.array_equal(gpu_fused("fp8", o, f), want), f"fused call {i}"
        assert np.array_equal(gpu_fp8(f), ffn_want), f"ffn call {i}"


def chunk_inputs(fmt, M):
    """O inputs of M rows and FFN weights of `fmt` with their own M-row residual (O's is unused:
    the call runs on one residual, the FFN's)."""
    o = synth.cfg_o(3, M=M, tag="offn_chunk")
    if fmt == "fp8":
        f = synth.cfg_ffn_fp8(3, M=M, tag="offn_chunk")
    else:
        f = dict(synth.cfg_ffn_mxfp4(3) if fmt == "mxfp4" else synth.ref_ffn_inputs(3))
        f["residual"] = synth.bf16_normal(f"offn_chunk.{fmt}.M{M}.residual", (M, 3840))
    o["residual"] = f["residual"].copy()
    return o, f


# 1030 rows: two chunks of the MFMA path (1024 rows each at most), the second of 6 rows
@pytest.mark.parametrize("fmt,M", [("fp8", 17), ("fp8", 100), ("fp8", 300), ("mxfp4", 256), ("nvfp4", 64),
                                   ("fp8", 1030)])
def test_chunk_rows_write_the_ffn_input_with_the_o_post_norm(fmt, M):
    """More than 16 rows take the MFMA path, where O's post rows also write the FFN's normalised
    input (chunk_post_pre_rows_kernel) and the FFN starts at its GEMM: the same bits as the two
    calls (whose MFMA path runs the FFN's own norm kernel), and the oracle's chain within the gate."""
    need_gpu()
    say(f"o->ffn {fmt} M{M} (MFMA path)")
    o, f = chunk_inputs(fmt, M)
    got = gpu_fused(fmt, o, f)
    two = gpu_two_calls(fmt, o, f)
    diff = np.count_nonzero(got.reshape(-1) != two.reshape(-1))
    say(f"[o->ffn {fmt} M{M}] fused vs two calls: {diff} of {got.size} differ")
    assert diff == 0
    if M <= 100:
        gate(oracle_chain(fmt, o, f), got, f"o->ffn {fmt} M{M}", atol=FFN_ATOL)
