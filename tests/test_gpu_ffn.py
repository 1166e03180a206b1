"""ops::decoder_feedforward (NVFP4, as the reference), and the FP8 / MXFP4 weight variants,
on the GPU vs the CPU oracle and the reference's known answer."""
import numpy as np
import pytest

from gpu_util import dev, gate, host, need_gpu, say, torch
from kat_inputs import GOLDEN, ffn_stress_inputs, ffn_stress_inputs_fp8, ffn_stress_inputs_mxfp4, unbf
from moa_amd import prng, synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu

FFN_ATOL = 1e-2  # the reference's own FFN atol (test_kernels.rs:461-464) equals BASELINE's


def gpu_nvfp4(d):
    from moa_amd import ops
    r = dev(d["residual"])
    ops.decoder_feedforward(r, dev(d["pre_ff_rms_weight"]), dev(d["up_weight_packed"]), dev(d["gate_weight_packed"]),
                            dev(d["down_weight_packed"]), dev(d["up_weight_scale"]), dev(d["gate_weight_scale"]),
                            dev(d["down_weight_scale"]), dev(d["up_global_scale"]), dev(d["gate_global_scale"]),
                            dev(d["down_global_scale"]), dev(d["post_ff_rms_weight"]), dev(d["layer_scalar"]))
    return host(r)


def oracle_nvfp4(d):
    w = O.ffn_weights(O.FFN_NVFP4, d["up_weight_packed"], d["gate_weight_packed"], d["down_weight_packed"],
                      d["up_weight_scale"], d["gate_weight_scale"], d["down_weight_scale"],
                      (d["up_global_scale"][0], d["gate_global_scale"][0], d["down_global_scale"][0]))
    r = d["residual"].copy()
    O.decoder_feedforward(r, d["pre_ff_rms_weight"], w, d["post_ff_rms_weight"], d["layer_scalar"])
    return r


def gpu_fp8(d, post=True, ls=True):
    from moa_amd import ops
    r = dev(d["residual"])
    ops.decoder_feedforward_fp8(r, dev(d["pre_ff_rms_weight"]), dev(d["up_weight"]), dev(d["gate_weight"]),
                                dev(d["down_weight"]), dev(d["up_weight_scale"]), dev(d["gate_weight_scale"]),
                                dev(d["down_weight_scale"]), dev(d["post_ff_rms_weight"]) if post else None,
                                dev(d["layer_scalar"]) if ls else None)
    return host(r)


def oracle_fp8(d, post=True, ls=True):
    w = O.ffn_weights(O.FFN_FP8, d["up_weight"], d["gate_weight"], d["down_weight"], d["up_weight_scale"],
                      d["gate_weight_scale"], d["down_weight_scale"])
    r = d["residual"].copy()
    O.decoder_feedforward(r, d["pre_ff_rms_weight"], w, d["post_ff_rms_weight"] if post else None,
                          d["layer_scalar"] if ls else None)
    return r


def gpu_mxfp4(d):
    from moa_amd import ops
    r = dev(d["residual"])
    ops.decoder_feedforward_mxfp4(r, dev(d["pre_ff_rms_weight"]), dev(d["up_weight_packed"]),
                                  dev(d["gate_weight_packed"]), dev(d["down_weight_packed"]),
                                  dev(d["up_weight_scale"]), dev(d["gate_weight_scale"]),
                                  dev(d["down_weight_scale"]), dev(d["post_ff_rms_weight"]), dev(d["layer_scalar"]))
    return host(r)


def oracle_mxfp4(d):
    w = O.ffn_weights(O.FFN_MXFP4, d["up_weight_packed"], d["gate_weight_packed"], d["down_weight_packed"],
                      d["up_weight_scale"], d["gate_weight_scale"], d["down_weight_scale"])
    r = d["residual"].copy()
    O.decoder_feedforward(r, d["pre_ff_rms_weight"], w, d["post_ff_rms_weight"], d["layer_scalar"])
    return r


def test_nvfp4_stress_known_answer():
    """full-ffn-stress: 3840 x 0x3ecf through the reference-contract NVFP4 entry point."""
    need_gpu()
    say("ffn nvfp4 stress")
    got = gpu_nvfp4(ffn_stress_inputs())
    want = np.fromfile(GOLDEN / "ffn_stress_expected_bf16.bin", dtype="<u2")
    assert np.array_equal(got, want)


@pytest.mark.parametrize("M", [1, 16, 256])
@pytest.mark.parametrize("fmt", ["fp8", "mxfp4"])
def test_stress_known_answer_other_formats(fmt, M):
    """The FP8 and MXFP4 restatements of full-ffn-stress (the same intermediates, closed-form
    answer 3840 x 0x3ecf, pinned on the oracle in test_oracle_ffn_formats.py) through the
    one-token kernel (M = 1), the rows kernels (M = 16) and the MFMA chunk path (M = 256)."""
    need_gpu()
    say(f"ffn {fmt} stress M{M}")
    d = ffn_stress_inputs_fp8() if fmt == "fp8" else ffn_stress_inputs_mxfp4()
    d["residual"] = np.broadcast_to(d["residual"], (M, 3840)).copy()
    got = (gpu_fp8 if fmt == "fp8" else gpu_mxfp4)(d)
    assert np.all(np.asarray(got).reshape(-1) == 0x3ECF), np.unique(got)


@pytest.mark.parametrize("run", range(9))
def test_nvfp4_reference_runs(run):
    """The reference harness's runs 0-2 (FO/src/bin/test_kernels.rs:168) and the extra runs 3-8 of
    its development sweep (moa-dev/extra_seeds.py:25,103-110: same names, RUN_OFFSET 3)."""
    need_gpu()
    say(f"ffn nvfp4 reference run {run}")
    d = synth.ref_ffn_inputs(run)
    gate(oracle_nvfp4(d), gpu_nvfp4(d), f"ffn nvfp4 run{run}", atol=FFN_ATOL)


@pytest.fixture(scope="module")
def cfg0():
    return synth.cfg_ffn_fp8(0)


@pytest.mark.parametrize("seed", range(3))
def test_fp8_config0(seed, cfg0):
    """BASELINE config 0 (the headline case) at M = 1, three seeds."""
    need_gpu()
    say(f"ffn fp8 cfg0 seed{seed}")
    d = cfg0 if seed == 0 else synth.cfg_ffn_fp8(seed)
    gate(oracle_fp8(d), gpu_fp8(d), f"ffn fp8 cfg0 seed{seed}", atol=FFN_ATOL)


def test_fp8_config0_literal_without_post_norm_and_gate(cfg0):
    """BASELINE config 0 read literally: pre-RMSNorm -> GeGLU -> down -> residual add."""
    need_gpu()
    gate(oracle_fp8(cfg0, False, False), gpu_fp8(cfg0, False, False), "ffn fp8 cfg0 literal", atol=FFN_ATOL)


def test_fp8_multi_row_and_determinism():
    need_gpu()
    d = synth.cfg_ffn_fp8(1, M=2)
    a = gpu_fp8(d)
    gate(oracle_fp8(d), a, "ffn fp8 M2", atol=FFN_ATOL)
    assert np.array_equal(a, gpu_fp8(d))


@pytest.mark.parametrize("M", [1, 16])
def test_mxfp4_config3(M):
    need_gpu()
    say(f"ffn mxfp4 cfg3 M{M}")
    d = synth.cfg_ffn_mxfp4(0, M=M)
    gate(oracle_mxfp4(d), gpu_mxfp4(d), f"ffn mxfp4 M{M}", atol=FFN_ATOL)


def cancel_fp4_codes(packed: np.ndarray) -> np.ndarray:
    """E2M1 rows whose elements 480k and 480k + 1 (the two nibbles of byte 240k, inside one block
    scale in both FP4 formats) carry the same code, as full-ffn-stress builds its rows from
    repeated codes (full-ffn-stress/generate_reference.py:44-60): weighted +a and -a, the
    normalised cancelling pair contributes exactly zero in every row."""
    w = packed.copy()
    lo = w[:, 0::240] & 0x0F
    w[:, 0::240] = lo | (lo << 4)
    return w


def cancellation_probe(d: dict, tiny_pow: int, fp8: bool) -> dict:
    """The probe applied to one FFN case: residual [+1, -1, 478 x 2^p] per 480, unit pre-norm
    weight, and up/gate rows that weight the pair equally."""
    d = dict(d)
    d["residual"] = cancellation_residual(tiny_pow)[None, :]
    d["pre_ff_rms_weight"] = np.full(3840, 0x3F80, np.uint16)
    for k in ("up", "gate"):
        if fp8:
            w = d[f"{k}_weight"].copy()
            w[:, 0::480] = 0x38  # 1.0
            w[:, 1::480] = 0x38
            d[f"{k}_weight"] = w
        else:
            d[f"{k}_weight_packed"] = cancel_fp4_codes(d[f"{k}_weight_packed"])
    return d


def assert_geglu_near_zero(d: dict, fmt: int, label: str, bound: float = 1e-2) -> float:
    """The oracle's GeGLU row p of a probe really is near zero (the pair cancelled): returns max |p|."""
    keys = ("up_weight", "gate_weight", "down_weight") if fmt == O.FFN_FP8 else \
        ("up_weight_packed", "gate_weight_packed", "down_weight_packed")
    g = (d["up_global_scale"][0], d["gate_global_scale"][0], d["down_global_scale"][0]) if fmt == O.FFN_NVFP4 \
        else (1.0, 1.0, 1.0)
    w = O.ffn_weights(fmt, *[d[k] for k in keys], d["up_weight_scale"], d["gate_weight_scale"], d["down_weight_scale"],
                      g)
    h = O.rmsnorm(np.ascontiguousarray(d["residual"]), d["pre_ff_rms_weight"])
    p = unbf(O.ffn_up_gate(h, w))
    mp = float(np.abs(p).max())
    say(f"[{label:40}] oracle max|GeGLU| = {mp:.3e}")
    assert mp < bound, f"{label}: the probe did not cancel (max |p| {mp})"
    return mp


def cancellation_residual(tiny_pow: int) -> np.ndarray:
    """residual chunk [+1, -1, 478 x 2^p] per 480 (the QKV probe's construction,
    qkv-boundary-probe-e53/generate_suite.py:48-49): after the pre-norm the large pair cancels
    exactly in every projection row that weights it [1, 1, ...], leaving the tiny terms."""
    x = np.full(3840, 2.0 ** tiny_pow, np.float32)
    x[0::480], x[1::480] = 1.0, -1.0
    return prng.f32_to_bf16_bits(x)


@pytest.mark.parametrize("tiny_pow", [-23, -12])
@pytest.mark.parametrize("fmt", ["fp8", "mxfp4", "nvfp4"])
def test_cancellation_probes(fmt, tiny_pow):
    """BASELINE config 3's cancellation probe (and the same in FP8 and NVFP4): up . gelu(gate)
    partial sums near zero, asserted on the oracle's GeGLU row before the kernel is compared."""
    need_gpu()
    say(f"ffn {fmt} cancellation probe 2^{tiny_pow}")
    base = {"fp8": lambda: synth.cfg_ffn_fp8(4), "mxfp4": lambda: synth.cfg_ffn_mxfp4(4),
            "nvfp4": lambda: synth.ref_ffn_inputs(4)}[fmt]()
    d = cancellation_probe(base, tiny_pow, fmt == "fp8")
    assert_geglu_near_zero(d, {"fp8": O.FFN_FP8, "mxfp4": O.FFN_MXFP4, "nvfp4": O.FFN_NVFP4}[fmt],
                           f"ffn {fmt} cancel 2^{tiny_pow}")
    want, got = {"fp8": (oracle_fp8, gpu_fp8), "mxfp4": (oracle_mxfp4, gpu_mxfp4),
                 "nvfp4": (oracle_nvfp4, gpu_nvfp4)}[fmt]
    gate(want(d), got(d), f"ffn {fmt} cancel 2^{tiny_pow}", atol=FFN_ATOL)
