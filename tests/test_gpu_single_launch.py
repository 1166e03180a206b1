"""The single-launch kernels (one token row) and the MFMA path of longer calls.

Calls of more than 16 rows take the MFMA path (every weight format): 17 rows (a partial row tile),
64 (one full tile), 100 and 256 (BASELINE config 4's chunk length). Repeated calls interleaving
different inputs check that no launch ever reads a tagged hand-off word left by an earlier launch
(the tags are per-launch epochs): results must not depend on call history."""
import numpy as np
import pytest

from gpu_util import gate, gate_addend, need_gpu, say
from moa_amd import synth
from test_gpu_ffn import (FFN_ATOL, assert_geglu_near_zero, cancel_fp4_codes, cancellation_residual, gpu_fp8,
                          gpu_mxfp4, gpu_nvfp4, oracle_fp8, oracle_mxfp4, oracle_nvfp4)
from oracle import oracle as O
from test_gpu_o import run_gpu as o_gpu
from test_gpu_o import run_oracle as o_oracle
from test_gpu_qkv import check_against_oracle
from test_gpu_qkv import run_gpu as qkv_gpu

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M", [17, 64, 100, 256, 300])
def test_ffn_fp8_mfma_rows(M):
    need_gpu()
    say(f"ffn fp8 M{M} (MFMA path)")
    d = synth.cfg_ffn_fp8(5, M=M)
    gate(oracle_fp8(d), gpu_fp8(d), f"ffn fp8 M{M}", atol=FFN_ATOL)


_fp4 = {}


def fp4_case(fmt: str, M: int, tag: str = "mfma") -> dict:
    if fmt not in _fp4:
        _fp4[fmt] = synth.cfg_ffn_mxfp4(5) if fmt == "mxfp4" else synth.ref_ffn_inputs(5)
    return dict(_fp4[fmt], residual=synth.bf16_normal(f"{tag}.{fmt}.M{M}.residual", (M, 3840)))


@pytest.mark.parametrize("M", [17, 64, 256, 300])
@pytest.mark.parametrize("fmt", ["mxfp4", "nvfp4"])
def test_ffn_fp4_mfma_rows(fmt, M):
    """FP4 weights on the MFMA path: E2M1 codes widened with their block scales while they are
    staged (weights read once per 256 rows)."""
    need_gpu()
    say(f"ffn {fmt} M{M} (MFMA path)")
    d = fp4_case(fmt, M)
    want, got = (oracle_mxfp4, gpu_mxfp4) if fmt == "mxfp4" else (oracle_nvfp4, gpu_nvfp4)
    gate(want(d), got(d), f"ffn {fmt} M{M}", atol=FFN_ATOL)


@pytest.mark.parametrize("fmt", ["mxfp4", "nvfp4", "fp8"])
def test_ffn_mfma_rows_with_cancellation_probes(fmt):
    """BASELINE config 3's cancellation probe at config 4's chunk length: rows 1 and 3 of 256 cancel
    in every up/gate row (asserted near zero on the oracle), the rest are ordinary rows."""
    need_gpu()
    say(f"ffn {fmt} M256 with cancellation-probe rows (MFMA path)")
    d = fp4_case(fmt, 256, "probe") if fmt != "fp8" else dict(synth.cfg_ffn_fp8(5, M=256))
    d["residual"] = d["residual"].copy()
    d["residual"][1] = cancellation_residual(-23)
    d["residual"][3] = cancellation_residual(-12)
    d["pre_ff_rms_weight"] = np.full(3840, 0x3F80, np.uint16)
    for k in ("up", "gate"):
        if fmt == "fp8":
            w = d[f"{k}_weight"].copy()
            w[:, 0::480] = 0x38
            w[:, 1::480] = 0x38
            d[f"{k}_weight"] = w
        else:
            d[f"{k}_weight_packed"] = cancel_fp4_codes(d[f"{k}_weight_packed"])
    probes = dict(d, residual=np.ascontiguousarray(d["residual"][[1, 3]]))
    assert_geglu_near_zero(probes, {"fp8": O.FFN_FP8, "mxfp4": O.FFN_MXFP4, "nvfp4": O.FFN_NVFP4}[fmt],
                           f"ffn {fmt} M256 probes")
    want, got = {"fp8": (oracle_fp8, gpu_fp8), "mxfp4": (oracle_mxfp4, gpu_mxfp4),
                 "nvfp4": (oracle_nvfp4, gpu_nvfp4)}[fmt]
    gate(want(d), got(d), f"ffn {fmt} M256 probes", atol=FFN_ATOL)


def test_ffn_fp8_mfma_rows_without_post_norm_and_scalar():
    need_gpu()
    say("ffn fp8 M33 literal (MFMA path)")
    d = synth.cfg_ffn_fp8(8, M=33)
    gate_addend(oracle_fp8(d, False, False), gpu_fp8(d, False, False), d["residual"], "ffn fp8 M33 literal",
                atol=FFN_ATOL)


@pytest.mark.parametrize("M", [17, 64, 100, 256, 300])
def test_o_mfma_rows(M):
    need_gpu()
    say(f"o M{M} (MFMA path)")
    d = synth.cfg_o(5, M=M)
    gate(o_oracle(d), o_gpu(d), f"o M{M}")


# 300 and 600 rows: past one 256-row block, the QKV heads run four per workgroup (two k splits at
# 300 rows, none at 600), and rows past the last multiple of 64 keep their own tile producers.
@pytest.mark.parametrize("M", [17, 100, 256, 300, 600])
def test_qkv_mfma_rows(M):
    need_gpu()
    say(f"qkv M{M} (MFMA path)")
    d = synth.cfg_qkv(5, M=M, pos=1020)  # the ring wraps inside the call
    check_against_oracle(d, f"qkv M{M}", M=M)


def test_o_results_do_not_depend_on_call_history():
    need_gpu()
    say("o: a, b, a")
    a, b = synth.cfg_o(11), synth.cfg_o(12)
    ra = o_gpu(a)
    rb = o_gpu(b)
    gate(o_oracle(a), ra, "o history a")
    gate(o_oracle(b), rb, "o history b")
    assert np.array_equal(ra, o_gpu(a)), "o: the same input gave different bits after another call"


def test_ffn_results_do_not_depend_on_call_history():
    need_gpu()
    say("ffn: single-launch a, per-row b (M=2), single-launch a")
    a, b = synth.cfg_ffn_fp8(6), synth.cfg_ffn_fp8(7, M=2)
    ra = gpu_fp8(a)
    rb = gpu_fp8(b)
    gate(oracle_fp8(b), rb, "ffn history b", atol=FFN_ATOL)
    assert np.array_equal(ra, gpu_fp8(a)), "ffn: the same input gave different bits after another call"
    assert np.array_equal(ra, gpu_fp8(a, True, True))
    gate(oracle_fp8(a), ra, "ffn history a", atol=FFN_ATOL)


def test_qkv_results_do_not_depend_on_call_history():
    need_gpu()
    say("qkv: a, b, a")
    a, b = synth.cfg_qkv(13), synth.cfg_qkv(14)
    qa = qkv_gpu(a)
    qb = qkv_gpu(b)
    check_against_oracle(b, "qkv history b")
    qa2 = qkv_gpu(a)
    for x, y, name in zip(qa, qa2, ("q_out", "k_cache", "v_cache")):
        assert np.array_equal(x, y), f"qkv: {name} differs for the same input after another call"
    assert not np.array_equal(qa[0], qb[0])
