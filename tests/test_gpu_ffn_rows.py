"""decoder_feedforward at 2..16 token rows: the matrix-core path (moa_rows.hip) that reads each
weight once for all rows, in all three weight formats, vs the CPU oracle (which runs the
reference's per-row algorithm, generate_references.py:375-414). Calls of more rows take the MFMA
path in every format. Each output row depends
on its own input row only: the first rows of a call give the same bits as a call of just those
rows."""
import numpy as np
import pytest

from gpu_util import gate, need_gpu, say
from moa_amd import synth
from oracle import oracle as O
from test_gpu_ffn import (FFN_ATOL, assert_geglu_near_zero, cancel_fp4_codes, cancellation_residual, gpu_fp8, gpu_mxfp4,
                          gpu_nvfp4, oracle_fp8, oracle_mxfp4, oracle_nvfp4)

pytestmark = pytest.mark.gpu
H = 3840
FORMATS = {"fp8": (oracle_fp8, gpu_fp8), "nvfp4": (oracle_nvfp4, gpu_nvfp4), "mxfp4": (oracle_mxfp4, gpu_mxfp4)}
_weights = {}


def case(fmt: str, M: int, tag: str = "rows") -> dict:
    """The format's weights (generated once) with M residual rows ~ N(0, 1)."""
    if fmt not in _weights:
        if fmt == "fp8":
            _weights[fmt] = synth.cfg_ffn_fp8(7)
        elif fmt == "mxfp4":
            _weights[fmt] = synth.cfg_ffn_mxfp4(7)
        else:
            _weights[fmt] = synth.ref_ffn_inputs(1)  # the reference harness's NVFP4 weights and scales
    d = dict(_weights[fmt])
    d["residual"] = synth.bf16_normal(f"{tag}.{fmt}.residual", (M, H))
    return d


@pytest.mark.parametrize("M", [2, 5, 16])
@pytest.mark.parametrize("fmt", ["fp8", "nvfp4", "mxfp4"])
def test_rows_match_oracle(fmt, M):
    need_gpu()
    say(f"ffn rows {fmt} M{M}")
    want, got = FORMATS[fmt]
    d = case(fmt, M)
    gate(want(d), got(d), f"ffn rows {fmt} M{M}", atol=FFN_ATOL)
    from moa_amd import ops
    assert ops.device_errors() == 0


@pytest.mark.parametrize("fmt", ["fp8", "nvfp4", "mxfp4"])
def test_rows_are_independent_and_repeatable(fmt):
    need_gpu()
    say(f"ffn rows {fmt}: M16 vs M3 prefix, repeat")
    _, got = FORMATS[fmt]
    d16 = case(fmt, 16, "indep")
    d3 = dict(d16, residual=d16["residual"][:3].copy())
    a = got(d16)
    assert np.array_equal(a[:3], got(d3))
    assert np.array_equal(a, got(d16))


def _rows_one_launch(on: bool) -> None:
    import ctypes as C
    from moa_amd import _lib
    _lib.call("moa_test_set_rows_one_launch", C.c_int(1 if on else 0))


@pytest.mark.parametrize("M", [2, 9, 16])
@pytest.mark.parametrize("fmt", ["fp8", "nvfp4", "mxfp4"])
def test_one_launch_equals_two_launches(fmt, M):
    """The up/gate and down contractions in one launch (rows_fused_kernel, the default where its
    grid fits) give the bits of the two launches. Four calls in a row, each on other rows: a GeGLU
    block read before its producer had written it, or a stale copy of an earlier call's, would
    show as a difference."""
    need_gpu()
    say(f"ffn rows {fmt} M{M}: one launch vs two")
    from moa_amd import ops
    _, got = FORMATS[fmt]
    ds = [case(fmt, M, f"launches{i}") for i in range(4)]
    one = [got(d) for d in ds]
    _rows_one_launch(False)
    try:
        two = [got(d) for d in ds]
    finally:
        _rows_one_launch(True)
    for i, (a, b) in enumerate(zip(one, two)):
        assert np.array_equal(a, b), f"call {i}: {int(np.sum(a != b))} outputs differ"
    assert ops.device_errors() == 0


@pytest.mark.parametrize("fmt", ["nvfp4", "mxfp4"])
def test_fp4_calls_of_17_rows(fmt):
    """17 rows: the first call length past the rows path (the MFMA path, a partial row tile)."""
    need_gpu()
    say(f"ffn rows {fmt} M17")
    want, got = FORMATS[fmt]
    d = case(fmt, 17, "tiles")
    gate(want(d), got(d), f"ffn rows {fmt} M17", atol=FFN_ATOL)


def test_rows_without_post_norm_and_layer_scalar():
    need_gpu()
    say("ffn rows fp8 M3 without post-norm and layer scalar")
    d = case("fp8", 3, "plain")
    gate(oracle_fp8(d, False, False), gpu_fp8(d, False, False), "ffn rows fp8 M3 plain", atol=FFN_ATOL)


@pytest.mark.parametrize("M", [4, 16])
@pytest.mark.parametrize("fmt", ["fp8", "mxfp4", "nvfp4"])
def test_rows_cancellation_probe(fmt, M):
    """Rows whose pre-normed activations cancel in every up/gate row (the config-3 probe), mixed
    with ordinary rows; the probe rows' GeGLU values are asserted near zero on the oracle."""
    need_gpu()
    say(f"ffn rows {fmt} cancellation probe M{M}")
    want, got = FORMATS[fmt]
    d = case(fmt, M, "cancel")
    d["residual"] = d["residual"].copy()
    d["residual"][1] = cancellation_residual(-23)
    d["residual"][3] = cancellation_residual(-12)
    d["pre_ff_rms_weight"] = np.full(H, 0x3F80, np.uint16)
    for k in ("up", "gate"):
        if fmt == "fp8":
            w = d[f"{k}_weight"].copy()
            w[:, 0::480] = 0x38  # 1.0
            w[:, 1::480] = 0x38
            d[f"{k}_weight"] = w
        else:
            d[f"{k}_weight_packed"] = cancel_fp4_codes(d[f"{k}_weight_packed"])
    probes = dict(d, residual=np.ascontiguousarray(d["residual"][[1, 3]]))
    assert_geglu_near_zero(probes, {"fp8": O.FFN_FP8, "mxfp4": O.FFN_MXFP4, "nvfp4": O.FFN_NVFP4}[fmt],
                           f"ffn rows {fmt} cancel M{M}")
    gate(want(d), got(d), f"ffn rows {fmt} cancel M{M}", atol=FFN_ATOL)
