"""sliding_project_qkv and sliding_attention_output at 3..16 token rows: the matrix-core rows path
(moa_rows.hip `rows_proj_kernel`, then the chunk path's row kernels), which reads the FP8 weights
once for all rows, vs the CPU oracle (the reference's per-row algorithm). F32 and BF16 scales, a
ring-cache wrap inside the call, and the 2-row calls that stay on the per-row kernels."""
import numpy as np
import pytest

from gpu_util import gate, need_gpu, say
from moa_amd import synth
from test_gpu_o import run_gpu as o_gpu, run_oracle as o_oracle
from test_gpu_qkv import check_against_oracle, run_gpu as qkv_gpu, run_oracle as qkv_oracle, slots

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M", [2, 3, 16])
def test_qkv_rows_match_oracle(M):
    need_gpu()
    say(f"qkv rows M{M}")
    d = synth.cfg_qkv(9, M=M, pos=1024 - M // 2)  # the ring wraps inside the call
    check_against_oracle(d, f"qkv rows M{M}", M=M)
    from moa_amd import ops
    assert ops.device_errors() == 0


def test_qkv_rows_bf16_scales():
    need_gpu()
    say("qkv rows M16 bf16 scales")
    d = synth.cfg_qkv(10, M=16, pos=3000)
    from moa_amd import prng
    for k in ("q_weight_scale", "k_weight_scale", "v_weight_scale"):  # the oracle sees the bf16 scales too
        d[k] = prng.f32_to_bf16_bits(d[k])
    q, kc, vc = qkv_gpu(d, 16, bf16_scales=True)
    qe, kce, vce = qkv_oracle(d, 16)
    gate(qe, q, "qkv rows M16 bf16 q")
    ss = slots(d, 16)
    gate(kce[ss], kc[ss], "qkv rows M16 bf16 k")
    gate(vce[ss], vc[ss], "qkv rows M16 bf16 v")


@pytest.mark.parametrize("M", [2, 3, 16])
@pytest.mark.parametrize("bf16_scales", [False, True])
def test_o_rows_match_oracle(M, bf16_scales):
    need_gpu()
    say(f"o rows M{M} bf16_scales={bf16_scales}")
    d = synth.cfg_o(11, M=M)
    if bf16_scales:  # the oracle then sees the bf16-rounded scales
        from moa_amd import prng
        d["o_weight_scale"] = prng.f32_to_bf16_bits(d["o_weight_scale"])
    a = o_gpu(d, bf16_scales=bf16_scales)
    gate(o_oracle(d), a, f"o rows M{M}")
    assert np.array_equal(a, o_gpu(d, bf16_scales=bf16_scales))


def test_o_rows_are_independent():
    """The first rows of a 16-row call equal a call of just those rows, bit for bit."""
    need_gpu()
    d16 = synth.cfg_o(12, M=16)
    d4 = dict(d16, x=d16["x"][:4].copy(), residual=d16["residual"][:4].copy())
    assert np.array_equal(o_gpu(d16)[:4], o_gpu(d4))
