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


@pytest.mark.parametrize("pos", [16, 3000])
def test_full_qkv_rows_match_oracle(pos):
    """full_project_qkv at 16 rows (17 heads of 512 from [Wq; Wk]; V the unweighted norm of K)."""
    need_gpu()
    from moa_amd import ops
    from test_gpu_full import TF, qkv_gpu as fq_gpu, qkv_oracle as fq_oracle
    say(f"full qkv rows M16 pos={pos}")
    d = synth.cfg_full_qkv(seed=13, M=16, pos=pos)
    gq, gk, gv = fq_gpu(d, 16)
    assert ops.device_errors() == 0
    wq, wk, wv = fq_oracle(d, 16)
    gate(wq, gq, f"full q_out rows pos{pos}")
    gate(wk, gk, f"full k page rows pos{pos}")
    gate(wv, gv, f"full v page rows pos{pos}")
    slot = pos % TF
    keep = np.ones(TF, bool)
    keep[slot:slot + 16] = False
    assert np.array_equal(gk[keep], d["k_cache"][keep]) and np.array_equal(gv[keep], d["v_cache"][keep])


@pytest.mark.parametrize("M", [2, 16])
def test_full_output_rows_match_oracle(M):
    """full_attention_output at 2 and 16 rows: x divided by the running sums (a head without a
    valid slot gives zeros), K = 8192."""
    need_gpu()
    from test_gpu_full import out_gpu as fo_gpu, out_oracle as fo_oracle
    say(f"full output rows M{M}")
    d = synth.cfg_full_o(seed=14, M=M)
    d["running_sum"][1, 7] = 0.0
    d["running_sum"][M - 1, 0] = 0.0
    a = fo_gpu(d)
    gate(fo_oracle(d), a, f"full output rows M{M}")
    assert np.array_equal(a, fo_gpu(d))
