"""The single-launch kernels (one token row) and the MFMA path of longer calls.

Calls of more than 16 rows take the MFMA path (FP8 weights): 17 rows (a partial row tile),
64 (one full tile), 100 and 256 (BASELINE config 4's chunk length). Repeated calls interleaving
different inputs check that no launch ever reads a tagged hand-off word left by an earlier launch
(the tags are per-launch epochs): results must not depend on call history."""
import numpy as np
import pytest

from gpu_util import gate, gate_addend, need_gpu, say
from moa_amd import synth
from test_gpu_ffn import FFN_ATOL, gpu_fp8, oracle_fp8
from test_gpu_o import run_gpu as o_gpu
from test_gpu_o import run_oracle as o_oracle
from test_gpu_qkv import check_against_oracle
from test_gpu_qkv import run_gpu as qkv_gpu

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M", [17, 64, 100, 256])
def test_ffn_fp8_mfma_rows(M):
    need_gpu()
    say(f"ffn fp8 M{M} (MFMA path)")
    d = synth.cfg_ffn_fp8(5, M=M)
    gate(oracle_fp8(d), gpu_fp8(d), f"ffn fp8 M{M}", atol=FFN_ATOL)


def test_ffn_fp8_mfma_rows_without_post_norm_and_scalar():
    need_gpu()
    say("ffn fp8 M33 literal (MFMA path)")
    d = synth.cfg_ffn_fp8(8, M=33)
    gate_addend(oracle_fp8(d, False, False), gpu_fp8(d, False, False), d["residual"], "ffn fp8 M33 literal",
                atol=FFN_ATOL)


@pytest.mark.parametrize("M", [17, 64, 100, 256])
def test_o_mfma_rows(M):
    need_gpu()
    say(f"o M{M} (MFMA path)")
    d = synth.cfg_o(5, M=M)
    gate(o_oracle(d), o_gpu(d), f"o M{M}")


@pytest.mark.parametrize("M", [17, 100, 256])
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
