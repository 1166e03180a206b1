"""ops::sliding_attention on the GPU (moa_sliding_attention) against the CPU oracle.

Inputs: q ~ N(0, q_std) (q_std = 1 is the real case after the head norm: scores of std 16, so
the softmax is peaky; 0.1 spreads it over many slots), ring caches ~ N(0, 1), the runtime's mask
rows for a position (FO/src/host/runtime.rs:160, 409). Gate: the reference's atol / rtol 1e-2."""
import numpy as np
import pytest

from gpu_util import dev, dev_zeros, gate, host, need_gpu, say, torch
from moa_amd import synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu
NS, GS, DS, TS = 8, 2, 256, 1024


def run_gpu(d):
    from moa_amd import ops
    M = d["q"].shape[0]
    out = dev_zeros(M * NS * GS * DS)
    ops.sliding_attention(dev(d["q"]), dev(d["k_cache"]), dev(d["v_cache"]), dev(d["mask"]), out)
    assert ops.device_errors() == 0
    return host(out).reshape(M, NS, GS, DS)


def run_oracle(d):
    return O.sliding_attention(d["q"], d["k_cache"], d["v_cache"], d["mask"])


@pytest.mark.parametrize("q_std,pos", [(1.0, 5000), (1.0, 1023), (1.0, 0), (1.0, 1), (0.1, 511), (0.1, 5000), (0.3, 31),
                                       (8.0, 5000)])
def test_matches_oracle(q_std, pos):
    need_gpu()
    say(f"attention q_std={q_std} pos={pos}")
    d = synth.cfg_attention(seed=1, M=1, pos=pos, q_std=q_std)
    gate(run_oracle(d), run_gpu(d), f"attention q{q_std} pos{pos}")


def test_rows_with_different_masks_in_one_call():
    need_gpu()
    say("attention M=3, positions 2, 700, 4000")
    d = synth.cfg_attention(seed=2, M=3, pos=[2, 700, 4000], q_std=0.5)
    gate(run_oracle(d), run_gpu(d), "attention M3")


def test_call_of_twenty_rows():
    """20 rows run as one full 16-row launch and one of 4 (each launch's counters per (row, head)),
    with mask rows from a single valid slot (position 0) to the full window (positions >= 1023)."""
    need_gpu()
    pos = [0, 1, 31, 32, 500, 1022, 1023, 1024, 1500, 2047, 2048, 3000, 4095, 4096, 5000, 6000, 7000, 7500, 8000, 8191]
    say("attention M=20 (launches of 16 and 4 rows)")
    d = synth.cfg_attention(seed=9, M=20, pos=pos, q_std=0.5)
    gate(run_oracle(d), run_gpu(d), "attention M20")


def test_scattered_mask():
    need_gpu()
    say("attention: random 0/1 mask")
    d = synth.cfg_attention(seed=7, M=2, q_std=0.3)
    rng = np.random.default_rng(7)
    d["mask"] = (rng.random((2, TS)) < 0.3).astype(np.float32)
    gate(run_oracle(d), run_gpu(d), "attention scattered mask")


def test_single_valid_slot_is_exact_and_no_valid_slot_gives_zeros():
    need_gpu()
    say("attention: one valid slot (row 0), none (row 1)")
    d = synth.cfg_attention(seed=8, M=2, q_std=1.0)
    d["mask"] = np.zeros((2, TS), np.float32)
    d["mask"][0, 900] = 1.0
    got = run_gpu(d)
    v = d["v_cache"].reshape(TS, NS, DS)[900]
    assert np.array_equal(got[0], np.repeat(v[:, None, :], GS, axis=1))
    assert not got[1].any()


def test_repeat_calls_give_the_same_bits():
    need_gpu()
    say("attention: a, b, a")
    a, b = synth.cfg_attention(seed=9, pos=800), synth.cfg_attention(seed=10, pos=3000)
    ra = run_gpu(a)
    rb = run_gpu(b)
    gate(run_oracle(b), rb, "attention history b")
    assert np.array_equal(ra, run_gpu(a))
