"""The sliding_attention oracle (oracle/moa_oracle.c: orc_sliding_attention) pinned on the CPU.

* Against torch's scaled_dot_product_attention, the call the reference's CPU path makes
  (FO/scripts/reference/gemma4.py:163-186, scale=1.0), with the key/value heads repeated over
  the query heads (repeat_interleave) and the boolean window mask. Torch computes in f32, the
  oracle in f64. Their bf16 outputs may differ by one bf16 ulp where the f32 result lies next
  to a rounding boundary, and by torch's f32 accumulation error (~1e-7) on outputs near zero.
* Closed forms: a single valid slot returns that slot's v; no valid slot returns zeros; q = 0
  averages the valid slots' v.
"""
import numpy as np
import pytest
import torch

from gpu_util import bf16_ulp
from kat_inputs import unbf
from moa_amd import prng, synth
from oracle import oracle as O

NS, GS, DS, TS = 8, 2, 256, 1024


def _torch_sdpa(d):
    q = torch.from_numpy(unbf(d["q"]).reshape(-1, NS * GS, DS)).float()          # [M, 16, 256]
    k = torch.from_numpy(unbf(d["k_cache"]).reshape(TS, NS, DS)).float()
    v = torch.from_numpy(unbf(d["v_cache"]).reshape(TS, NS, DS)).float()
    M = q.shape[0]
    k = k.permute(1, 0, 2).repeat_interleave(GS, dim=0)                              # [16, T, 256]
    v = v.permute(1, 0, 2).repeat_interleave(GS, dim=0)
    mask = torch.from_numpy(d["mask"] != 0)                                          # [M, T]
    outs = []
    for m in range(M):
        o = torch.nn.functional.scaled_dot_product_attention(
            q[m][:, None, :], k, v, attn_mask=mask[m][None, None, :], scale=1.0)  # [16, 1, 256]
        outs.append(o[:, 0, :].numpy())
    return prng.f32_to_bf16_bits(np.stack(outs).astype(np.float32)).reshape(M, NS, GS, DS)


@pytest.mark.parametrize("q_std,pos", [(1.0, 1023), (0.1, 1023), (0.1, 300), (1.0, 7)])
def test_oracle_matches_torch_sdpa(q_std, pos):
    d = synth.cfg_attention(seed=3, M=2, pos=[pos, max(0, pos // 2)], q_std=q_std)
    got = O.sliding_attention(d["q"], d["k_cache"], d["v_cache"], d["mask"])
    want = _torch_sdpa(d)
    a, b = unbf(got.reshape(-1)).astype(np.float64), unbf(want.reshape(-1)).astype(np.float64)
    # same bits, or within one bf16 ulp plus torch's f32 accumulation error (sums of ~1000
    # unit-size terms: a few 1e-7 absolute, visible only on outputs near zero); rarely
    bound = bf16_ulp(np.maximum(np.abs(a), np.abs(b))) + 1e-6
    assert np.all(np.abs(a - b) <= bound)
    assert np.count_nonzero(got != want) <= got.size // 100


def test_single_valid_slot_returns_its_value():
    d = synth.cfg_attention(seed=4, M=1, q_std=1.0)
    d["mask"] = np.zeros((1, TS), np.float32)
    d["mask"][0, 517] = 1.0
    got = O.sliding_attention(d["q"], d["k_cache"], d["v_cache"], d["mask"])
    v = d["v_cache"].reshape(TS, NS, DS)[517]                                        # [8, 256]
    assert np.array_equal(got[0], np.repeat(v[:, None, :], GS, axis=1))


def test_no_valid_slot_gives_zeros():
    d = synth.cfg_attention(seed=5, M=1)
    d["mask"] = np.zeros((1, TS), np.float32)
    got = O.sliding_attention(d["q"], d["k_cache"], d["v_cache"], d["mask"])
    assert not got.any()


def test_zero_query_averages_the_valid_values():
    d = synth.cfg_attention(seed=6, M=1, pos=99)
    d["q"] = np.zeros_like(d["q"])
    got = unbf(O.sliding_attention(d["q"], d["k_cache"], d["v_cache"], d["mask"]).reshape(-1)).reshape(NS, GS, DS)
    v = unbf(d["v_cache"].reshape(-1)).reshape(TS, NS, DS).astype(np.float64)[:100].mean(axis=0)
    want = unbf(prng.f32_to_bf16_bits(v.astype(np.float32)).reshape(-1)).reshape(NS, DS)
    for g in range(GS):
        assert np.array_equal(got[:, g], want)
