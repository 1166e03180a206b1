"""The final_norm_and_logits oracle (oracle/moa_oracle.c: orc_softcap30, orc_final_norm_and_logits)
pinned on the CPU.

* The softcap over all 65536 bf16 inputs against torch's f32 tanh (the device chain of
  FO/src/ops.rs:256-293: widen, divide by 30, tanh, multiply by 30, one rounding): at most one
  bf16 ulp apart, rarely; and the closed forms: odd, monotone, +-30 at the ends, the identity for
  small logits (tanh(u) * 30 = l (1 - l^2 / 2700 + ...)).
* The whole operator on a run of vocabulary rows against torch's CPU modules as gemma4.py:75-89,
  258-261 use them (RMSNorm in f32, nn.Linear in bf16), with the softcap of the device chain.
* Known answers: a one-hot lm_head row returns the softcap of that element of the normed input;
  a zero input row gives zero logits.
"""
import numpy as np
import torch

from gpu_util import bf16_ulp
from kat_inputs import unbf
from moa_amd import prng, synth
from oracle import oracle as O

H = 3840
ALL = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)


def _softcap_all():
    return np.array([O.softcap30(int(b)) for b in ALL], np.uint16)


def _torch_softcap_bits(bits):
    t = torch.from_numpy(unbf(bits).astype(np.float32))
    return prng.f32_to_bf16_bits((torch.tanh(t / 30.0) * 30.0).numpy())


def test_softcap_all_bf16_against_torch_f32_tanh():
    got = _softcap_all()
    want = _torch_softcap_bits(ALL)
    a, b = unbf(got).astype(np.float64), unbf(want).astype(np.float64)
    nan = np.isnan(unbf(ALL))
    assert np.array_equal(np.isnan(a), nan) and np.array_equal(np.isnan(b), nan)
    a, b = a[~nan], b[~nan]
    assert np.all(np.abs(a - b) <= bf16_ulp(np.maximum(np.abs(a), np.abs(b))))
    assert np.count_nonzero(a != b) <= 8


def test_softcap_closed_forms():
    got = unbf(_softcap_all()).astype(np.float64)
    with np.errstate(invalid="ignore"):
        x = unbf(ALL).astype(np.float64)
    fin = np.isfinite(x)
    # odd
    neg = ALL ^ np.uint16(0x8000)
    assert np.array_equal(got[fin], -got[neg.astype(np.int64)][fin])
    # monotone over the positive finite values (bits ascending = values ascending)
    pos = np.arange(0x0000, 0x7f80)
    assert np.all(np.diff(got[pos]) >= 0)
    # the ends: +-30 for large and infinite logits
    assert got[0x7f80] == 30.0 and got[0xff80] == -30.0
    assert np.all(got[(x > 200.0) & fin] == 30.0)
    # small logits pass unchanged (relative change below l^2 / 2700 << half a bf16 ulp)
    small = fin & (np.abs(x) < 0.5)
    assert np.array_equal(got[small], x[small])
    # and the bound: |softcap(l)| <= min(|l|, 30)
    assert np.all(np.abs(got[fin]) <= np.minimum(np.abs(x[fin]), 30.0))


def _torch_logits(d, w_rows):
    x = torch.from_numpy(unbf(d["input"].reshape(-1)).reshape(-1, H)).to(torch.bfloat16)
    rw = torch.from_numpy(unbf(d["rms_weight"]))
    # gemma4.py:83-89 (eps 1e-6)
    xf = x.float()
    h = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6) * rw.float()).to(torch.bfloat16)
    w = torch.from_numpy(unbf(w_rows.reshape(-1)).reshape(-1, H)).to(torch.bfloat16)
    logits = torch.nn.functional.linear(h, w)                         # bf16 output, f32 accumulation
    return prng.f32_to_bf16_bits((torch.tanh(logits.float() / 30.0) * 30.0).numpy())


def test_oracle_matches_torch_modules():
    d = synth.cfg_logits(seed=1, M=2)
    w = synth.lm_head_rows(1, 1536)
    got = O.final_norm_and_logits(d["input"], d["rms_weight"], w)
    want = _torch_logits(d, w)
    a, b = unbf(got.reshape(-1)).astype(np.float64), unbf(want.reshape(-1)).astype(np.float64)
    # the logit itself is a bf16 rounding of an f32 sum (~3840 terms): one bf16 ulp of the logit
    # where the two sums straddle a rounding midpoint, passed through the softcap (slope <= 1)
    assert np.all(np.abs(a - b) <= 2 * bf16_ulp(np.maximum(np.abs(a), np.abs(b))))
    assert np.count_nonzero(a != b) <= got.size // 50
    assert np.abs(b).max() > 20.0 and np.std(b) > 5.0  # the softcap's curve is exercised


def test_one_hot_rows_return_softcapped_normed_elements():
    d = synth.cfg_logits(seed=2, M=1)
    rows = np.array([0, 1, 7, 1000, 3839], np.int64)
    w = np.zeros((rows.size, H), np.uint16)
    w[np.arange(rows.size), rows] = 0x3F80  # 1.0
    got = O.final_norm_and_logits(d["input"], d["rms_weight"], w)[0]
    h = O.rmsnorm(d["input"].reshape(H), d["rms_weight"])
    want = np.array([O.softcap30(int(h[r])) for r in rows], np.uint16)
    assert np.array_equal(got, want)


def test_zero_input_gives_zero_logits():
    d = synth.cfg_logits(seed=3, M=1)
    d["input"] = np.zeros_like(d["input"])
    got = O.final_norm_and_logits(d["input"], d["rms_weight"], synth.lm_head_rows(3, 64))
    assert not (got & np.uint16(0x7fff)).any()
