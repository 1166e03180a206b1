"""ops::final_norm_and_logits on the GPU (moa_final_norm_and_logits) against the CPU oracle.

The lm_head is the full [262144, 3840] bf16 matrix (2 GB), drawn on the device (synth.lm_head_device:
|w| in [1/32, 1/2), logits of std ~14 that span the softcap's curve). The oracle computes a sample
of vocabulary rows (the first and last 2048 and 4096 scattered ones), whose weights are copied back;
every row is also checked against torch's f32 product on the device. Gate: the reference's atol /
rtol 1e-2."""
import numpy as np
import pytest

from gpu_util import bf16_ulp, dev, dev_zeros, gate, host, need_gpu, say, torch
from kat_inputs import unbf
from moa_amd import synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu
H, W = 3840, 262144

_lm = {}


def lm_head(seed=0):
    if seed not in _lm:
        _lm.clear()
        _lm[seed] = synth.lm_head_device(seed)
    return _lm[seed]


def sample_rows(seed=0):
    rng = np.random.default_rng(seed)
    mid = rng.choice(np.arange(2048, W - 2048), 4096, replace=False)
    return np.sort(np.concatenate([np.arange(2048), mid, np.arange(W - 2048, W)]))


def run_gpu(d, w):
    from moa_amd import ops
    M = d["input"].shape[0]
    out = dev_zeros(M * W)
    ops.final_norm_and_logits(dev(d["input"]), dev(d["rms_weight"]), w, out)
    assert ops.device_errors() == 0
    return host(out).reshape(M, W)


def check_sampled(d, w, got, label, seed=0):
    rows = sample_rows(seed)
    w_rows = host(w[torch.from_numpy(rows).cuda()]).reshape(rows.size, H)
    want = O.final_norm_and_logits(d["input"], d["rms_weight"], w_rows)
    gate(want, got[:, rows], label)


def test_softcap_all_bf16_inputs():
    """The device softcap (words 66564.. of the format self-test) on every bf16 value."""
    need_gpu()
    say("softcap: all 65536 bf16 inputs")
    from moa_amd import ops
    got = host(ops.format_selftest())[66564:66564 + 65536].astype(np.uint16)
    want = np.array([O.softcap30(b) for b in range(1 << 16)], np.uint16)
    with np.errstate(invalid="ignore"):
        a, b = unbf(got).astype(np.float64), unbf(want).astype(np.float64)
    assert np.array_equal(np.isnan(a), np.isnan(b))
    fin = ~np.isnan(b)
    a, b = a[fin], b[fin]
    n_diff = int(np.count_nonzero(a != b))
    say(f"softcap: {n_diff} of {b.size} differ from the f64 rounding")
    assert np.all(np.abs(a - b) <= bf16_ulp(np.maximum(np.abs(a), np.abs(b))))
    assert n_diff <= 64


def test_one_row_full_vocabulary():
    need_gpu()
    say("logits M=1: sampled rows vs oracle, every row vs torch f32")
    d = synth.cfg_logits(seed=1, M=1)
    w = lm_head(0)
    got = run_gpu(d, w)
    check_sampled(d, w, got, "logits M1 sampled")
    # every row: torch's f32 product of the oracle's normed row, the bf16 logit, softcap in f32
    h = torch.from_numpy(unbf(O.rmsnorm(d["input"].reshape(H), d["rms_weight"]))).cuda()
    wf = w.view(torch.bfloat16)
    logit = torch.mv(wf.float(), h.float()).to(torch.bfloat16).float()
    want = (torch.tanh(logit / 30.0) * 30.0).to(torch.bfloat16).view(torch.int16)
    gate(host(want).reshape(1, W), got, "logits M1 all rows vs torch f32")
    assert np.abs(unbf(got.reshape(-1))).max() <= 30.0


@pytest.mark.parametrize("M", [3, 17])
def test_several_rows(M):
    need_gpu()
    say(f"logits M={M}: sampled rows vs oracle")
    d = synth.cfg_logits(seed=2, M=M)
    w = lm_head(0)
    got = run_gpu(d, w)
    check_sampled(d, w, got, f"logits M{M} sampled", seed=M)
    # each row alone through the one-row kernel gives the same bits
    for m in (0, M - 1):
        one = dict(input=d["input"][m:m + 1], rms_weight=d["rms_weight"])
        assert np.array_equal(run_gpu(one, w)[0], got[m]), f"row {m} differs from its one-row call"


def test_one_hot_lm_head_returns_softcapped_normed_elements():
    need_gpu()
    say("logits: one-hot lm_head rows (row r has 1.0 at r mod 3840)")
    d = synth.cfg_logits(seed=4, M=1)
    d["input"][0, 0] = 0x4120  # a 10.0 so one normed element leaves the identity range
    w = torch.zeros((W, H), dtype=torch.int16, device="cuda")
    r = torch.arange(W, device="cuda")
    w[r, r % H] = 0x3F80
    got = run_gpu(d, w)[0]
    from moa_amd import ops
    h = O.rmsnorm(d["input"].reshape(H), d["rms_weight"])
    # the device's own softcap table (checked on every input by the test above)
    cap = host(ops.format_selftest())[66564 + h.astype(np.int64)].astype(np.uint16)
    assert np.array_equal(got, cap[np.arange(W) % H])


def test_zero_input_row_gives_zero_logits():
    need_gpu()
    say("logits: zero input row")
    d = synth.cfg_logits(seed=5, M=2)
    d["input"][1] = 0
    got = run_gpu(d, lm_head(0))
    assert not (got[1] & np.uint16(0x7fff)).any()
    assert (got[0] & np.uint16(0x7fff)).any()
