"""The full-attention-layer oracle (oracle/moa_oracle.c: orc_full_project_qkv,
orc_full_attention_pages, orc_full_attention_output) pinned on the CPU.

* QKV against torch modules in the form of gemma4.py:75-89, 116-122, 152-166 (RMSNorm in f32,
  RoPE on bf16 tensors, attention_k_eq_v: V is the unweighted norm of the raw K projection), the
  FP8 projection as generate_references.py:265-274 states it (torch's own E4M3 decode); only the
  written page slot changes.
* The paged softmax state against torch's scaled_dot_product_attention over the valid slots of all
  pages (the CPU reference's call, gemma4.py:180-184, scale 1.0); closed forms: one valid slot gives
  that slot's v with sum 1, none gives -inf / 0 / zeros.
* The output op against torch (x / sum in f32, rounded to bf16, then the FP8 projection, post-norm
  and residual); closed form: a one-hot attention row projects to one weight column.
"""
import numpy as np
import pytest
import torch

from gpu_util import bf16_ulp
from kat_inputs import unbf
from moa_amd import prng, synth
from oracle import oracle as O

H, GF, DF, QF, TF = 3840, 16, 512, 8192, 512


def bf(t):
    return torch.from_numpy(unbf(np.asarray(t).reshape(-1)).astype(np.float32)).to(torch.bfloat16)


def bits(t):
    return prng.f32_to_bf16_bits(t.float().numpy())


def rms(x, w=None):  # gemma4.py:83-89 on bf16 tensors
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
    if w is not None:
        y = y * w.float()
    return y.to(torch.bfloat16)


def proj(h, codes, scale):  # bf16((h . dec(W)^T) * s), generate_references.py:265-274
    w = torch.from_numpy(np.ascontiguousarray(codes)).view(torch.float8_e4m3fn).float()
    return ((h.float() @ w.T) * torch.from_numpy(scale.astype(np.float32))).to(torch.bfloat16)


def rope(x, cos_row, sin_row):  # gemma4.py:116-122 with the table's sin low half un-negated
    c = bf(cos_row)
    s_dev = bf(sin_row)
    s = torch.cat([-s_dev[: DF // 2], s_dev[DF // 2:]])
    rot = torch.cat([-x[..., DF // 2:], x[..., : DF // 2]], dim=-1)
    return x * c + rot * s


def close(a_bits, b_bits, ulps=1, frac=0.01):
    a, b = unbf(np.asarray(a_bits).reshape(-1)).astype(np.float64), unbf(np.asarray(b_bits).reshape(-1)).astype(np.float64)
    assert np.all(np.abs(a - b) <= ulps * bf16_ulp(np.maximum(np.abs(a), np.abs(b))) + 1e-30)
    assert np.count_nonzero(a != b) <= frac * a.size, np.count_nonzero(a != b)


def test_full_qkv_matches_torch_modules_and_writes_one_slot():
    d = synth.cfg_full_qkv(seed=1, M=2, pos=1000)   # page 1, slots 488 and 489
    kp, vp = d["k_cache"].copy(), d["v_cache"].copy()
    q_out = np.zeros((2, QF), np.uint16)
    O.full_project_qkv(d["x"], d["q_weight"], d["k_weight"], unbf(d["q_weight_scale"]), unbf(d["k_weight_scale"]),
                       d["input_rms_weight"], d["q_rms_weight"], d["k_rms_weight"], d["kv_offset"], d["rope_offset"],
                       d["cos"], d["sin"], kp, vp, q_out)
    for m in range(2):
        h = rms(bf(d["x"][m]), bf(d["input_rms_weight"]))
        q = rms(proj(h, d["q_weight"], unbf(d["q_weight_scale"])).view(GF, DF), bf(d["q_rms_weight"]))
        k_raw = proj(h, d["k_weight"], unbf(d["k_weight_scale"]))
        k = rms(k_raw, bf(d["k_rms_weight"]))
        v = rms(k_raw)
        p = d["pos"] + m
        close(q_out[m], bits(rope(q, d["cos"][p], d["sin"][p])))
        close(kp[488 + m], bits(rope(k, d["cos"][p], d["sin"][p])))
        close(vp[488 + m], bits(v))
        # V has unit RMS (the unweighted norm)
        assert abs(np.mean(unbf(vp[488 + m]).astype(np.float64) ** 2) - 1.0) < 1e-2
    keep = np.ones(TF, bool)
    keep[488:490] = False
    assert np.array_equal(kp[keep], d["k_cache"][keep]) and np.array_equal(vp[keep], d["v_cache"][keep])


def test_full_rope_tables_leave_three_quarters_unrotated():
    cos, sin = synth.rope_tables_full([3])
    c, s = unbf(cos[3]), unbf(sin[3])
    assert np.all(c[64:256] == 1.0) and np.all(c[320:] == 1.0) and np.all(s[64:256] == 0.0) and np.all(s[320:] == 0.0)
    assert np.array_equal(s[:64], -s[256:320]) and np.array_equal(c[:64], c[256:320])
    # with a table of cos 1 / sin 0, RoPE is the identity: K is the weighted norm itself
    d = synth.cfg_full_qkv(seed=2, M=1, pos=0)
    d["cos"][0] = prng.f32_to_bf16_bits(np.ones(DF, np.float32))
    d["sin"][0] = 0
    kp, vp, q_out = d["k_cache"].copy(), d["v_cache"].copy(), np.zeros((1, QF), np.uint16)
    O.full_project_qkv(d["x"], d["q_weight"], d["k_weight"], unbf(d["q_weight_scale"]), unbf(d["k_weight_scale"]),
                       d["input_rms_weight"], d["q_rms_weight"], d["k_rms_weight"], 0, 0, d["cos"], d["sin"], kp, vp,
                       q_out)
    h = rms(bf(d["x"][0]), bf(d["input_rms_weight"]))
    k = rms(proj(h, d["k_weight"], unbf(d["k_weight_scale"])), bf(d["k_rms_weight"]))
    close(kp[0], bits(k))


def _torch_paged(d):
    q = torch.from_numpy(unbf(d["q"].reshape(-1)).reshape(-1, GF, DF)).double()
    k = torch.from_numpy(unbf(d["k_pages"].reshape(-1)).reshape(-1, DF)).double()
    v = torch.from_numpy(unbf(d["v_pages"].reshape(-1)).reshape(-1, DF)).double()
    P, M = d["masks"].shape[:2]
    outs, mxs, sums = [], [], []
    for m in range(M):
        valid = torch.from_numpy(d["masks"][:, m].reshape(-1) != 0)
        o = torch.nn.functional.scaled_dot_product_attention(q[m][:, None, :], k[valid][None], v[valid][None], scale=1.0)
        s = q[m] @ k[valid].T
        outs.append(o[:, 0, :])
        mx = s.max(dim=1).values
        mxs.append(mx)
        sums.append(torch.exp(s - mx[:, None]).sum(dim=1))
    return torch.stack(outs).numpy(), torch.stack(mxs).numpy(), torch.stack(sums).numpy()


@pytest.mark.parametrize("P,q_std", [(1, 1.0), (3, 1.0), (2, 0.05)])
def test_paged_state_matches_torch_sdpa(P, q_std):
    d = synth.cfg_full_attention(seed=3, M=2, P=P, pos=[P * TF - 1, (P - 1) * TF + 100], q_std=q_std)
    mx, sm, out = O.full_attention_pages(d["q"], d["k_pages"], d["v_pages"], d["masks"])
    want, tmx, tsum = _torch_paged(d)
    assert np.allclose(mx, tmx, rtol=1e-6, atol=1e-5)
    assert np.allclose(sm, tsum, rtol=1e-6)
    norm = unbf(out.reshape(-1)).astype(np.float64).reshape(out.shape) / sm[:, :, None].astype(np.float64)
    # out is bf16 of the un-normalised sum: one bf16 rounding relative to the normalised value
    assert np.all(np.abs(norm - want) <= 2 * bf16_ulp(np.abs(want)) + 1e-7)


def test_paged_state_closed_forms():
    d = synth.cfg_full_attention(seed=4, M=2, P=2)
    d["masks"][:] = 0.0
    d["masks"][1, 0, 77] = 1.0             # row 0: only slot 77 of page 1
    mx, sm, out = O.full_attention_pages(d["q"], d["k_pages"], d["v_pages"], d["masks"])
    assert np.all(sm[0] == 1.0)
    assert np.array_equal(out[0], np.repeat(d["v_pages"][1, 77][None], GF, axis=0))
    s = unbf(d["q"][0].reshape(-1)).reshape(GF, DF).astype(np.float64) @ unbf(d["k_pages"][1, 77]).astype(np.float64)
    assert np.allclose(mx[0], s, rtol=1e-6)
    assert np.all(mx[1] == -np.inf) and np.all(sm[1] == 0.0) and not out[1].any()   # row 1: none


def test_full_output_matches_torch_and_one_hot():
    d = synth.cfg_full_o(seed=5, M=2)
    d["running_sum"][1, 3] = 0.0           # a head with no valid slot: a zero attention row
    r = d["residual"].copy()
    O.full_attention_output(d["x"], d["running_sum"], d["post_attn_rms_weight"], d["o_weight"],
                            unbf(d["o_weight_scale"]), r)
    for m in range(2):
        x = torch.from_numpy(unbf(d["x"][m].reshape(-1))).float().view(GF, DF)
        sums = torch.from_numpy(d["running_sum"][m])[:, None]
        xd = torch.where(sums > 0, x / torch.where(sums > 0, sums, torch.ones_like(sums)), torch.zeros_like(x))
        p = proj(xd.reshape(-1).to(torch.bfloat16), d["o_weight"], unbf(d["o_weight_scale"]))
        n = rms(p, bf(d["post_attn_rms_weight"]))
        want = (bf(d["residual"][m]) + n).to(torch.bfloat16)
        close(r[m], bits(want), ulps=1, frac=0.02)
    # one-hot: x = 3 at element k of head k / 512 with sum 2 -> x' = 1.5, p_n = bf16(1.5 w[n,k] s_n)
    k = 1234
    x = np.zeros((1, QF), np.uint16)
    x[0, k] = prng.f32_to_bf16_bits(np.array([3.0], np.float32))[0]
    rs = np.full((1, GF), 2.0, np.float32)
    r = np.zeros((1, H), np.uint16)
    w = np.ones(H, np.uint16) * np.uint16(0x3F80)
    O.full_attention_output(x, rs, w, d["o_weight"], unbf(d["o_weight_scale"]), r)
    col = torch.from_numpy(np.ascontiguousarray(d["o_weight"][:, k])).view(torch.float8_e4m3fn).float()
    p = (1.5 * col * torch.from_numpy(unbf(d["o_weight_scale"]))).to(torch.bfloat16)
    close(r[0], bits(rms(p, bf(w))), ulps=0, frac=0.0)
