"""The full-attention-layer operators on the GPU against the CPU oracle:
moa_full_project_qkv, moa_full_attention_first_page / moa_full_attention_page (the running
softmax state over 512-slot pages) and moa_full_attention_output, alone and chained.

The state is compared as the reference defines it: running_max (scores on the matrix cores in f32
from bf16 operands: within 1e-3 absolute), running_sum and the un-normalised out within the gate's
rtol / atol (the exp weights enter the MFMA as bf16 and the state's out is bf16 between pages), and
out / sum -- what the layer uses -- within the gate."""
import numpy as np
import pytest

from gpu_util import bf16_ulp, dev, dev_zeros, gate, gate_addend, host, need_gpu, say, torch
from kat_inputs import unbf
from moa_amd import synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu
H, GF, DF, QF, TF = 3840, 16, 512, 8192, 512


def i32(v):
    return torch.tensor([int(v)], dtype=torch.int32, device="cuda")


def qkv_gpu(d, M):
    from moa_amd import ops
    kc, vc, q_out = dev(d["k_cache"]), dev(d["v_cache"]), dev_zeros(M * QF)
    ops.full_project_qkv(dev(d["x"]), dev(d["q_weight"]), dev(d["k_weight"]), dev(d["q_weight_scale"]),
                         dev(d["k_weight_scale"]), dev(d["input_rms_weight"]), dev(d["q_rms_weight"]),
                         dev(d["k_rms_weight"]), i32(d["kv_offset"]), i32(d["rope_offset"]), dev(d["cos"]),
                         dev(d["sin"]), kc, vc, q_out)
    return host(q_out).reshape(M, QF), host(kc).reshape(TF, DF), host(vc).reshape(TF, DF)


def qkv_oracle(d, M):
    kp, vp, q_out = d["k_cache"].copy(), d["v_cache"].copy(), np.zeros((M, QF), np.uint16)
    O.full_project_qkv(d["x"], d["q_weight"], d["k_weight"], unbf(d["q_weight_scale"]), unbf(d["k_weight_scale"]),
                       d["input_rms_weight"], d["q_rms_weight"], d["k_rms_weight"], d["kv_offset"], d["rope_offset"],
                       d["cos"], d["sin"], kp, vp, q_out)
    return q_out, kp, vp


@pytest.mark.parametrize("pos,M", [(0, 1), (511, 1), (700, 1), (32767, 1), (1000, 3)])
def test_full_qkv_matches_oracle(pos, M):
    need_gpu()
    from moa_amd import ops
    say(f"full qkv pos={pos} M={M}")
    d = synth.cfg_full_qkv(seed=1, M=M, pos=pos)
    gq, gk, gv = qkv_gpu(d, M)
    assert ops.device_errors() == 0
    wq, wk, wv = qkv_oracle(d, M)
    gate(wq, gq, f"full q_out pos{pos}")
    gate(wk, gk, f"full k page pos{pos}")
    gate(wv, gv, f"full v page pos{pos}")
    slot = pos % TF
    keep = np.ones(TF, bool)
    keep[slot:slot + M] = False
    assert np.array_equal(gk[keep], d["k_cache"][keep]) and np.array_equal(gv[keep], d["v_cache"][keep])


def test_full_qkv_row_past_the_page_writes_nothing():
    need_gpu()
    from moa_amd import _lib, ops
    say("full qkv: rows 510..512 of one page (the third falls past it)")
    d = synth.cfg_full_qkv(seed=2, M=3, pos=510)
    gq, gk, gv = qkv_gpu(d, 3)
    assert ops.device_errors() == _lib.DEVERR_KV_OFFSET
    wq, wk, wv = qkv_oracle(dict(d, x=d["x"][:2]), 2)
    gate(wq, gq[:2], "full q_out rows 0-1")
    assert not gq[2].any()
    gate(wk[510:], gk[510:], "full k slots 510-511")
    assert np.array_equal(gk[:510], d["k_cache"][:510]) and np.array_equal(gv[:510], d["v_cache"][:510])


def pages_gpu(d, first_only=False):
    from moa_amd import ops
    P, M = d["masks"].shape[:2]
    q = dev(d["q"])
    mx = torch.zeros(M * GF, dtype=torch.float32, device="cuda")
    sm = torch.zeros(M * GF, dtype=torch.float32, device="cuda")
    out = dev_zeros(M * QF)
    for pg in range(P):
        fn = ops.full_attention_first_page if pg == 0 else ops.full_attention_page
        fn(q, dev(d["k_pages"][pg]), dev(d["v_pages"][pg]), dev(d["masks"][pg]), mx, sm, out)
    return host(mx).reshape(M, GF), host(sm).reshape(M, GF), host(out).reshape(M, GF, DF)


def state_rounding(d):
    """What the bf16 out state between pages can contribute, element by element: each page's
    state is rounded to bf16 once (half a bf16 ulp of its value), then rescaled by
    exp(max then - final max) with every later page. The interface fixes this rounding
    (out_hbm is bf16, FO/src/ops.rs:148-174); the oracle computes the pages at once."""
    P = d["masks"].shape[0]
    wm, _, _ = O.full_attention_pages(d["q"], d["k_pages"], d["v_pages"], d["masks"])
    allow = np.zeros(d["q"].shape, np.float64).reshape(wm.shape + (DF,))
    for k in range(1, P):
        mk, _, ok = O.full_attention_pages(d["q"], d["k_pages"][:k], d["v_pages"][:k], d["masks"][:k])
        with np.errstate(invalid="ignore", over="ignore"):
            f = np.where(np.isfinite(mk), np.exp(mk.astype(np.float64) - wm), 0.0)
        allow += 0.5 * bf16_ulp(unbf(ok.reshape(-1)).reshape(ok.shape)) * f[..., None]
    return allow


def check_state(d, label):
    gm, gs, go = pages_gpu(d)
    wm, ws, wo = O.full_attention_pages(d["q"], d["k_pages"], d["v_pages"], d["masks"])
    fin = np.isfinite(wm)
    assert np.array_equal(np.isfinite(gm), fin), f"{label}: heads with no valid slot differ"
    assert np.all(np.abs(gm[fin] - wm[fin]) <= 1e-3 * (1.0 + np.abs(wm[fin]))), f"{label}: running_max"
    assert np.all(np.abs(gs - ws) <= 1e-2 * np.abs(ws) + 1e-6), f"{label}: running_sum"
    allow = state_rounding(d)
    e = unbf(wo.reshape(-1)).reshape(wo.shape).astype(np.float64)
    a = unbf(go.reshape(-1)).reshape(go.shape).astype(np.float64)
    diff = np.abs(a - e)
    plain = 1e-2 + 1e-2 * np.abs(e)
    n_fail = int(np.count_nonzero(diff > plain + allow))
    say(f"[{label + ' out (un-normalised)':40}] max|d|={diff.max():.5f} exact={int(np.count_nonzero(diff == 0))}/"
        f"{diff.size} past-gate={int(np.count_nonzero(diff > plain))} fail={n_fail}")
    assert n_fail == 0, f"{label}: {n_fail} outside the gate plus the bf16 state rounding"
    # out / sum, the attention the layer uses
    with np.errstate(invalid="ignore", divide="ignore"):
        gn = np.where(gs[..., None] > 0, a / gs[..., None], 0.0)
        wn = np.where(ws[..., None] > 0, e / ws[..., None], 0.0)
        an = np.where(ws[..., None] > 0, allow / ws[..., None], 0.0)
    dn = np.abs(gn - wn)
    n_fail = int(np.count_nonzero(dn > 1e-2 + 1e-2 * np.abs(wn) + an))
    say(f"[{label + ' out / sum':40}] max|d|={dn.max():.5f} fail={n_fail}")
    assert n_fail == 0, f"{label}: out / sum, {n_fail} outside the gate plus the bf16 state rounding"


@pytest.mark.parametrize("P,q_std", [(1, 1.0), (1, 0.05), (3, 1.0), (3, 0.05)])
def test_paged_attention_matches_oracle(P, q_std):
    need_gpu()
    say(f"full attention P={P} q_std={q_std}")
    d = synth.cfg_full_attention(seed=3, M=2, P=P, pos=[P * TF - 1, (P - 1) * TF + 100], q_std=q_std)
    check_state(d, f"pages P{P} q{q_std}")


def test_paged_attention_scattered_masks_and_empty_pages():
    need_gpu()
    say("full attention: random masks, a row with nothing valid on page 0")
    d = synth.cfg_full_attention(seed=4, M=3, P=2, q_std=0.2)
    rng = np.random.default_rng(4)
    d["masks"] = (rng.random(d["masks"].shape) < 0.2).astype(np.float32)
    d["masks"][0, 1] = 0.0          # row 1: page 0 empty, so its state starts at -inf / 0 / 0
    d["masks"][:, 2] = 0.0          # row 2: no valid slot at all
    check_state(d, "pages scattered")


def test_paged_attention_single_slot_is_exact():
    need_gpu()
    say("full attention: one valid slot")
    d = synth.cfg_full_attention(seed=5, M=1, P=2)
    d["masks"][:] = 0.0
    d["masks"][1, 0, 300] = 1.0
    gm, gs, go = pages_gpu(d)
    assert np.all(gs == 1.0)
    assert np.array_equal(go[0], np.repeat(d["v_pages"][1, 300][None], GF, axis=0))


def out_gpu(d):
    from moa_amd import ops
    r = dev(d["residual"])
    ops.full_attention_output(dev(d["x"]), torch.from_numpy(d["running_sum"]).cuda(), dev(d["post_attn_rms_weight"]),
                              dev(d["o_weight"]), dev(d["o_weight_scale"]), r)
    return host(r)


def out_oracle(d):
    r = d["residual"].copy()
    O.full_attention_output(d["x"], d["running_sum"], d["post_attn_rms_weight"], d["o_weight"],
                            unbf(d["o_weight_scale"]), r)
    return r


@pytest.mark.parametrize("M", [1, 3])
def test_full_output_matches_oracle(M):
    need_gpu()
    say(f"full attention output M={M}")
    d = synth.cfg_full_o(seed=6, M=M)
    d["running_sum"][0, 5] = 0.0    # a head with no valid slot
    gate(out_oracle(d), out_gpu(d), f"full output M{M}")


def test_full_layer_attention_chain():
    """QKV of the token at position 700 (page 1, slot 188) into a cache whose earlier slots hold
    N(0, 1) K / V, attention over pages 0 and 1, then the output projection."""
    need_gpu()
    from moa_amd import ops
    say("full layer chain: qkv -> pages 0, 1 -> output")
    pos = 700
    d = synth.cfg_full_qkv(seed=7, M=1, pos=pos)
    page0 = synth.cfg_full_attention(seed=7, M=1, P=1)
    k0, v0 = page0["k_pages"][0], page0["v_pages"][0]
    gq, gk1, gv1 = qkv_gpu(d, 1)
    wq, wk1, wv1 = qkv_oracle(d, 1)
    masks = synth.full_masks(2, [pos])
    att = dict(q=wq, k_pages=np.stack([k0, wk1]), v_pages=np.stack([v0, wv1]), masks=masks)
    wm, ws, wo = O.full_attention_pages(att["q"], att["k_pages"], att["v_pages"], masks)
    # the GPU chain runs on its own QKV results
    gm, gs, go = pages_gpu(dict(q=gq, k_pages=np.stack([k0, gk1]), v_pages=np.stack([v0, gv1]), masks=masks))
    o = synth.cfg_full_o(seed=7, M=1)
    w_res = out_oracle(dict(o, x=wo, running_sum=ws))
    g_res = out_gpu(dict(o, x=go, running_sum=gs))
    assert ops.device_errors() == 0
    # residual + bf16(post-norm output): a one-ulp step of the addend may survive a cancellation
    gate_addend(w_res, g_res, o["residual"], "full layer chain residual")


def fused_gpu(d):
    from moa_amd import ops
    P, M = d["masks"].shape[:2]
    mx = torch.zeros(M * GF, dtype=torch.float32, device="cuda")
    sm = torch.zeros(M * GF, dtype=torch.float32, device="cuda")
    out = dev_zeros(M * QF)
    ops.full_attention(dev(d["q"]), dev(d["k_pages"]), dev(d["v_pages"]), dev(d["masks"]), mx, sm, out)
    return host(mx).reshape(M, GF), host(sm).reshape(M, GF), host(out).reshape(M, GF, DF)


@pytest.mark.parametrize("P,M,q_std", [(1, 1, 1.0), (3, 2, 0.05), (8, 1, 1.0), (9, 2, 0.2), (64, 1, 0.05),
                                       (12, 1, 6.0)])
def test_fused_pages_match_oracle(P, M, q_std):
    """moa_full_attention: all pages in two launches (spans of chunks with an online softmax for
    P > 8). Its out is rounded to bf16 once, so the plain gate applies to the state itself."""
    need_gpu()
    say(f"full attention fused P={P} M={M} q_std={q_std}")
    pos = [P * TF - 1] + [(P - 1) * TF + 37 * (m + 1) for m in range(1, M)]
    d = synth.cfg_full_attention(seed=8, M=M, P=P, pos=pos, q_std=q_std)
    gm, gs, go = fused_gpu(d)
    wm, ws, wo = O.full_attention_pages(d["q"], d["k_pages"], d["v_pages"], d["masks"])
    assert np.all(np.abs(gm - wm) <= 1e-3 * (1.0 + np.abs(wm))), "running_max"
    assert np.all(np.abs(gs - ws) <= 1e-3 * np.abs(ws)), "running_sum"
    gate(wo, go, f"fused P{P} out")


def test_fused_pages_agree_with_the_per_page_calls():
    need_gpu()
    say("full attention: fused and per-page states, scattered masks and an empty row")
    d = synth.cfg_full_attention(seed=9, M=3, P=4, q_std=0.3)
    rng = np.random.default_rng(9)
    d["masks"] = (rng.random(d["masks"].shape) < 0.3).astype(np.float32)
    d["masks"][:, 2] = 0.0
    fm, fs, fo = fused_gpu(d)
    pm, ps, po = pages_gpu(d)
    wm, ws, wo = O.full_attention_pages(d["q"], d["k_pages"], d["v_pages"], d["masks"])
    assert np.all(fm[2] == -np.inf) and np.all(fs[2] == 0.0) and not fo[2].any()
    assert np.array_equal(np.isfinite(fm), np.isfinite(pm))
    gate(wo, fo, "fused scattered out")
    fin = np.isfinite(wm)
    assert np.all(np.abs(fm[fin] - pm[fin]) <= 1e-3 * (1.0 + np.abs(pm[fin])))
