"""Pins for the oracle's FP8 and MXFP4 decoder_feedforward branches and its E8M0 decode.

The reference's operator is NVFP4 only (FO/src/ops.rs:201-239); BASELINE configs 0 and 3 use FP8
and MXFP4 weights. Three independent checks pin those branches:
  * orc_e8m0_decode on all 256 codes against torch's float8_e8m0fnu and 2^(e - 127);
  * the whole operator against a torch composition of the reference's own rules at the
    BASELINE shapes: torch's E4M3 / E8M0 decodes, scaled_projection
    (generate_references.py:265-274) for FP8, a bf16 nn.functional.linear over the folded weights
    for MXFP4 (as gen_decoder_feedforward folds its block scales, :395-410), and the bf16 per-op
    chain of gemma4.py:75-89,189-197 and generate_references.py:411-413;
  * FP8 and MXFP4 restatements of the reference's full-FFN stress construction
    (full-ffn-stress/generate_reference.py:34-92) whose answer is derived here in closed form,
    with the intermediates the reference asserts (p[0] = 1024, p[7680] = 0.5, 2^-22 elsewhere).
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as Fn

from kat_inputs import GOLDEN, ffn_stress_inputs_fp8, ffn_stress_inputs_mxfp4, unbf
from moa_amd import synth
from oracle import oracle as O

BF = torch.bfloat16
# E2M1 magnitudes of the OCP MX specification (sign in bit 3), written out independently of the
# oracle's table.
E2M1 = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])


def test_e8m0_decode_all_codes():
    f = O.lib().orc_e8m0_decode
    codes = torch.arange(256, dtype=torch.uint8)
    lib = codes.view(torch.float8_e8m0fnu).float().numpy()
    for e in range(256):
        got = f(e)
        if e == 255:
            assert math.isnan(got) and math.isnan(lib[e])
            continue
        assert got == math.ldexp(1.0, e - 127) == lib[e], e


# ----------------------------------------------------------------- torch composition
def t_bf(bits) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).view(BF)


def t_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def rms_norm(x: torch.Tensor, w: torch.Tensor | None) -> torch.Tensor:
    """gemma4.py:83-89."""
    y = x.float()
    y = y * torch.rsqrt(y.pow(2).mean(-1, keepdim=True) + 1e-6)
    if w is not None:
        y = y * w.float()
    return y.to(BF)


def fp8_proj(x: torch.Tensor, codes: np.ndarray, scale: np.ndarray) -> torch.Tensor:
    """scaled_projection, generate_references.py:265-274, with torch's own E4M3 decode."""
    w = torch.from_numpy(codes).view(torch.float8_e4m3fn).float()
    return ((x.float() @ w.T) * torch.from_numpy(scale).float()).to(BF)


def mxfp4_weight(packed: np.ndarray, scale: np.ndarray, block: int = 32, bias: int = 127) -> torch.Tensor:
    """E2M1 codes (low nibble first) times their E8M0 block scale, folded to bf16 as
    generate_references.py:398,407 folds the NVFP4 local scale."""
    p = torch.from_numpy(packed).long()
    codes = torch.stack([p & 0xF, p >> 4], dim=-1).reshape(packed.shape[0], -1)
    s = torch.from_numpy(scale.astype(np.int64) - (bias - 127)).to(torch.uint8).view(torch.float8_e8m0fnu).float()
    n, k = codes.shape
    # scale of element (n, k) at flat index n * K/32 + k / block (block 16 models a wrong index,
    # running into the next row's scales as a C loop with that index would; wrapped at the end)
    idx = (torch.arange(n)[:, None] * s.shape[1] + torch.arange(k)[None, :] // block) % s.numel()
    return (E2M1[codes] * s.reshape(-1)[idx]).to(BF)


def torch_ffn(d: dict, fmt: str, post=True, scalar=True, **mx):
    """decoder_feedforward composed in torch: returns (output bits, GeGLU row p bits)."""
    r = t_bf(d["residual"]).reshape(-1, 3840)
    h = rms_norm(r, t_bf(d["pre_ff_rms_weight"]))
    if fmt == "fp8":
        proj = {k: (lambda x, k=k: fp8_proj(x, d[f"{k}_weight"], d[f"{k}_weight_scale"])) for k in ("up", "gate", "down")}
    else:
        ws = {k: mxfp4_weight(d[f"{k}_weight_packed"], d[f"{k}_weight_scale"], **mx) for k in ("up", "gate", "down")}
        proj = {k: (lambda x, k=k: Fn.linear(x, ws[k])) for k in ws}
    p = Fn.gelu(proj["gate"](h), approximate="tanh") * proj["up"](h)  # gemma4.py:197, bf16 per op
    y = proj["down"](p)
    if post:
        y = rms_norm(y, t_bf(d["post_ff_rms_weight"]))
    out = (r + y).to(BF)
    if scalar:
        out = (out * t_bf(d["layer_scalar"])[0]).to(BF)
    return t_bits(out), t_bits(p)


def oracle_ffn(d: dict, fmt: str, post=True, scalar=True):
    if fmt == "fp8":
        w = O.ffn_weights(O.FFN_FP8, d["up_weight"], d["gate_weight"], d["down_weight"], d["up_weight_scale"],
                          d["gate_weight_scale"], d["down_weight_scale"])
    else:
        w = O.ffn_weights(O.FFN_MXFP4, d["up_weight_packed"], d["gate_weight_packed"], d["down_weight_packed"],
                          d["up_weight_scale"], d["gate_weight_scale"], d["down_weight_scale"])
    r = np.ascontiguousarray(d["residual"]).reshape(-1, 3840).copy()
    h = np.stack([O.rmsnorm(row, d["pre_ff_rms_weight"]) for row in r])
    p = O.ffn_up_gate(h, w)
    O.decoder_feedforward(r, d["pre_ff_rms_weight"], w, d["post_ff_rms_weight"] if post else None,
                          d["layer_scalar"] if scalar else None)
    return r, p


def ulps(a_bits, b_bits) -> np.ndarray:
    """|a - b| in bf16 ulps of the larger magnitude (0 where equal)."""
    a, b = unbf(a_bits).astype(np.float64), unbf(b_bits).astype(np.float64)
    m = np.maximum(np.abs(a), np.abs(b))
    ulp = np.where(m > 0, np.exp2(np.floor(np.log2(np.where(m > 0, m, 1))) - 7), 1)
    return np.abs(a - b) / ulp


@pytest.fixture(scope="module")
def cfg0():
    return synth.cfg_ffn_fp8(0)


@pytest.fixture(scope="module")
def cfg3():
    return synth.cfg_ffn_mxfp4(0, M=2)


def check_vs_torch(d, fmt, post=True, scalar=True):
    want, want_p = torch_ffn(d, fmt, post, scalar)
    got, got_p = oracle_ffn(d, fmt, post, scalar)
    got, got_p = got.reshape(want.shape), got_p.reshape(want_p.shape)
    # The f32 sums are exactly rounded in the oracle and in torch's own order in torch: a bf16
    # rounding of up or gate may flip by one ulp where a sum lies within an f32 ulp of a midpoint
    # (cfg0 seed 0: 2 of 15360 GeGLU elements, no output). p = bf16(a x up) then moves by up to
    # two ulps of p (seen: one element of seed 1, 0x3b4d vs 0x3b4b). torch's vectorised tanh also
    # lets 1 + tanh cancel to 0 near gate = -5 where libm's leaves ~1e-7 (cfg3: gelu(-5.125) gives
    # -1.8e-7 vs -0.0), the gelu difference test_formats.py bounds by 2^-20.
    far = (ulps(got_p, want_p) > 2.0) & (np.abs(unbf(got_p) - unbf(want_p)) > 2.0 ** -20)
    assert not far.any(), np.argwhere(far)
    assert np.count_nonzero(got_p != want_p) <= want_p.size // 1000
    np.testing.assert_array_less(ulps(got, want), 1.0 + 1e-9)
    assert np.count_nonzero(got != want) <= max(1, want.size // 1000)
    return int(np.count_nonzero(got != want)), int(np.count_nonzero(got_p != want_p))


def test_fp8_ffn_vs_torch_composition_config0(cfg0):
    """BASELINE config 0 (M = 1, seed 0), the full operator with post-norm and layer scalar."""
    n_out, n_p = check_vs_torch(cfg0, "fp8")
    print(f"fp8 cfg0: {n_out} outputs, {n_p} GeGLU elements differ from torch")


def test_fp8_ffn_vs_torch_composition_literal(cfg0):
    """Config 0 read literally: no post-norm, no layer scalar (r + bf16(d))."""
    check_vs_torch(cfg0, "fp8", post=False, scalar=False)


def test_fp8_ffn_vs_torch_composition_two_rows():
    check_vs_torch(synth.cfg_ffn_fp8(1, M=2), "fp8")


def test_mxfp4_ffn_vs_torch_composition_config3(cfg3):
    """BASELINE config 3 (seed 0) on two rows."""
    n_out, n_p = check_vs_torch(cfg3, "mxfp4")
    print(f"mxfp4 cfg3: {n_out} outputs, {n_p} GeGLU elements differ from torch")


def test_mxfp4_composition_detects_a_wrong_block_index_or_bias(cfg3):
    """The check above bites: a block-16 index or an E8M0 bias of 128 in the composition moves
    most outputs away from the oracle's."""
    got, _ = oracle_ffn(cfg3, "mxfp4")
    for mx in (dict(block=16), dict(bias=128)):
        out, _ = torch_ffn(cfg3, "mxfp4", **mx)
        assert np.count_nonzero(out != got.reshape(out.shape)) > out.size // 2, mx


# ----------------------------------------------------------------- closed-form stress answers
def stress_expected() -> np.uint16:
    """The stress answer from the construction: h = RMSNorm(1) = 1; every down row gives
    d = 169 x 2^-21; the post-norm of a vector of equal d is d / sqrt(d^2 + eps) (eps matters:
    d^2 = 6.5e-9); out = bf16(bf16(1 + n) x 0.375)."""
    d = 169 * 2.0 ** -21
    n_exact = d / math.sqrt(d * d + 1e-6)
    n = float(unbf(O.bf16_rne(np.float32(n_exact)))[0])
    # n lies 0.006 bf16 ulps above a rounding midpoint: no f32 evaluation order can cross it
    assert abs(n_exact * 2 ** 11 - 164.5) > 1e-3
    s = float(unbf(O.bf16_rne(np.float32(1.0 + n)))[0])
    out = O.bf16_rne(np.float32(s * 0.375))[0]
    return out


def check_stress(d: dict, fmt: str):
    want = stress_expected()
    ref = np.fromfile(GOLDEN / "ffn_stress_expected_bf16.bin", dtype="<u2")
    assert want == 0x3ECF and np.all(ref == want)  # the reference's recorded NVFP4 answer
    r, p = oracle_ffn(d, fmt)
    pf = unbf(p[0])
    assert pf[0] == 1024 and pf[7680] == 0.5
    assert np.all(pf[1:7680] == 2.0 ** -22) and np.all(pf[7681:] == 2.0 ** -22)
    assert np.all(r == want)
    # the torch composition agrees on the same inputs
    t_out, t_p = torch_ffn(d, fmt)
    assert np.array_equal(t_p, p.reshape(t_p.shape)) and np.all(t_out == want)


def test_fp8_stress_known_answer():
    check_stress(ffn_stress_inputs_fp8(), "fp8")


def test_mxfp4_stress_known_answer():
    check_stress(ffn_stress_inputs_mxfp4(), "mxfp4")


def test_mxfp4_stress_detects_a_wrong_block_index_or_bias():
    """The stress construction itself bites: with a block-16 index or a bias of 128 the torch
    composition leaves the closed-form answer."""
    d = ffn_stress_inputs_mxfp4()
    for mx in (dict(block=16), dict(bias=128)):
        out, _ = torch_ffn(d, "mxfp4", **mx)
        assert np.all(out != 0x3ECF), mx


def test_fp8_stress_detects_a_row_scale_index_error():
    d = ffn_stress_inputs_fp8()
    bad = dict(d)
    bad["down_weight_scale"] = np.roll(d["down_weight_scale"], 1)
    out, _ = torch_ffn(bad, "fp8")
    assert np.all(out != 0x3ECF)
