"""Guard bands and non-finite inputs.

Canaries: every in-place or written output (QKV's q_out and both ring caches, O's and the FFN's
residual) is placed inside a larger device buffer whose bytes before and after it hold a canary
pattern; after the call the canaries must be intact and the output must equal, bit for bit, the
same call on an unguarded buffer. This runs each operator's paths: one token row (single-launch
kernels), 16 rows (matrix-core rows path) and 17 / 256 rows (MFMA chunk path, FP8 weights; FP4
weights in tiles of 16).

Non-finite inputs: the reference's gate fails on any non-finite output
(FO/src/bin/test_kernels.rs:641-644). A NaN injected into an input must reach exactly the outputs
the oracle's NaN reaches (propagation parity), and the gate must reject the result."""
import numpy as np
import pytest

from gpu_util import dev, host, need_gpu, say, torch
from kat_inputs import compare, unbf
from moa_amd import synth
from oracle import oracle as O
from test_gpu_ffn import oracle_fp8, oracle_mxfp4, oracle_nvfp4

pytestmark = pytest.mark.gpu
G = 512  # guard elements on each side (1 KB of bf16): keeps the output 16-byte aligned
CANARY = 0x7E5A  # a finite bf16 (about 7.2e37) that no output of these inputs takes


def guarded(a: np.ndarray):
    """(buffer, view): the view is the output, framed by G canary elements on each side."""
    flat = np.ascontiguousarray(a).reshape(-1)
    buf = np.full(flat.size + 2 * G, CANARY, np.uint16)
    buf[G:G + flat.size] = flat
    t = dev(buf)
    return t, t[G:G + flat.size]


def intact(t, label: str):
    b = host(t)
    assert np.all(b[:G] == CANARY) and np.all(b[-G:] == CANARY), f"{label}: a canary was overwritten"
    return b[G:-G]


def ffn_call(fmt: str, d: dict, residual):
    from moa_amd import ops
    if fmt == "fp8":
        ops.decoder_feedforward_fp8(residual, dev(d["pre_ff_rms_weight"]), dev(d["up_weight"]), dev(d["gate_weight"]),
                                    dev(d["down_weight"]), dev(d["up_weight_scale"]), dev(d["gate_weight_scale"]),
                                    dev(d["down_weight_scale"]), dev(d["post_ff_rms_weight"]), dev(d["layer_scalar"]))
    elif fmt == "mxfp4":
        ops.decoder_feedforward_mxfp4(residual, dev(d["pre_ff_rms_weight"]), dev(d["up_weight_packed"]),
                                      dev(d["gate_weight_packed"]), dev(d["down_weight_packed"]),
                                      dev(d["up_weight_scale"]), dev(d["gate_weight_scale"]),
                                      dev(d["down_weight_scale"]), dev(d["post_ff_rms_weight"]), dev(d["layer_scalar"]))
    else:
        ops.decoder_feedforward(residual, dev(d["pre_ff_rms_weight"]), dev(d["up_weight_packed"]),
                                dev(d["gate_weight_packed"]), dev(d["down_weight_packed"]), dev(d["up_weight_scale"]),
                                dev(d["gate_weight_scale"]), dev(d["down_weight_scale"]), dev(d["up_global_scale"]),
                                dev(d["gate_global_scale"]), dev(d["down_global_scale"]), dev(d["post_ff_rms_weight"]),
                                dev(d["layer_scalar"]))


_ffn = {}


def ffn_case(fmt: str, M: int) -> dict:
    if fmt not in _ffn:
        _ffn[fmt] = {"fp8": lambda: synth.cfg_ffn_fp8(9), "mxfp4": lambda: synth.cfg_ffn_mxfp4(9),
                     "nvfp4": lambda: synth.ref_ffn_inputs(2)}[fmt]()
    return dict(_ffn[fmt], residual=synth.bf16_normal(f"guard.{fmt}.M{M}", (M, 3840)))


@pytest.mark.parametrize("fmt,M", [("fp8", 1), ("fp8", 16), ("fp8", 17), ("fp8", 256), ("nvfp4", 1), ("nvfp4", 16),
                                   ("mxfp4", 1), ("mxfp4", 16), ("mxfp4", 17)])
def test_ffn_residual_guard_bands(fmt, M):
    need_gpu()
    say(f"guards: ffn {fmt} M{M}")
    d = ffn_case(fmt, M)
    buf, r = guarded(d["residual"])
    ffn_call(fmt, d, r)
    got = intact(buf, f"ffn {fmt} M{M}")
    plain = dev(d["residual"])
    ffn_call(fmt, d, plain)
    assert np.array_equal(got, host(plain).reshape(-1))


@pytest.mark.parametrize("M", [1, 16, 17, 256])
def test_o_residual_guard_bands(M):
    need_gpu()
    from moa_amd import ops
    say(f"guards: o M{M}")
    d = synth.cfg_o(9, M=M)
    args = (dev(d["x"]), dev(d["post_attn_rms_weight"]), dev(d["o_weight"]), dev(d["o_weight_scale"]))
    buf, r = guarded(d["residual"])
    ops.sliding_attention_output(*args, r)
    got = intact(buf, f"o M{M}")
    plain = dev(d["residual"])
    ops.sliding_attention_output(*args, plain)
    assert np.array_equal(got, host(plain).reshape(-1))


@pytest.mark.parametrize("M", [1, 16, 17, 256])
def test_qkv_output_guard_bands(M):
    need_gpu()
    from moa_amd import ops
    say(f"guards: qkv M{M}")
    d = synth.cfg_qkv(9, M=M, pos=1000)  # the ring wraps inside the longer calls
    w = [dev(d[k]) for k in ("x", "q_weight", "k_weight", "v_weight", "q_weight_scale", "k_weight_scale",
                             "v_weight_scale", "input_rms_weight", "q_rms_weight", "k_rms_weight")]
    kv = torch.tensor([d["kv_offset"]], dtype=torch.int32, device="cuda")
    ro = torch.tensor([d["rope_offset"]], dtype=torch.int32, device="cuda")
    tabs = [dev(d["cos"]), dev(d["sin"])]
    kb, kc = guarded(d["k_cache"])
    vb, vc = guarded(d["v_cache"])
    qb, qo = guarded(np.zeros(M * 4096, np.uint16))
    ops.sliding_project_qkv(*w, kv, ro, *tabs, kc, vc, qo)
    got = [intact(kb, "k_cache"), intact(vb, "v_cache"), intact(qb, "q_out")]
    kc2, vc2, qo2 = dev(d["k_cache"]), dev(d["v_cache"]), dev(np.zeros(M * 4096, np.uint16))
    ops.sliding_project_qkv(*w, kv, ro, *tabs, kc2, vc2, qo2)
    for g, p, name in zip(got, (kc2, vc2, qo2), ("k_cache", "v_cache", "q_out")):
        assert np.array_equal(g, host(p).reshape(-1)), name


# ------------------------------------------------------------------ non-finite inputs

def nan_parity(want_bits, got_bits, label: str):
    want_bits, got_bits = np.asarray(want_bits).reshape(-1), np.asarray(got_bits).reshape(-1)
    wn, gn = np.isnan(unbf(want_bits)), np.isnan(unbf(got_bits))
    say(f"[{label:40}] oracle NaN outputs {int(wn.sum())}, kernel NaN outputs {int(gn.sum())}")
    assert wn.any(), f"{label}: the injected NaN did not reach the oracle's output"
    assert np.array_equal(wn, gn), f"{label}: NaN reaches different outputs"
    fin = ~wn
    ok, _, _, _ = compare(unbf(want_bits)[fin], got_bits[fin], 1e-2)
    assert ok, f"{label}: finite outputs outside the gate"
    ok, _, _, nfail = compare(unbf(want_bits), got_bits, 1e-2)
    assert not ok and nfail > 0, f"{label}: the gate accepted non-finite outputs"


@pytest.mark.parametrize("M", [1, 16])
def test_nan_residual_element_in_ffn(M):
    need_gpu()
    say(f"nan: ffn fp8 residual M{M}")
    d = ffn_case("fp8", M)
    d["residual"] = d["residual"].copy()
    d["residual"][M - 1, 1234] = 0x7FC0
    r = dev(d["residual"])
    ffn_call("fp8", d, r)
    nan_parity(oracle_fp8(d), host(r), f"nan ffn fp8 M{M}")


def test_nan_weight_code_in_o():
    """E4M3 code 0x7F is NaN: one O weight row carries it."""
    need_gpu()
    from moa_amd import ops
    from test_gpu_o import run_oracle
    say("nan: o weight code")
    d = synth.cfg_o(10)
    d["o_weight"] = d["o_weight"].copy()
    d["o_weight"][77, 4000] = 0x7F
    r = dev(d["residual"])
    ops.sliding_attention_output(dev(d["x"]), dev(d["post_attn_rms_weight"]), dev(d["o_weight"]),
                                 dev(d["o_weight_scale"]), r)
    nan_parity(run_oracle(d), host(r), "nan o weight")


def test_nan_activation_in_qkv():
    need_gpu()
    from test_gpu_qkv import run_gpu, run_oracle
    say("nan: qkv x")
    d = synth.cfg_qkv(10)
    d["x"] = d["x"].copy()
    d["x"][0, 5] = 0xFFC0
    q, kc, vc = run_gpu(d)
    qe, kce, vce = run_oracle(d)
    nan_parity(qe, q, "nan qkv q_out")
    slot = d["kv_offset"] // 4096
    nan_parity(kce[slot], kc[slot], "nan qkv k slot")
    keep = np.ones(1024, bool)
    keep[slot] = False
    assert np.array_equal(kc[keep], d["k_cache"][keep]) and np.array_equal(vc[keep], d["v_cache"][keep])
