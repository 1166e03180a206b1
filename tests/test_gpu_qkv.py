"""ops::sliding_project_qkv on the GPU vs the CPU oracle and the reference's known answers.
Every cache slot outside the written window must stay bit-identical."""
import numpy as np
import pytest

from gpu_util import dev, dev_zeros, gate, host, need_gpu, say, torch
from kat_inputs import qkv_boundary_case, qkv_raw_case, load_json, sha, unbf
from moa_amd import prng, synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def run_gpu(d, M=1, bf16_scales=False, kc=None, vc=None):
    from moa_amd import ops
    t = {k: dev(d[k]) for k in ("x", "q_weight", "k_weight", "v_weight", "input_rms_weight", "q_rms_weight",
                                "k_rms_weight", "cos", "sin")}
    sc = {}
    for k in ("q_weight_scale", "k_weight_scale", "v_weight_scale"):
        a = d[k]
        if bf16_scales:
            sc[k] = dev(a if a.dtype == np.uint16 else prng.f32_to_bf16_bits(a))
        else:
            sc[k] = dev(a if a.dtype == np.float32 else unbf(a))
    kc_t = dev(d["k_cache"] if kc is None else kc)
    vc_t = dev(d["v_cache"] if vc is None else vc)
    q_out = dev(d.get("q_out", np.zeros(M * 4096, np.uint16)))
    kv = torch.tensor([d["kv_offset"]], dtype=torch.int32, device="cuda")
    ro = torch.tensor([d["rope_offset"]], dtype=torch.int32, device="cuda")
    ops.sliding_project_qkv(t["x"], t["q_weight"], t["k_weight"], t["v_weight"], sc["q_weight_scale"],
                            sc["k_weight_scale"], sc["v_weight_scale"], t["input_rms_weight"], t["q_rms_weight"],
                            t["k_rms_weight"], kv, ro, t["cos"], t["sin"], kc_t, vc_t, q_out)
    return host(q_out), host(kc_t), host(vc_t)


def run_oracle(d, M=1):
    kc, vc = d["k_cache"].copy(), d["v_cache"].copy()
    qo = np.zeros(M * 4096, np.uint16)
    f = lambda k: d[k] if d[k].dtype == np.float32 else unbf(d[k])
    O.sliding_project_qkv(d["x"], d["q_weight"], d["k_weight"], d["v_weight"], f("q_weight_scale"),
                          f("k_weight_scale"), f("v_weight_scale"), d["input_rms_weight"], d["q_rms_weight"],
                          d["k_rms_weight"], d["kv_offset"], d["rope_offset"], d["cos"], d["sin"], kc, vc, qo)
    return qo, kc, vc


def slots(d, M):
    s0 = d["kv_offset"] // 4096
    return [(s0 + m) % 1024 for m in range(M)]


def check_against_oracle(d, label, M=1):
    """The reference's own gate (test_kernels.rs:626-671) plus the sign rule on q, k and v: no
    per-element allowance on these decode paths."""
    q, kc, vc = run_gpu(d, M)
    qe, kce, vce = run_oracle(d, M)
    gate(qe, q, f"{label} q")
    ss = slots(d, M)
    gate(kce[ss], kc[ss], f"{label} k")
    gate(vce[ss], vc[ss], f"{label} v")
    keep = np.ones(1024, bool)
    keep[ss] = False
    assert np.array_equal(kc[keep], d["k_cache"][keep]), f"{label}: k_cache changed outside the slot"
    assert np.array_equal(vc[keep], d["v_cache"][keep]), f"{label}: v_cache changed outside the slot"


@pytest.mark.parametrize("case", [0, 1])
def test_boundary_known_answer_exact(case):
    """qkv-boundary-probe-e53: expected q/k/v bits; sentinel-filled caches preserved."""
    need_gpu()
    say(f"qkv boundary case {case}")
    d = qkv_boundary_case(case)
    q, kc, vc = run_gpu(d, bf16_scales=True)
    slot = d["kv_offset"] // 4096
    assert np.array_equal(unbf(q), d["expected"]["q"])
    assert np.array_equal(unbf(kc[slot].reshape(-1)), d["expected"]["k"])
    assert np.array_equal(unbf(vc[slot].reshape(-1)), d["expected"]["v"])
    keep = np.ones(1024, bool)
    keep[slot] = False
    assert np.all(kc[keep] == 0x3E80) and np.all(vc[keep] == 0xBF00)


@pytest.mark.parametrize("run", range(9))
def test_reference_runs(run):
    """The reference harness's runs 0-2 and the extra seeds 3-8 (moa-dev/extra_seeds.py:25,103-110),
    with the caches pre-filled by seeded sentinels instead of zeros."""
    need_gpu()
    say(f"qkv reference run {run}")
    d = synth.ref_qkv_inputs(run)
    d["k_cache"] = prng.bf16_uniform(f"run{run}.sentinel.k_cache", 1024 * 8 * 256, -2, 2).reshape(1024, 8, 256)
    d["v_cache"] = prng.bf16_uniform(f"run{run}.sentinel.v_cache", 1024 * 8 * 256, -2, 2).reshape(1024, 8, 256)
    check_against_oracle(d, f"qkv run{run}")


@pytest.mark.parametrize("seed,theta", [(0, 1e4), (1, 1e4), (2, 1e6)])
def test_baseline_config2(seed, theta):
    need_gpu()
    say(f"qkv cfg2 seed {seed} theta {theta}")
    d = synth.cfg_qkv(seed, theta=theta)
    check_against_oracle(d, f"qkv cfg2 s{seed}")


def test_multi_row_wraps_the_ring():
    """M = 4 rows at positions 1022..1025: slots 1022, 1023, 0, 1."""
    need_gpu()
    d = synth.cfg_qkv(5, M=4, pos=1022)
    check_against_oracle(d, "qkv M4 wrap", M=4)


def test_bf16_scale_entry_point_bit_identical():
    need_gpu()
    d = synth.ref_qkv_inputs(1)
    d["k_cache"] = np.zeros((1024, 8, 256), np.uint16)
    d["v_cache"] = np.zeros((1024, 8, 256), np.uint16)
    a = run_gpu(d, bf16_scales=True)
    b = run_gpu(d, bf16_scales=False)
    c = run_gpu(d, bf16_scales=False)
    for x, y, z in zip(a, b, c):
        assert np.array_equal(x, y) and np.array_equal(y, z)  # exact widening; deterministic


def test_bad_offsets_write_nothing_and_raise_a_device_error():
    need_gpu()
    from moa_amd import ops
    d = synth.cfg_qkv(3)
    for field, value, bit in (("rope_offset", 32768 * 512, ops._lib.DEVERR_ROPE_OFFSET),
                              ("kv_offset", 1024 * 4096, ops._lib.DEVERR_KV_OFFSET),
                              ("kv_offset", 100, ops._lib.DEVERR_KV_OFFSET)):
        e = dict(d)
        e[field] = value
        ops.device_errors()  # clear
        e["q_out"] = np.full(4096, 0x3FC0, np.uint16)
        q, kc, vc = run_gpu(e)
        assert ops.device_errors() & bit
        assert np.array_equal(kc, d["k_cache"]) and np.array_equal(vc, d["v_cache"])
        assert np.all(q == 0x3FC0)
    assert ops.device_errors() == 0


@pytest.mark.parametrize("case", range(9))
def test_raw_projection_known_answers(case):
    """The 9 QKV raw-projection probes through the projection entry point: exact sha256."""
    need_gpu()
    from moa_amd import ops
    rec = load_json("qkv_raw_truth.json")["cases"][case]
    x, mats = qkv_raw_case(case)
    for key in ("q", "k", "v"):
        codes, sbits = mats[key]
        out = dev_zeros(codes.shape[0])
        ops.fp8_scaled_projection(dev(x), dev(codes), dev(unbf(sbits)), out)
        assert sha(host(out)) == rec["outputs"][key]["expected_sha256"], (case, key)
