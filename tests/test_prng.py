"""The reference's name-addressed input synthesis: oracle (C) and package (numpy) restatements
against published hash/PRNG vectors, the reference's recorded values, and golden vectors."""
import json

import numpy as np
import pytest

from kat_inputs import GOLDEN, qkv_boundary_case, qkv_raw_case, load_json
from moa_amd import prng
from oracle import oracle as O

# FNV-1a 64 published test vectors (Fowler/Noll/Vo reference set).
FNV = {"": 0xCBF29CE484222325, "a": 0xAF63DC4C8601EC8C, "foobar": 0x85944171F73967E8}


@pytest.mark.parametrize("s,h", FNV.items())
def test_fnv1a_published_vectors(s, h):
    assert prng.name_hash(s) == h
    assert O.name_hash(s) == h


def test_splitmix64_published_first_output():
    # Vigna's splitmix64 from state 0 yields 0xe220a8397b1dcdaf first; the reference's word is
    # that output for state (hash ^ index), so hash ^ index == 0 must reproduce it.
    h = prng.name_hash("x")
    assert int(prng.words("x", 1, offset=h)[0]) == 0xE220A8397B1DCDAF
    assert O.word(h, h) == 0xE220A8397B1DCDAF


def test_run0_position_is_1763():
    # qkv-boundary-probe-e53/generate_suite.py:41-42 asserts the reference's _run_pos(0) == 1763.
    assert prng.run_pos(0) == 1763
    assert O.run_pos(0) == 1763
    assert all(1 <= prng.run_pos(r) <= 2047 and prng.run_pos(r) == O.run_pos(r) for r in range(9))


def test_golden_prng_vectors():
    g = json.loads((GOLDEN / "prng_vectors.json").read_text())
    for name, h in g["name_hash"].items():
        assert prng.name_hash(name) == h and O.name_hash(name) == h
    for name, ws in g["words"].items():
        assert [int(w) for w in prng.words(name, 4, 1000)] == ws
    for c in g["cases"]:
        kind, name, args, want = c["kind"], c["name"], c["args"], c["values"]
        n = len(want)
        if kind == "bf16_uniform":
            ours, orc = prng.bf16_uniform(name, n, *args), O.bf16_uniform(name, n, *args)
        elif kind == "f32_uniform":
            ours, orc = prng.f32_uniform(name, n, *args), O.f32_uniform(name, n, *args)
            want = np.array(want, np.float32)
        elif kind == "bf16_signs":
            ours, orc = prng.bf16_signs(name, n, *args), O.bf16_signs(name, n, *args)
        elif kind == "f8_banded":
            ours, orc = prng.f8_banded(name, n, *args), O.f8_banded(name, n, *args)
        elif kind == "f4_nibbles":
            ours, orc = prng.f4_nibbles(name, 2 * n), O.f4_nibbles(name, 2 * n)
        else:
            raise AssertionError(kind)
        assert np.array_equal(ours, np.asarray(want, dtype=ours.dtype)), (kind, name)
        assert np.array_equal(orc, ours), (kind, name)
        assert prng.checksum(ours) == c["checksum"] == O.checksum(ours), (kind, name)


def test_checksum_matches_qkv_boundary_fixture():
    # boundary.safetensors records the reference checksum of every (formula-built) input.
    for case in (0, 1):
        d = qkv_boundary_case(case)
        want = d["checksums"]
        for key in ("x", "input_rms_weight", "q_rms_weight", "k_rms_weight", "q_weight", "k_weight",
                    "v_weight", "q_weight_scale", "k_weight_scale", "v_weight_scale"):
            assert prng.checksum(d[key]) == want[key] == O.checksum(d[key]), (case, key)
        assert prng.checksum(d["cos"]) == want["cos"]
        assert prng.checksum(d["sin"]) == want["sin"]
        assert prng.checksum(d["k_cache"]) == want["k_cache_init"]
        assert prng.checksum(d["q_out"]) == want["q_out_init"]
        assert prng.checksum(np.array([d["kv_offset"]], np.int32)) == want["kv_offset"]
        assert prng.checksum(np.array([d["rope_offset"]], np.int32)) == want["rope_offset"]


@pytest.mark.parametrize("case", range(9))
def test_checksum_matches_qkv_raw_truth(case):
    rec = load_json("qkv_raw_truth.json")["cases"][case]
    x, mats = qkv_raw_case(case)
    assert prng.checksum(x) == rec["checksums"]["x"]
    for key in ("q", "k", "v"):
        codes, scale = mats[key]
        assert prng.checksum(scale) == rec["checksums"][f"{key}_scale"], (case, key)
        assert prng.checksum(codes) == rec["checksums"][f"{key}_weight"], (case, key)


def test_reference_run_synthesis_is_self_consistent():
    # x_exact = bf16(sign / input_rms_weight) (test_kernels.rs:360-379): (x * inv) * w = sign * inv,
    # so the normalised activation is one magnitude with the drawn signs (up to bf16 rounding).
    from moa_amd import synth
    d = synth.ref_qkv_inputs(0)
    h = O.rmsnorm(d["x"], d["input_rms_weight"])
    vals = O.bf16_to_f32(h)
    assert d["pos"] == 1763 and d["kv_offset"] == 739 * 4096 and d["rope_offset"] == 1763 * 512
    mag = np.median(np.abs(vals))
    assert np.all(np.abs(np.abs(vals) - mag) <= 2 * mag * 2 ** -8)
    assert np.array_equal(np.signbit(vals), np.signbit(O.bf16_to_f32(d["x"])))
