"""The C++ host interface (moa-workspace_amd/host/moa_ops.hpp) through its harness,
tests/cpp/test_kernels: the reference harness's flow (FO/src/bin/test_kernels.rs) in C++ --
inputs synthesised from the reference PRNG by name, the three operators run through moa::ops,
each output graded against the oracle.

CPU: the harness's synthesis agrees with the Python one (moa_amd.synth, whose checksums the
golden PRNG vectors pin) tensor by tensor, as the reference's Synth::verify checks its inputs
against the fixture's checksums before anything runs. GPU: every check of runs 0-2 passes."""
import subprocess
from pathlib import Path

import pytest

from moa_amd import synth

HARNESS = Path(__file__).resolve().parent / "cpp" / "test_kernels"


def run(*args, timeout=120):
    if not HARNESS.exists():
        pytest.fail(f"{HARNESS} is not built (run __graft_entry__.build())")
    return subprocess.run([str(HARNESS), *args], capture_output=True, text=True, timeout=timeout)


def test_harness_synthesis_matches_python():
    res = run("--checksums", "--runs", "2")
    assert res.returncode == 0, res.stderr
    got = {}
    for line in res.stdout.splitlines():
        test, r, name, c = line.split()
        got[(test, int(r), name)] = int(c)
    want = {}
    for r in range(2):
        for test, fn in (("sliding_project_qkv", synth.ref_qkv_inputs), ("sliding_attention_output", synth.ref_o_inputs),
                         ("decoder_feedforward", synth.ref_ffn_inputs)):
            for name, c in fn(r)["checks"].items():
                want[(test, r, name)] = c
    assert len(want) == 62
    bad = {k: (got.get(k), v) for k, v in want.items() if got.get(k) != v}
    assert not bad, bad
    assert set(got) == set(want)


def test_harness_lists_the_reference_table():
    res = run("--list")
    assert res.returncode == 0
    assert [l.split()[0] for l in res.stdout.splitlines()] == [
        "sliding_project_qkv", "sliding_attention_output", "decoder_feedforward"]


def test_harness_rejects_bad_arguments():
    assert run("--runs", "0").returncode == 2
    assert run("--bogus").returncode == 2


@pytest.mark.gpu
def test_harness_passes_on_the_gpu():
    from gpu_util import need_gpu, say
    need_gpu()
    say("C++ harness, runs 0-2")
    res = run("--runs", "3", "--time", "50", "--graph", timeout=300)
    print(res.stdout, flush=True)
    assert res.returncode == 0, res.stdout + res.stderr
    lines = res.stdout.splitlines()
    assert sum(1 for l in lines if l.rstrip().endswith("-> PASS")) == 3 * (4 + 1 + 1) + 1 + 1
    assert any(l.startswith("PASS: 0 of 11 checks failed") for l in lines)
    # host-driven through moa::ops: one line per operator, a positive time per call
    times = [l for l in lines if l.startswith("[time ")]
    assert len(times) == 3
    assert all(float(l.split("]")[1].split()[0]) > 0 for l in times)
    # the step captured into a HIP graph through moa::ops replays with the eager bits
    assert any(l.startswith("[graph: QKV, O, FFN") and l.rstrip().endswith("-> PASS") for l in lines)


def test_harness_without_a_device_fails_with_the_library_error():
    """No GPU (this container): moa::Device's set-up throws moa::Error carrying the library's
    reason, and the harness exits 1 instead of aborting."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a device is visible")
    res = run("--runs", "1")
    assert res.returncode == 1, res.stdout + res.stderr
    assert "FAIL:" in res.stdout and "code" in res.stdout, res.stdout
