"""moa_decoder_feedforward_fp8_noalloc (static device scratch, no allocation) against
moa_decoder_feedforward_fp8 (the per-device hipMalloc'd scratch), both called through the C ABI:
the same kernels must give the same bits. Two calls in a row, the second with fewer rows (16 rows
on the matrix-core rows path, then one row on the single-launch kernel, then five), so the second
runs on the scratch the first left behind; then a call beyond the stated maximum is rejected.
A fresh process that makes the no-allocation call first, and reads its error word, never creates
the hipMalloc'd scratch of the other entry points."""
import ctypes as C
import json
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from gpu_util import dev, host, need_gpu, say, torch
from moa_amd import _lib, synth

pytestmark = pytest.mark.gpu


def _call(name, d, r):
    M = r.numel() // 3840
    args = [C.c_void_p(r.data_ptr())] + [C.c_void_p(d[k].data_ptr()) for k in (
        "pre_ff_rms_weight", "up_weight", "gate_weight", "down_weight", "up_weight_scale", "gate_weight_scale",
        "down_weight_scale", "post_ff_rms_weight", "layer_scalar")]
    return getattr(_lib.load(), name)(*args, M, C.c_void_p(torch.cuda.current_stream().cuda_stream))


def test_noalloc_matches_the_allocating_entry_point():
    need_gpu()
    from moa_amd import ops
    w = synth.cfg_ffn_fp8(12)
    d = {k: dev(v) for k, v in w.items() if k != "residual"}
    for M in (16, 1, 5):
        say(f"no-alloc fp8 ffn M{M} vs moa_decoder_feedforward_fp8")
        res = synth.bf16_normal(f"noalloc.M{M}.residual", (M, 3840))
        a, b = dev(res), dev(res)
        assert _call("moa_decoder_feedforward_fp8_noalloc", d, a) == 0, _lib.load().moa_last_error_string()
        assert _call("moa_decoder_feedforward_fp8", d, b) == 0, _lib.load().moa_last_error_string()
        ga, gb = host(a), host(b)
        assert np.array_equal(ga, gb), f"M{M}: {np.count_nonzero(ga != gb)} elements differ"
        assert not np.array_equal(ga, res.reshape(-1)), f"M{M}: the residual was not updated"
    assert ops.device_errors() == 0


def test_noalloc_rejects_more_rows_than_its_scratch_holds():
    need_gpu()
    lib = _lib.load()
    w = synth.cfg_ffn_fp8(12)
    d = {k: dev(v) for k, v in w.items() if k != "residual"}
    r = dev(np.zeros((17, 3840), np.uint16))
    assert _call("moa_decoder_feedforward_fp8_noalloc", d, r) == -1
    assert b"no-allocation" in lib.moa_last_error_string()
    assert np.all(host(r) == 0)


CHILD = r"""
import ctypes as C, json, sys
import numpy as np, torch
sys.path[:0] = sys.argv[1].split(os.pathsep)
from moa_amd import _lib, synth
lib = _lib.load()
w = synth.cfg_ffn_fp8(12)
d = {k: torch.from_numpy(np.ascontiguousarray(v).view(np.int16) if v.dtype == np.uint16 else v).cuda()
     for k, v in w.items() if k != "residual"}
out = {}
for M in (1, 4):
    r = torch.from_numpy(synth.bf16_normal(f"noalloc.M{M}.residual", (M, 3840)).view(np.int16)).cuda()
    args = [C.c_void_p(r.data_ptr())] + [C.c_void_p(d[k].data_ptr()) for k in (
        "pre_ff_rms_weight", "up_weight", "gate_weight", "down_weight", "up_weight_scale", "gate_weight_scale",
        "down_weight_scale", "post_ff_rms_weight", "layer_scalar")]
    rc = lib.moa_decoder_feedforward_fp8_noalloc(*args, M, C.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, lib.moa_last_error_string()
    bits = C.c_uint32(99)
    assert lib.moa_device_errors(C.c_void_p(torch.cuda.current_stream().cuda_stream), C.byref(bits)) == 0
    state = C.c_uint32(0)
    assert lib.moa_test_scratch_state(C.byref(state)) == 0
    out[M] = dict(bits=bits.value, state=state.value, residual=r.cpu().numpy().view(np.uint16).tolist())
print(json.dumps(out))
""".replace("import ctypes as C, json, sys", "import ctypes as C, json, os, sys")


def test_noalloc_first_call_in_a_fresh_process_allocates_nothing():
    """In a fresh process: no-allocation calls (1 and 4 rows) and moa_device_errors leave only
    the static scratch set up (moa_test_scratch_state == 2: the hipMalloc'd scratch was never
    created), raise no device error, and give the allocating entry point's bits."""
    need_gpu()
    root = Path(__file__).resolve().parent.parent
    paths = os.pathsep.join(str(p) for p in (root, root / "moa-workspace_amd", root / "tests"))
    say("no-alloc fp8 ffn in a fresh process (M1, M4)")
    res = subprocess.run([sys.executable, "-c", CHILD, paths], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-3000:]
    child = json.loads(res.stdout.strip().splitlines()[-1])
    w = synth.cfg_ffn_fp8(12)
    d = {k: dev(v) for k, v in w.items() if k != "residual"}
    for M in (1, 4):
        c = child[str(M)]
        assert c["bits"] == 0, f"M{M}: device error bits {c['bits']:#x}"
        assert c["state"] == 2, f"M{M}: scratch state {c['state']} (1 = the hipMalloc'd scratch was created)"
        r = dev(synth.bf16_normal(f"noalloc.M{M}.residual", (M, 3840)))
        assert _call("moa_decoder_feedforward_fp8", d, r) == 0, _lib.load().moa_last_error_string()
        want = host(r).reshape(-1)
        got = np.array(c["residual"], np.uint16).reshape(-1)
        assert np.array_equal(got, want), f"M{M}: {np.count_nonzero(got != want)} elements differ"
