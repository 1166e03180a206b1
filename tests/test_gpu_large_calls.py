"""Calls longer than one MFMA-path chunk (1024 rows): the entry points run them as consecutive
chunks (`moa_api.hip` qkv_common / o_common / ffn_common). A 1030-row call is a 1024-row chunk and
a 6-row chunk. Its first 1024 rows must equal a separate 1024-row call bit for bit, and its last six
rows must match the oracle run on those rows alone (at their positions, for QKV)."""
import numpy as np
import pytest

from gpu_util import gate, need_gpu, say
from moa_amd import synth
from test_gpu_ffn import FFN_ATOL, gpu_fp8, oracle_fp8
from test_gpu_o import run_gpu as o_gpu
from test_gpu_o import run_oracle as o_oracle
from test_gpu_qkv import run_gpu as qkv_gpu
from test_gpu_qkv import run_oracle as qkv_oracle
from gpu_util import gate_rope

pytestmark = pytest.mark.gpu

M, HEAD = 1030, 1024  # rows of the call; rows of its first chunk


def split(d, keys, lo, hi):
    return dict(d, **{k: np.ascontiguousarray(d[k][lo:hi]) for k in keys})


def test_o_call_of_two_chunks():
    need_gpu()
    say(f"o M{M}: chunks of {HEAD} and {M - HEAD} rows")
    d = synth.cfg_o(21, M=M)
    got = o_gpu(d)
    assert np.array_equal(got[:HEAD], o_gpu(split(d, ("x", "residual"), 0, HEAD))), "first chunk differs"
    gate(o_oracle(split(d, ("x", "residual"), HEAD, M)), got[HEAD:], f"o M{M} last chunk")


def test_ffn_call_of_two_chunks():
    need_gpu()
    say(f"ffn fp8 M{M}: chunks of {HEAD} and {M - HEAD} rows")
    d = synth.cfg_ffn_fp8(21, M=M)
    got = gpu_fp8(d)
    assert np.array_equal(got[:HEAD], gpu_fp8(split(d, ("residual",), 0, HEAD))), "first chunk differs"
    gate(oracle_fp8(split(d, ("residual",), HEAD, M)), got[HEAD:], f"ffn M{M} last chunk", atol=FFN_ATOL)


def test_qkv_call_of_two_chunks():
    """Rows m and m + 1024 share a ring slot; the later row's K/V must be the one left there, as if
    the rows ran one after the other."""
    need_gpu()
    pos = 100
    say(f"qkv M{M} at position {pos}: chunks of {HEAD} and {M - HEAD} rows")
    d = synth.cfg_qkv(21, M=M, pos=pos)
    q, kc, vc = qkv_gpu(d, M)
    q = q.reshape(M, -1)
    # the first chunk alone
    qh, kh, vh = qkv_gpu(split(d, ("x",), 0, HEAD), HEAD)
    assert np.array_equal(q[:HEAD], qh.reshape(HEAD, -1)), "first chunk's q differs"
    tail_slots = [(pos + HEAD + m) % 1024 for m in range(M - HEAD)]
    keep = np.ones(1024, bool)
    keep[tail_slots] = False
    assert np.array_equal(kc[keep], kh[keep]) and np.array_equal(vc[keep], vh[keep]), \
        "slots not rewritten by the second chunk differ from the first chunk's"
    # the second chunk against the oracle at positions pos + 1024 ..
    t = split(d, ("x",), HEAD, M)
    t["rope_offset"] = (pos + HEAD) * 256 * 2
    qe, kce, vce = qkv_oracle(t, M - HEAD)
    gate_rope(qe, q[HEAD:].reshape(-1), f"qkv M{M} last chunk q", 256)
    gate_rope(kce[tail_slots], kc[tail_slots], f"qkv M{M} last chunk k", 256)
    gate(vce[tail_slots], vc[tail_slots], f"qkv M{M} last chunk v")
