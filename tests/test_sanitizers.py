"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

* The checkpoint reader parses untrusted files (moa_ckpt.hip: its own JSON reader over a mapped
  safetensors header). Its host code, built with ASan + UBSan (tests/sanitize/Makefile), runs over
  well-formed files written by the `safetensors` package and over mutations of them: every
  truncation of a small file, seeded byte flips in the header, bad header lengths, data offsets
  reversed / past the end / overlapping, deep nesting, long strings and escapes. Every file must be
  opened or rejected cleanly, with no sanitizer report.
* The C oracle (oracle/moa_oracle.c), built with ASan + UBSan, runs the CPU oracle tests (golden
  vectors, formats, PRNG) inside Python with the sanitizer runtime preloaded.
"""
import json
import os
import random
import shutil
import struct
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
SAN = ROOT / "tests" / "sanitize"
OUT = SAN / "_out"


@pytest.fixture(scope="module")
def built():
    if shutil.which("gcc") is None or not Path("/opt/rocm/bin/hipcc").exists():
        pytest.skip("needs gcc and hipcc")
    r = subprocess.run(["make", "-s", "-C", str(SAN)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    return OUT


def _header_file(path: Path, header: bytes, data: bytes, length: int | None = None) -> None:
    path.write_bytes(struct.pack("<Q", len(header) if length is None else length) + header + data)


def _corpus(d: Path) -> int:
    from safetensors.numpy import save_file
    rng = random.Random(7)
    good = []
    tensors = {
        "model.layers.0.mlp.up_proj.weight": np.arange(64, dtype=np.uint8).reshape(8, 8),
        "scale": np.array([2.5], np.float32),
        "zero_scale": np.array([0.0], np.float32),
        "bf16": np.arange(12, dtype=np.uint16).reshape(3, 4),
        'esc"aped\\nameé': np.zeros((2, 2), np.float32),
        "empty": np.zeros((0, 4), np.float32),
    }
    p = d / "good0.safetensors"
    save_file(tensors, str(p), metadata={"format": "pt", "note": "x" * 300})
    good.append(p.read_bytes())
    p = d / "good1.safetensors"
    save_file({"w": np.ones((4, 16), np.uint8)}, str(p))
    good.append(p.read_bytes())
    n = len(good)
    for gi, raw in enumerate(good):
        hlen = struct.unpack("<Q", raw[:8])[0]
        # every truncation of the file up to the end of the header, then some of the data
        for cut in list(range(0, 8 + hlen + 1)) + list(range(8 + hlen + 1, len(raw), 7)):
            (d / f"trunc{gi}_{cut}.safetensors").write_bytes(raw[:cut]); n += 1
        # seeded byte flips inside the header
        for k in range(300):
            b = bytearray(raw)
            for _ in range(rng.randint(1, 4)):
                b[8 + rng.randrange(hlen)] = rng.randrange(256)
            (d / f"flip{gi}_{k}.safetensors").write_bytes(bytes(b)); n += 1
        # wrong header lengths
        for L in (0, 1, hlen - 1, hlen + 1, len(raw), 2**31, 2**63, 2**64 - 1):
            _header_file(d / f"len{gi}_{L}.safetensors", raw[8:8 + hlen], raw[8 + hlen:], L); n += 1
    body = bytes(64)
    cases = {
        "reversed": {"t": {"dtype": "U8", "shape": [8], "data_offsets": [8, 0]}},
        "past_end": {"t": {"dtype": "U8", "shape": [80], "data_offsets": [0, 80]}},
        "size_mismatch": {"t": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}},
        "huge_shape": {"t": {"dtype": "F32", "shape": [2**62, 4], "data_offsets": [0, 16]}},
        "neg_shape": {"t": {"dtype": "U8", "shape": [-8], "data_offsets": [0, 8]}},
        "float_shape": {"t": {"dtype": "U8", "shape": [8.0], "data_offsets": [0, 8]}},
        "exp_number": {"t": {"dtype": "U8", "shape": [8], "data_offsets": [0, 8e0]}},
        "many_dims": {"t": {"dtype": "U8", "shape": [1] * 40, "data_offsets": [0, 1]}},
        "unknown_dtype": {"t": {"dtype": "Q7", "shape": [8], "data_offsets": [0, 8]}},
        "overlap": {"a": {"dtype": "U8", "shape": [16], "data_offsets": [0, 16]},
                    "b": {"dtype": "U8", "shape": [16], "data_offsets": [8, 24]}},
        "not_object": [1, 2, 3],
        "missing_offsets": {"t": {"dtype": "U8", "shape": [8]}},
    }
    for name, obj in cases.items():
        _header_file(d / f"case_{name}.safetensors", json.dumps(obj).encode(), body); n += 1
    raw_cases = {
        "deep": b'{"__metadata__":' + b"[" * 5000 + b"]" * 5000 + b"}",
        "deep_obj": b'{"__metadata__":' + b'{"a":' * 3000 + b"1" + b"}" * 3000 + b"}",
        "long_string": b'{"' + b"a" * 200000 + b'":{"dtype":"U8","shape":[1],"data_offsets":[0,1]}}',
        "bad_escape": b'{"\\q":{"dtype":"U8","shape":[1],"data_offsets":[0,1]}}',
        "surrogate": b'{"\\ud800\\udc00\\ud800":{"dtype":"U8","shape":[1],"data_offsets":[0,1]}}',
        "short_unicode": b'{"\\u12":{"dtype":"U8","shape":[1],"data_offsets":[0,1]}}',
        "nul_in_key": b'{"a\x00b":{"dtype":"U8","shape":[1],"data_offsets":[0,1]}}',
        "trailing": b'{"t":{"dtype":"U8","shape":[1],"data_offsets":[0,1]}} x',
        "duplicate": b'{"t":{"dtype":"U8","shape":[1],"data_offsets":[0,1]},"t":{"dtype":"U8","shape":[1],"data_offsets":[0,1]}}',
        "unterminated": b'{"t":{"dtype":"U8","shape":[1],"data_offsets":[0,1',
        "big_int": b'{"t":{"dtype":"U8","shape":[99999999999999999999999],"data_offsets":[0,1]}}',
    }
    for name, hdr in raw_cases.items():
        _header_file(d / f"raw_{name}.safetensors", hdr, body); n += 1
    (d / "empty.safetensors").write_bytes(b""); n += 1
    return n


def test_checkpoint_reader_under_asan_and_ubsan(built, tmp_path):
    n = _corpus(tmp_path)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([str(built / "ckpt_fuzz"), str(tmp_path)], capture_output=True, text=True, env=env,
                       timeout=600)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "runtime error" not in out and "AddressSanitizer" not in out, out[-4000:]
    assert f"files {n} " in out, out
    print(out.strip().splitlines()[-1])


def test_oracle_under_asan_and_ubsan(built):
    asan = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    ubsan = subprocess.run(["gcc", "-print-file-name=libubsan.so"], capture_output=True, text=True).stdout.strip()
    env = dict(os.environ, LD_PRELOAD=f"{asan}:{ubsan}", ORACLE_LIB=str(built / "liboracle_asan.so"),
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1", UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
               OMP_NUM_THREADS="4")
    tests = [str(ROOT / "tests" / t) for t in ("test_oracle_golden.py", "test_formats.py", "test_prng.py")]
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider", *tests],
                       capture_output=True, text=True, env=env, timeout=1500, cwd=str(ROOT))
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "runtime error" not in out and "AddressSanitizer" not in out, out[-4000:]
