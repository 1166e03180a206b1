"""The checkpoint reader (include/moa_ckpt.h; moa_amd/checkpoint.py) on the CPU.

Files are written by the `safetensors` package itself, an implementation independent of the
reader: the header the reader parses (dtypes, shapes, offsets, escaped names, metadata) and the
bytes it returns must match what that writer stored. Malformed files are built by hand. The checks
of dtype and shape (load.rs:93-190) run before any device call, so their errors are testable here
with a dummy destination; copies to the device are tested on the GPU."""
import ctypes as C
import math
import struct

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from moa_amd import _lib, checkpoint

NOT_FOUND, FORMAT, IO, INVALID = -6, -7, -8, -1


def tensors():
    g = torch.Generator().manual_seed(0)
    return {
        "model.language_model.norm.weight": torch.randn(3840, generator=g).to(torch.bfloat16),
        "w.fp8": torch.randint(0, 0x7f, (64, 96), generator=g, dtype=torch.uint8).view(torch.float8_e4m3fn),
        "w.scale": torch.rand(64, 1, generator=g).to(torch.bfloat16),
        "w.packed": torch.randint(0, 256, (32, 48), generator=g, dtype=torch.uint8),
        "w.global": torch.tensor([448.0 * 6.0 / 3.5], dtype=torch.float32),
        "w.global_shaped": torch.tensor(2.0, dtype=torch.float32),
        "w.zero_global": torch.tensor([0.0], dtype=torch.float32),
        "w.inf_global": torch.tensor([math.inf], dtype=torch.float32),
        "w.two_globals": torch.tensor([1.0, 2.0], dtype=torch.float32),
        "layer_scalar": torch.tensor([0.375], dtype=torch.bfloat16),
        'name with "quotes", \\ and é': torch.arange(6, dtype=torch.int32).reshape(2, 3),
        "empty": torch.zeros(0, 4, dtype=torch.bfloat16),
    }


@pytest.fixture()
def ckfile(tmp_path):
    t = tensors()
    p = tmp_path / "model.safetensors"
    save_file(t, str(p), metadata={"format": "pt", "note": 'a "quoted" value'})
    return p, t


def raw(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().reshape(-1).view(torch.uint8).numpy() if t.numel() else np.zeros(0, np.uint8)


def test_header_and_bytes_match_the_writer(ckfile):
    p, t = ckfile
    with checkpoint.Checkpoint(p) as ck:
        assert sorted(ck.names()) == sorted(t)
        want_dtype = {torch.bfloat16: "BF16", torch.float8_e4m3fn: "F8_E4M3", torch.uint8: "U8",
                      torch.float32: "F32", torch.int32: "I32"}
        for name, v in t.items():
            dt, shape, nb = ck.info(name)
            assert dt == want_dtype[v.dtype], name
            assert shape == tuple(v.shape), name
            assert nb == v.numel() * v.element_size(), name
            assert np.array_equal(ck.read(name), raw(v)), name


def test_global_scale_is_the_reciprocal_and_bad_values_are_rejected(ckfile):
    p, t = ckfile
    with checkpoint.Checkpoint(p) as ck:
        assert ck.global_scale("w.global") == np.float32(1.0) / np.float32(t["w.global"].item())
        assert ck.global_scale("w.global_shaped") == 0.5  # read_f32 takes any one-value shape
        for name, code in (("w.zero_global", FORMAT), ("w.inf_global", FORMAT), ("w.two_globals", FORMAT),
                           ("w.scale", FORMAT), ("absent", NOT_FOUND)):
            with pytest.raises(_lib.MoaError) as e:
                ck.global_scale(name)
            assert e.value.code == code, name


def _lib_call(name, *args):
    lib = _lib.load()
    return getattr(lib, name)(*args), lib.moa_last_error_string().decode()


@pytest.mark.parametrize("fn,name,args,code,needle", [
    ("moa_ckpt_load_f8", b"w.fp8", (64, 96), 0, None),
    ("moa_ckpt_load_f8", b"w.fp8", (96, 64), FORMAT, "expected F8_E4M3 [96, 64]"),
    ("moa_ckpt_load_f8", b"w.packed", (32, 48), FORMAT, "is U8 [32, 48]"),
    ("moa_ckpt_load_f8", b"nope", (1, 1), NOT_FOUND, "not in"),
    ("moa_ckpt_load_f4", b"w.packed", (32, 96), 0, None),
    ("moa_ckpt_load_f4", b"w.packed", (32, 48), FORMAT, "expected U8 [32, 24]"),
    ("moa_ckpt_load_f4", b"w.packed", (32, 97), INVALID, "even"),
    ("moa_ckpt_load_bf16_column", b"w.scale", (64,), 0, None),
    ("moa_ckpt_load_bf16_column", b"w.scale", (65,), FORMAT, "expected BF16 [65, 1]"),
    ("moa_ckpt_load_bf16_column", b"model.language_model.norm.weight", (3840,), FORMAT, "BF16 [3840]"),
    ("moa_ckpt_load_scalar_bf16", b"layer_scalar", (), 0, None),
    ("moa_ckpt_load_scalar_bf16", b"w.scale", (), FORMAT, "expected BF16 [1]"),
])
def test_typed_loaders_check_dtype_and_shape_before_copying(ckfile, fn, name, args, code, needle):
    p, _ = ckfile
    with checkpoint.Checkpoint(p) as ck:
        # a null destination: a tensor that passes the checks stops at the copy (INVALID, no HIP call)
        rc, msg = _lib_call(fn, ck._h, name, *args, None, None)
        if code == 0:
            assert rc == INVALID and "null destination" in msg, msg
        else:
            assert rc == code, msg
            assert needle in msg, msg


def test_load_bf16_checks_the_full_shape(ckfile):
    p, _ = ckfile
    with checkpoint.Checkpoint(p) as ck:
        for shape, code in (((3840,), INVALID), ((1920, 2), FORMAT), ((3841,), FORMAT)):
            arr = (C.c_int64 * len(shape))(*shape)
            rc, msg = _lib_call("moa_ckpt_load_bf16", ck._h, b"model.language_model.norm.weight", arr, len(shape),
                                None, None)
            assert rc == code, (shape, msg)


def _file(header: bytes, data: bytes = b"", length: int | None = None) -> bytes:
    n = len(header) if length is None else length
    return struct.pack("<Q", n) + header + data


def _entry(dtype="U8", shape=(4,), offsets=(0, 4)):
    return ('{"t":{"dtype":"%s","shape":[%s],"data_offsets":[%d,%d]}}'
            % (dtype, ",".join(map(str, shape)), *offsets)).encode()


@pytest.mark.parametrize("blob,needle", [
    (b"\x01\x00", "shorter than"),
    (_file(b"{}", length=1 << 40), "too large"),
    (_file(b"{}", length=100), "past the end"),
    (_file(b"[]"), "not a JSON object"),
    (_file(b'{"t":{"dtype":"U8","shape":[4]}}', b"abcd"), "lacks"),
    (_file(_entry(offsets=(0, 8)), b"abcd"), "outside the data section"),
    (_file(_entry(offsets=(3, 2)), b"abcd"), "outside the data section"),
    (_file(_entry(shape=(3,)), b"abcd"), "does not match"),
    (_file(_entry(dtype="BF16", shape=(3,)), b"abcd"), "does not match"),
    (_file(b'{"t":{"dtype":"U8","shape":[-4],"data_offsets":[0,4]}}', b"abcd"), "non-negative integer"),
    (_file(b'{"t":{"dtype":"U8","shape":[4],"data_offsets":[0,4]},"t":{"dtype":"U8","shape":[4],'
           b'"data_offsets":[0,4]}}', b"abcd"), "appears twice"),
    (_file(_entry() + b"x", b"abcd"), "trailing bytes"),
    (_file(b'{"t":{"dtype":"U8","shape":[4],"data_offsets":[0,4]}', b"abcd"), "expected ',' or '}'"),
    (_file(b'{"t\\q":{"dtype":"U8","shape":[4],"data_offsets":[0,4]}}', b"abcd"), "bad escape"),
    (_file(b'{"t\xc3":{"dtype":"U8","shape":[4],"data_offsets":[0,4]}}', b"abcd"), "not valid UTF-8"),
    (_file(b'{"t\xed\xa0\x80":{"dtype":"U8","shape":[4],"data_offsets":[0,4]}}', b"abcd"), "not valid UTF-8"),
])
def test_malformed_files_are_rejected(tmp_path, blob, needle):
    p = tmp_path / "bad.safetensors"
    p.write_bytes(blob)
    with pytest.raises(_lib.MoaError) as e:
        checkpoint.Checkpoint(p)
    assert e.value.code == FORMAT
    assert needle in str(e.value), str(e.value)


def test_header_padding_unknown_fields_and_dtypes_are_accepted(tmp_path):
    hdr = (b'{"__metadata__":{"k":"v"},"t":{"dtype":"U8","shape":[2,2],"data_offsets":[0,4],"extra":[1,{"a":null}]},'
           b'"u":{"dtype":"F4","shape":[8],"data_offsets":[4,8]}}    ')
    p = tmp_path / "ok.safetensors"
    p.write_bytes(_file(hdr, b"abcdefgh"))
    with checkpoint.Checkpoint(p) as ck:
        assert ck.names() == ["t", "u"]
        assert ck.info("t") == ("U8", (2, 2), 4)
        assert bytes(ck.read("t")) == b"abcd"
        assert ck.info("u") == ("F4", (8,), 4)  # an unsized dtype is listed, not size-checked


def test_every_truncation_of_a_valid_file_is_rejected_cleanly(ckfile, tmp_path):
    p, _ = ckfile
    blob = p.read_bytes()
    n = struct.unpack("<Q", blob[:8])[0]
    q = tmp_path / "cut.safetensors"
    for cut in sorted({0, 4, 7, 8, 9, 8 + n // 2, 8 + n - 1, 8 + n, len(blob) - 1}):
        q.write_bytes(blob[:cut])
        with pytest.raises(_lib.MoaError) as e:
            checkpoint.Checkpoint(q)
        assert e.value.code == FORMAT, cut


def test_missing_file_is_an_io_error(tmp_path):
    with pytest.raises(_lib.MoaError) as e:
        checkpoint.Checkpoint(tmp_path / "absent.safetensors")
    assert e.value.code == IO


def test_model_dir_resolution(tmp_path, monkeypatch):
    monkeypatch.delenv("MOA_MODEL_DIR", raising=False)
    monkeypatch.delenv("RNGD_MODEL_DIR", raising=False)
    with pytest.raises(FileNotFoundError):
        checkpoint.model_dir()
    sub = tmp_path / "gemma-4-12b-it-NVFP4"
    sub.mkdir()
    (sub / "model.safetensors").write_bytes(b"")
    monkeypatch.setenv("RNGD_MODEL_DIR", str(tmp_path))
    assert checkpoint.model_dir() == sub
    (tmp_path / "model.safetensors").write_bytes(b"")
    monkeypatch.setenv("MOA_MODEL_DIR", str(tmp_path))
    assert checkpoint.model_dir() == tmp_path


def test_layer_pattern():
    full = [i for i in range(checkpoint.LAYERS) if checkpoint.is_full_layer(i)]
    assert full == [5, 11, 17, 23, 29, 35, 41, 47]


def test_mutated_headers_are_parsed_or_rejected_never_crash(ckfile, tmp_path):
    """Random byte flips, insertions and deletions in the JSON header of a valid file: every
    result is a clean open (the bytes still form a valid header) or MOA_ERROR_FORMAT."""
    p, _ = ckfile
    blob = p.read_bytes()
    n = struct.unpack("<Q", blob[:8])[0]
    header, data = bytearray(blob[8:8 + n]), blob[8 + n:]
    rng = np.random.default_rng(1234)
    q = tmp_path / "mut.safetensors"
    opened = rejected = 0
    for _ in range(300):
        h = bytearray(header)
        for _ in range(int(rng.integers(1, 4))):
            at = int(rng.integers(0, len(h)))
            kind = int(rng.integers(0, 3))
            if kind == 0:
                h[at] = int(rng.integers(0, 256))
            elif kind == 1:
                h.insert(at, int(rng.choice(list(b'{}[],:"\\\\0123456789 eE-.u'))))
            elif len(h) > 2:
                del h[at]
        q.write_bytes(struct.pack("<Q", len(h)) + bytes(h) + data)
        try:
            with checkpoint.Checkpoint(q) as ck:
                for name in ck.names():
                    dt, shape, nb = ck.info(name)
                    assert len(ck.read(name)) == nb
            opened += 1
        except _lib.MoaError as e:
            assert e.code == FORMAT, str(e)
            rejected += 1
    assert rejected > 100
