"""The C ABI library: loads, exports every symbol include/*.h declares, and rejects bad
arguments on the host before touching a device (no compute calls here)."""
import ctypes as C
import re
from pathlib import Path

import pytest

from moa_amd import _lib

ROOT = Path(__file__).resolve().parent.parent


def header_functions():
    names = set()
    for h in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(moa_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_library_builds_and_loads():
    assert _lib.LIB_PATH.exists(), "run `python moa-workspace_amd/build.py` (or __graft_entry__.build())"
    lib = _lib.load()
    assert lib.moa_version().decode().startswith("moa-gfx950")


def test_every_declared_symbol_is_exported_and_bound():
    lib = _lib.load()
    names = header_functions()
    assert len(names) >= 12
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(_lib.SIGNATURES) == names


def _null(n):
    return [None] * n


@pytest.mark.parametrize("fn,nptr,tail", [
    ("moa_sliding_project_qkv", 17, (1, None)),
    ("moa_sliding_attention_output", 5, (1, None)),
    ("moa_decoder_feedforward", 13, (1, None)),
    ("moa_decoder_feedforward_fp8", 10, (1, None)),
    ("moa_decoder_feedforward_mxfp4", 10, (1, None)),
    ("moa_decoder_feedforward_fp8_noalloc", 10, (1, None)),
    ("moa_sliding_attention", 5, (1, None)),
    ("moa_final_norm_and_logits", 4, (1, None)),
    ("moa_full_project_qkv", 15, (1, None)),
    ("moa_full_attention_first_page", 7, (1, None)),
    ("moa_full_attention_page", 7, (1, None)),
    ("moa_full_attention_output", 6, (1, None)),
    ("moa_sliding_attention_output_feedforward", 17, (1, None)),
    ("moa_sliding_attention_output_feedforward_fp8", 14, (1, None)),
    ("moa_sliding_attention_output_feedforward_mxfp4", 14, (1, None)),
])
def test_null_pointers_rejected_on_host(fn, nptr, tail):
    lib = _lib.load()
    rc = getattr(lib, fn)(*_null(nptr), *tail)
    assert rc == -1
    assert b"NULL" in lib.moa_last_error_string()


def test_misaligned_and_bad_rows_rejected_on_host():
    lib = _lib.load()
    buf = (C.c_uint8 * 4096)()
    base = (C.addressof(buf) + 15) // 16 * 16
    ok = C.c_void_p(base)
    bad = C.c_void_p(base + 2)
    # residual misaligned
    rc = lib.moa_sliding_attention_output(ok, ok, ok, ok, bad, 1, None)
    assert rc == -2 and b"residual" in lib.moa_last_error_string()
    # M out of range
    rc = lib.moa_sliding_attention_output(ok, ok, ok, ok, ok, 0, None)
    assert rc == -1 and b"M must be" in lib.moa_last_error_string()
    # projection shape check
    rc = lib.moa_fp8_scaled_projection(ok, ok, ok, ok, 1, 8, 12, None)
    assert rc == -1 and b"multiple of 16" in lib.moa_last_error_string()
    # NVFP4 needs its global scales; FP8 accepts NULL post-norm / layer scalar but not NULL scales
    rc = lib.moa_decoder_feedforward(*([ok] * 8), None, ok, ok, ok, ok, 1, None)
    assert rc == -1 and b"up_global_scale" in lib.moa_last_error_string()
    rc = lib.moa_decoder_feedforward_fp8(*([ok] * 5), None, ok, ok, None, None, 1, None)
    assert rc == -1 and b"up_weight_scale" in lib.moa_last_error_string()


def test_next_row_entry_points_check_alignment_and_sizes_on_host():
    lib = _lib.load()
    buf = (C.c_uint8 * 4096)()
    base = (C.addressof(buf) + 15) // 16 * 16
    ok, bad2, bad4 = C.c_void_p(base), C.c_void_p(base + 2), C.c_void_p(base + 4)
    # full attention: the page count must lie in [1, 64]
    for P in (0, 65):
        rc = lib.moa_full_attention(ok, ok, ok, ok, P, ok, ok, ok, 1, None)
        assert rc == -1 and b"P must be" in lib.moa_last_error_string()
    rc = lib.moa_full_attention(None, ok, ok, ok, 2, ok, ok, ok, 1, None)
    assert rc == -1 and b"q is NULL" in lib.moa_last_error_string()
    # 4-byte-aligned f32 state is enough; 16-byte tensors are not
    rc = lib.moa_full_attention_page(ok, ok, ok, ok, bad2, ok, ok, 1, None)
    assert rc == -2 and b"running_max" in lib.moa_last_error_string()
    rc = lib.moa_full_attention_page(ok, ok, bad4, ok, ok, ok, ok, 1, None)
    assert rc == -2 and b"v " in lib.moa_last_error_string()
    rc = lib.moa_sliding_attention(ok, ok, ok, bad2, ok, 1, None)
    assert rc == -2 and b"mask" in lib.moa_last_error_string()
    rc = lib.moa_final_norm_and_logits(ok, ok, ok, ok, 0, None)
    assert rc == -1 and b"M must be" in lib.moa_last_error_string()
    # 2-byte-aligned bf16 scales pass the host checks; a 2-byte-aligned cos table does not
    rc = lib.moa_full_project_qkv(*([ok] * 3), bad2, ok, *([ok] * 5), bad2, *([ok] * 4), 1, None)
    assert rc == -2 and b"cos" in lib.moa_last_error_string()
    rc = lib.moa_full_attention_output(ok, bad2, ok, ok, ok, ok, 1, None)
    assert rc == -2 and b"running_sum" in lib.moa_last_error_string()


def test_python_front_end_rejects_host_tensors():
    torch = pytest.importorskip("torch")
    from moa_amd import ops
    x = torch.zeros(4096, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="ROCm device"):
        ops.sliding_attention_output(x, x[:3840], torch.zeros(3840 * 4096, dtype=torch.uint8),
                                     torch.zeros(3840), x[:3840].clone())
