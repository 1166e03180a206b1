"""ctypes binding of libmoa_gfx950.so (declarations mirror include/moa_ops.h and include/moa_ckpt.h).

Loading fails loudly when the library is missing: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent.parent
LIB_PATH = Path(os.environ.get("MOA_LIB", PKG_ROOT / "libmoa_gfx950.so"))

MOA_SUCCESS = 0
ERRORS = {
    -1: "MOA_ERROR_INVALID_VALUE",
    -2: "MOA_ERROR_MISALIGNED",
    -3: "MOA_ERROR_HIP",
    -4: "MOA_ERROR_NO_DEVICE",
    -5: "MOA_ERROR_DEVICE_STATE",
    -6: "MOA_ERROR_NOT_FOUND",
    -7: "MOA_ERROR_FORMAT",
    -8: "MOA_ERROR_IO",
}
DEVERR_ROPE_OFFSET = 1
DEVERR_KV_OFFSET = 2
DEVERR_SPIN_TIMEOUT = 4


class MoaError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"{ERRORS.get(code, code)}: {message}")
        self.code = code


P, I32, U32P = C.c_void_p, C.c_int, C.POINTER(C.c_uint32)
S, I64, U64 = C.c_char_p, C.c_int64, C.c_uint64

# name -> argtypes (restype is int unless listed in _RESTYPES)
SIGNATURES = {
    "moa_version": [],
    "moa_last_error_string": [],
    "moa_init": [I32],
    # include/moa_ckpt.h
    "moa_ckpt_open": [S, C.POINTER(P)],
    "moa_ckpt_close": [P],
    "moa_ckpt_count": [P, C.POINTER(C.c_int)],
    "moa_ckpt_name": [P, I32, C.POINTER(S)],
    "moa_ckpt_info": [P, S, C.POINTER(S), C.POINTER(I64), C.POINTER(C.c_int), C.POINTER(U64)],
    "moa_ckpt_read": [P, S, P, U64],
    "moa_ckpt_load_bf16": [P, S, C.POINTER(I64), I32, P, P],
    "moa_ckpt_load_bf16_column": [P, S, I64, P, P],
    "moa_ckpt_load_f8": [P, S, I64, I64, P, P],
    "moa_ckpt_load_f4": [P, S, I64, I64, P, P],
    "moa_ckpt_load_scalar_bf16": [P, S, P, P],
    "moa_ckpt_global_scale": [P, S, C.POINTER(C.c_float)],
    "moa_ckpt_load_global_scale": [P, S, P, P],
    "moa_device_errors": [P, U32P],
    "moa_sliding_project_qkv": [P] * 17 + [I32, P],
    "moa_sliding_project_qkv_bf16_scales": [P] * 17 + [I32, P],
    "moa_sliding_attention": [P] * 5 + [I32, P],
    "moa_final_norm_and_logits": [P] * 4 + [I32, P],
    "moa_full_project_qkv": [P] * 15 + [I32, P],
    "moa_full_attention_first_page": [P] * 7 + [I32, P],
    "moa_full_attention_page": [P] * 7 + [I32, P],
    "moa_full_attention_output": [P] * 6 + [I32, P],
    "moa_full_attention": [P] * 4 + [I32] + [P] * 3 + [I32, P],
    "moa_sliding_attention_output": [P] * 5 + [I32, P],
    "moa_sliding_attention_output_bf16_scales": [P] * 5 + [I32, P],
    "moa_decoder_feedforward": [P] * 13 + [I32, P],
    "moa_decoder_feedforward_fp8": [P] * 10 + [I32, P],
    "moa_decoder_feedforward_mxfp4": [P] * 10 + [I32, P],
    "moa_decoder_feedforward_fp8_noalloc": [P] * 10 + [I32, P],
    "moa_sliding_attention_output_feedforward": [P] * 17 + [I32, P],
    "moa_sliding_attention_output_feedforward_fp8": [P] * 14 + [I32, P],
    "moa_sliding_attention_output_feedforward_mxfp4": [P] * 14 + [I32, P],
    "moa_fp8_scaled_projection": [P] * 4 + [I32, I32, I32, P],
    "moa_format_selftest": [P, P],
    "moa_test_epoch_layout": [I32, C.POINTER(C.c_int), C.POINTER(C.c_int)],
    "moa_test_epoch_tag": [I32, U64, U32P],
    "moa_test_preset_epochs": [U64],
    "moa_test_set_stall": [C.c_uint32, C.c_uint32, C.POINTER(C.c_int32)],
    "moa_test_take_overs": [U32P],
    "moa_test_set_rows_one_launch": [C.c_int],
    "moa_test_scratch_state": [U32P],
    "moa_test_trip_device_state": [I32],
    "moa_clear_device_state": [I32],
    # include/moa_bench.h
    "moa_bench_stream_read": [P, U64, I32, I32, P, P],
}
_RESTYPES = {"moa_version": C.c_char_p, "moa_last_error_string": C.c_char_p}

_lib: C.CDLL | None = None


def load() -> C.CDLL:
    """Load and declare the library (once). Raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise MoaError(-4, f"{LIB_PATH} is not built; run `python moa-workspace_amd/build.py`")
    lib = C.CDLL(str(LIB_PATH))
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPES.get(name, C.c_int)
    _lib = lib
    return lib


def check(code: int) -> None:
    if code != MOA_SUCCESS:
        raise MoaError(code, load().moa_last_error_string().decode())


_fns: dict = {}


def call(name: str, *args) -> None:
    fn = _fns.get(name)
    if fn is None:
        fn = _fns[name] = getattr(load(), name)
    check(fn(*args))
