"""ctypes front-end to oracle/liboracle.so -- the CPU restatement of the reference.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker. The product path (moa-workspace_amd/) never imports it.

All bf16 tensors are numpy uint16 arrays of raw bits; E4M3/E2M1/E8M0 are uint8 codes.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# ORACLE_LIB names another build of the same source (tests/test_sanitizers.py: the ASan/UBSan one)
LIB_PATH = Path(os.environ["ORACLE_LIB"]) if os.environ.get("ORACLE_LIB") else HERE / "liboracle.so"

H, L, NS, GS, DS, QS, PS, TS, E, W = 3840, 15360, 8, 2, 256, 4096, 2048, 1024, 32768, 262144
FFN_NVFP4, FFN_FP8, FFN_MXFP4 = 0, 1, 2

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = C.CDLL(str(LIB_PATH))
        _declare(_lib)
    return _lib


P = C.c_void_p


def _declare(l: C.CDLL) -> None:
    l.orc_bf16_rne.restype = C.c_uint16
    l.orc_bf16_rne.argtypes = [C.c_float]
    l.orc_e4m3_decode.restype = C.c_float
    l.orc_e4m3_decode.argtypes = [C.c_uint8]
    l.orc_e4m3_encode_rne.restype = C.c_uint8
    l.orc_e4m3_encode_rne.argtypes = [C.c_float]
    l.orc_e2m1_decode.restype = C.c_float
    l.orc_e2m1_decode.argtypes = [C.c_uint8]
    l.orc_e2m1_encode_rne.restype = C.c_uint8
    l.orc_e2m1_encode_rne.argtypes = [C.c_float]
    l.orc_e8m0_decode.restype = C.c_float
    l.orc_e8m0_decode.argtypes = [C.c_uint8]
    l.orc_name_hash.restype = C.c_uint64
    l.orc_name_hash.argtypes = [C.c_char_p]
    l.orc_word.restype = C.c_uint64
    l.orc_word.argtypes = [C.c_uint64, C.c_uint64]
    l.orc_bf16_uniform.argtypes = [C.c_char_p, C.c_size_t, C.c_float, C.c_float, P]
    l.orc_f32_uniform.argtypes = [C.c_char_p, C.c_size_t, C.c_float, C.c_float, P]
    l.orc_bf16_signs.argtypes = [C.c_char_p, C.c_size_t, C.c_float, P]
    l.orc_f8_banded.argtypes = [C.c_char_p, C.c_size_t, C.c_int, C.c_int, C.c_int, P]
    l.orc_f4_nibbles.argtypes = [C.c_char_p, C.c_size_t, P]
    l.orc_checksum.restype = C.c_uint32
    l.orc_checksum.argtypes = [P, C.c_size_t]
    l.orc_run_pos.restype = C.c_int
    l.orc_run_pos.argtypes = [C.c_int]
    l.orc_rope_row.argtypes = [C.c_int, C.c_double, C.c_double, C.c_int, P, P]
    l.orc_rmsnorm_row.argtypes = [P, P, C.c_int, P]
    l.orc_gelu_tanh.restype = C.c_float
    l.orc_gelu_tanh.argtypes = [C.c_float]
    l.orc_scaled_projection_fp8.argtypes = [P, C.c_int, C.c_int, P, P, C.c_int, P]
    l.orc_sliding_project_qkv.argtypes = [P] * 10 + [C.c_int32, C.c_int32] + [P] * 5 + [C.c_int]
    l.orc_sliding_attention_output.argtypes = [P, P, P, P, P, C.c_int]
    l.orc_sliding_attention.argtypes = [P, P, P, P, P, C.c_int]
    l.orc_full_project_qkv.argtypes = [P] * 8 + [C.c_int32, C.c_int32] + [P] * 5 + [C.c_int]
    l.orc_full_attention_pages.argtypes = [P, P, P, P, C.c_int, P, P, P, C.c_int]
    l.orc_full_attention_output.argtypes = [P] * 6 + [C.c_int]
    l.orc_softcap30.argtypes = [C.c_uint16]
    l.orc_softcap30.restype = C.c_uint16
    l.orc_final_norm_and_logits.argtypes = [P, P, P, C.c_int, P, C.c_int]
    l.orc_decoder_feedforward.argtypes = [P, P, P, P, P, C.c_int]
    l.orc_ffn_up_gate.argtypes = [P, P, P, C.c_int]
    l.orc_ffn_down.argtypes = [P, P, P, C.c_int]
    l.orc_set_threads.restype = C.c_int
    l.orc_set_threads.argtypes = [C.c_int]


class FfnWeights(C.Structure):
    _fields_ = [("format", C.c_int), ("up", P), ("gate", P), ("down", P),
                ("up_scale", P), ("gate_scale", P), ("down_scale", P),
                ("up_inv_global", C.c_float), ("gate_inv_global", C.c_float),
                ("down_inv_global", C.c_float)]


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle inputs must be C-contiguous"
    return a.ctypes.data


def _u16(a) -> np.ndarray:
    a = np.ascontiguousarray(a)
    assert a.dtype == np.uint16, a.dtype
    return a


# ---------------------------------------------------------------- formats

def bf16_rne(values) -> np.ndarray:
    """Vectorised twin of orc_bf16_rne for numpy arrays (f32 -> bf16 bits)."""
    b = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32)
    out = ((b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    nan = (b & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    out[nan] = 0x7FC0
    return out


def bf16_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def e4m3_table() -> np.ndarray:
    l = lib()
    return np.array([l.orc_e4m3_decode(i) for i in range(256)], dtype=np.float32)


def e2m1_table() -> np.ndarray:
    l = lib()
    return np.array([l.orc_e2m1_decode(i) for i in range(16)], dtype=np.float32)


# ------------------------------------------------------------------- PRNG

def name_hash(name: str) -> int:
    return int(lib().orc_name_hash(name.encode()))


def word(seed: int, index: int) -> int:
    return int(lib().orc_word(seed, index))


def bf16_uniform(name: str, count: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(count, np.uint16)
    lib().orc_bf16_uniform(name.encode(), count, lo, hi, _p(out))
    return out


def f32_uniform(name: str, count: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(count, np.float32)
    lib().orc_f32_uniform(name.encode(), count, lo, hi, _p(out))
    return out


def bf16_signs(name: str, count: int, scale: float = 1.0) -> np.ndarray:
    out = np.empty(count, np.uint16)
    lib().orc_bf16_signs(name.encode(), count, scale, _p(out))
    return out


def f8_banded(name: str, count: int, exp_min: int, exp_max: int, signed: bool = True) -> np.ndarray:
    out = np.empty(count, np.uint8)
    lib().orc_f8_banded(name.encode(), count, exp_min, exp_max, int(signed), _p(out))
    return out


def f4_nibbles(name: str, count: int) -> np.ndarray:
    assert count % 2 == 0
    out = np.empty(count // 2, np.uint8)
    lib().orc_f4_nibbles(name.encode(), count, _p(out))
    return out


def checksum(data: np.ndarray) -> int:
    data = np.ascontiguousarray(data)
    return int(lib().orc_checksum(_p(data), data.nbytes))


def run_pos(run: int) -> int:
    return int(lib().orc_run_pos(run))


def rope_row(head_dim: int, theta: float, factor: float, pos: int):
    c = np.empty(head_dim, np.float32)
    s = np.empty(head_dim, np.float32)
    lib().orc_rope_row(head_dim, theta, factor, pos, _p(c), _p(s))
    return c, s


# -------------------------------------------------------------------- ops

def rmsnorm(x: np.ndarray, w: np.ndarray | None) -> np.ndarray:
    x = _u16(x)
    n = x.shape[-1]
    out = np.empty_like(x)
    xr, orr = x.reshape(-1, n), out.reshape(-1, n)
    for r in range(xr.shape[0]):
        lib().orc_rmsnorm_row(_p(xr[r]), _p(None if w is None else _u16(w)), n, _p(orr[r]))
    return out


def gelu_tanh(x: float) -> float:
    return float(lib().orc_gelu_tanh(x))


def scaled_projection_fp8(x: np.ndarray, w: np.ndarray, scale: np.ndarray) -> np.ndarray:
    x = _u16(x).reshape(-1, x.shape[-1])
    M, K = x.shape
    N = w.shape[0]
    assert w.shape == (N, K) and w.dtype == np.uint8
    scale = np.ascontiguousarray(scale, dtype=np.float32)
    out = np.empty((M, N), np.uint16)
    lib().orc_scaled_projection_fp8(_p(x), M, K, _p(np.ascontiguousarray(w)), _p(scale), N, _p(out))
    return out


def sliding_project_qkv(x, q_w, k_w, v_w, q_s, k_s, v_s, in_rms, q_rms, k_rms, kv_offset,
                        rope_offset, cos, sin, k_cache, v_cache, q_out):
    """ops::sliding_project_qkv (FO/src/ops.rs:37-76). Updates k_cache/v_cache/q_out in place."""
    x = _u16(x).reshape(-1, H)
    M = x.shape[0]
    f = lambda s: np.ascontiguousarray(s, dtype=np.float32)
    for a in (k_cache, v_cache, q_out):
        assert a.dtype == np.uint16 and a.flags["C_CONTIGUOUS"]
    lib().orc_sliding_project_qkv(_p(x), _p(q_w), _p(k_w), _p(v_w), _p(f(q_s)), _p(f(k_s)), _p(f(v_s)),
                                  _p(_u16(in_rms)), _p(_u16(q_rms)), _p(_u16(k_rms)), int(kv_offset),
                                  int(rope_offset), _p(_u16(cos)), _p(_u16(sin)), _p(k_cache),
                                  _p(v_cache), _p(q_out), M)


def sliding_attention_output(x, post_rms, o_w, o_s, residual):
    """ops::sliding_attention_output (FO/src/ops.rs:130-146). Updates residual in place."""
    x = _u16(x).reshape(-1, QS)
    assert residual.dtype == np.uint16 and residual.flags["C_CONTIGUOUS"]
    lib().orc_sliding_attention_output(_p(x), _p(_u16(post_rms)), _p(np.ascontiguousarray(o_w)),
                                       _p(np.ascontiguousarray(o_s, dtype=np.float32)), _p(residual),
                                       x.shape[0])


def sliding_attention(q, k, v, mask):
    """ops::sliding_attention (FO/src/ops.rs:118-128). Returns out bf16 bits [M, 8, 2, 256]."""
    q = _u16(q).reshape(-1, QS)
    M = q.shape[0]
    mask = np.ascontiguousarray(mask, dtype=np.float32).reshape(M, TS)
    out = np.zeros((M, QS), np.uint16)
    lib().orc_sliding_attention(_p(q), _p(_u16(k)), _p(_u16(v)), _p(mask), _p(out), M)
    return out.reshape(M, NS, GS, DS)


GF, DF, QF, TF = 16, 512, 8192, 512


def full_project_qkv(x, q_w, k_w, q_s, k_s, in_rms, q_rms, k_rms, kv_offset, rope_offset, cos, sin,
                     k_page, v_page, q_out):
    """ops::full_project_qkv (FO/src/ops.rs:78-116). Updates k_page / v_page / q_out in place."""
    x = _u16(x).reshape(-1, H)
    f = lambda s: np.ascontiguousarray(s, dtype=np.float32)
    for a in (k_page, v_page, q_out):
        assert a.dtype == np.uint16 and a.flags["C_CONTIGUOUS"]
    lib().orc_full_project_qkv(_p(x), _p(np.ascontiguousarray(q_w)), _p(np.ascontiguousarray(k_w)), _p(f(q_s)),
                               _p(f(k_s)), _p(_u16(in_rms)), _p(_u16(q_rms)), _p(_u16(k_rms)), int(kv_offset),
                               int(rope_offset), _p(_u16(cos)), _p(_u16(sin)), _p(k_page), _p(v_page), _p(q_out),
                               x.shape[0])


def full_attention_pages(q, k_pages, v_pages, masks):
    """The state after full_attention_first_page + full_attention_page over the given pages
    (FO/src/ops.rs:148-174). k_pages / v_pages [P, 512, 512] bf16; masks [P, M, 512] f32.
    Returns (running_max [M, 16] f32, running_sum [M, 16] f32, out [M, 16, 512] bf16 bits)."""
    q = _u16(q).reshape(-1, QF)
    M = q.shape[0]
    k_pages = _u16(k_pages).reshape(-1, TF, DF)
    P = k_pages.shape[0]
    masks = np.ascontiguousarray(masks, dtype=np.float32).reshape(P, M, TF)
    mx = np.zeros((M, GF), np.float32)
    sm = np.zeros((M, GF), np.float32)
    out = np.zeros((M, GF, DF), np.uint16)
    lib().orc_full_attention_pages(_p(q), _p(k_pages), _p(_u16(v_pages)), _p(masks), P, _p(mx), _p(sm), _p(out), M)
    return mx, sm, out


def full_attention_output(x, running_sum, post_rms, o_w, o_s, residual):
    """ops::full_attention_output (FO/src/ops.rs:176-199). Updates residual in place."""
    x = _u16(x).reshape(-1, QF)
    assert residual.dtype == np.uint16 and residual.flags["C_CONTIGUOUS"]
    lib().orc_full_attention_output(_p(x), _p(np.ascontiguousarray(running_sum, dtype=np.float32)),
                                    _p(_u16(post_rms)), _p(np.ascontiguousarray(o_w)),
                                    _p(np.ascontiguousarray(o_s, dtype=np.float32)), _p(residual), x.shape[0])


def softcap30(l: int) -> int:
    """Gemma's final-logit softcap of one bf16 logit (FO/src/ops.rs:256-293), bf16 bits."""
    return int(lib().orc_softcap30(int(l)))


def final_norm_and_logits(x, rms_w, lm_head_rows):
    """ops::final_norm_and_logits (FO/src/ops.rs:241-298) over the vocabulary rows given
    (lm_head_rows [W, 3840] bf16, any subset). Returns out bf16 bits [M, W]."""
    x = _u16(x).reshape(-1, H)
    w = _u16(lm_head_rows).reshape(-1, H)
    out = np.zeros((x.shape[0], w.shape[0]), np.uint16)
    lib().orc_final_norm_and_logits(_p(x), _p(_u16(rms_w)), _p(w), w.shape[0], _p(out), x.shape[0])
    return out


def ffn_weights(fmt: int, up, gate, down, up_s, gate_s, down_s, inv_g=(1.0, 1.0, 1.0)):
    keep = [np.ascontiguousarray(a) for a in (up, gate, down, up_s, gate_s, down_s)]
    w = FfnWeights(fmt, *[a.ctypes.data for a in keep], *[float(g) for g in inv_g])
    w._keep = keep  # keep the arrays alive with the struct
    return w


def decoder_feedforward(residual, pre_rms, weights: FfnWeights, post_rms=None, layer_scalar=None):
    """ops::decoder_feedforward (FO/src/ops.rs:201-239). Updates residual in place."""
    assert residual.dtype == np.uint16 and residual.flags["C_CONTIGUOUS"]
    M = residual.size // H
    lib().orc_decoder_feedforward(_p(residual), _p(_u16(pre_rms)), C.addressof(weights),
                                  _p(None if post_rms is None else _u16(post_rms)),
                                  _p(None if layer_scalar is None else _u16(layer_scalar)), M)


def ffn_up_gate(h, weights: FfnWeights) -> np.ndarray:
    h = _u16(h).reshape(-1, H)
    p = np.empty((h.shape[0], L), np.uint16)
    lib().orc_ffn_up_gate(_p(h), C.addressof(weights), _p(p), h.shape[0])
    return p


def ffn_down(p, weights: FfnWeights) -> np.ndarray:
    p = _u16(p).reshape(-1, L)
    d = np.empty((p.shape[0], H), np.uint16)
    lib().orc_ffn_down(_p(p), C.addressof(weights), _p(d), p.shape[0])
    return d


def set_threads(n: int) -> int:
    return int(lib().orc_set_threads(n))
