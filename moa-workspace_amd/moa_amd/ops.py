"""The reference operator interface (FO/src/ops.rs) over the gfx950 C ABI.

Each function keeps the argument order and in-place semantics of the reference's
`#[device] fn` (the `device` handle becomes torch device memory on the current HIP
stream). Tensors are torch tensors on a ROCm device:

  bf16 tensors    torch.bfloat16 (or int16/uint16 bit views)
  E4M3 / E2M1 / E8M0 codes    torch.uint8 (E4M3 may also be torch.float8_e4m3fn)
  per-channel scales    torch.float32 (ops.rs uses bf16: pass torch.bfloat16 and the
                        exact bf16 entry point is used)

Errors from the library raise MoaError; nothing falls back to a CPU path. In checked mode
(set_checked(True), or MOA_CHECK_DEVICE_ERRORS=1 in the environment) every operator call is
followed by device_errors(), which synchronises, and any device-side error bit raises MoaError
(MOA_ERROR_DEVICE_STATE); off by default, since the check synchronises the stream.
"""
from __future__ import annotations

import ctypes as C
import os

import torch

from . import _lib

_checked = os.environ.get("MOA_CHECK_DEVICE_ERRORS", "") not in ("", "0")


def set_checked(on: bool) -> None:
    """Checked mode on or off (see the module docstring)."""
    global _checked
    _checked = bool(on)


def _call(name: str, *args) -> None:
    """One operator entry point; in checked mode, then the device's error bits."""
    _lib.call(name, *args)
    if _checked:
        bits = device_errors()
        if bits:
            raise _lib.MoaError(-5, f"{name}: device error bits {bits:#x} (1 rope offset, 2 kv offset, "
                                    f"4 expired wait: the device state is now tripped, see clear_device_state)")

H, L, NS, GS, DS, QS, PS, TS, E, W = 3840, 15360, 8, 2, 256, 4096, 2048, 1024, 32768, 262144


def _ptr(t: torch.Tensor | None, name: str, dtypes, numel: int | None = None):
    """The tensor's device address after the checks (an int: the signatures declare void*, so
    ctypes converts it). The cheapest torch attributes are used: every operator call runs this for
    each of its tensors, and `t.device` alone costs about 0.4 us per tensor."""
    if t is None:
        return None
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must live on a ROCm device, got {t.device}")
    if t.dtype not in dtypes:
        raise TypeError(f"{name}: dtype {t.dtype} not in {dtypes}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if numel is not None and t.numel() != numel:
        raise ValueError(f"{name}: expected {numel} elements, got {t.numel()}")
    return t.data_ptr()


_BF16 = (torch.bfloat16, torch.int16, torch.uint16)
_U8 = (torch.uint8, torch.float8_e4m3fn)
_F32 = (torch.float32,)
_I32 = (torch.int32,)


def _stream(t: torch.Tensor) -> int:
    """The current HIP stream of the current device (its handle as an int). The library serves a
    call from the scratch of the current device, so the call's tensors must live there: a tensor
    of another device is refused here rather than run against the wrong device's scratch."""
    dev = t.get_device()
    cur = torch.cuda.current_device()
    if dev != cur:
        raise ValueError(f"the call's tensors live on cuda:{dev} but the current device is cuda:{cur}; "
                         f"call it under torch.cuda.device({dev})")
    return torch.cuda.current_stream(dev).cuda_stream


def _rows(x: torch.Tensor, width: int, name: str) -> int:
    if x.numel() % width:
        raise ValueError(f"{name}: {x.numel()} elements is not a multiple of {width}")
    return x.numel() // width


def _scales(*ts):
    kinds = {t.dtype for t in ts}
    if kinds == {torch.float32}:
        return _F32, False
    if kinds <= set(_BF16):
        return _BF16, True
    raise TypeError(f"per-channel scales must all be float32 or all bfloat16, got {kinds}")


def sliding_project_qkv(x, q_weight, k_weight, v_weight, q_weight_scale, k_weight_scale, v_weight_scale,
                        input_rms_weight, q_rms_weight, k_rms_weight, kv_offset, rope_offset, cos, sin,
                        k_cache, v_cache, q_out) -> None:
    """ops::sliding_project_qkv (FO/src/ops.rs:37-76). Writes q_out and the K/V cache slot(s)."""
    M = _rows(x, H, "x")
    sd, bf = _scales(q_weight_scale, k_weight_scale, v_weight_scale)
    args = [
        _ptr(x, "x", _BF16), _ptr(q_weight, "q_weight", _U8, QS * H), _ptr(k_weight, "k_weight", _U8, PS * H),
        _ptr(v_weight, "v_weight", _U8, PS * H), _ptr(q_weight_scale, "q_weight_scale", sd, QS),
        _ptr(k_weight_scale, "k_weight_scale", sd, PS), _ptr(v_weight_scale, "v_weight_scale", sd, PS),
        _ptr(input_rms_weight, "input_rms_weight", _BF16, H), _ptr(q_rms_weight, "q_rms_weight", _BF16, DS),
        _ptr(k_rms_weight, "k_rms_weight", _BF16, DS), _ptr(kv_offset, "kv_offset", _I32, 1),
        _ptr(rope_offset, "rope_offset", _I32, 1), _ptr(cos, "cos", _BF16, E * DS), _ptr(sin, "sin", _BF16, E * DS),
        _ptr(k_cache, "k_cache", _BF16, TS * NS * DS), _ptr(v_cache, "v_cache", _BF16, TS * NS * DS),
        _ptr(q_out, "q_out", _BF16, M * QS),
    ]
    name = "moa_sliding_project_qkv_bf16_scales" if bf else "moa_sliding_project_qkv"
    _call(name, *args, M, _stream(x))


def sliding_attention(q, k, v, mask, out) -> None:
    """ops::sliding_attention (FO/src/ops.rs:118-128): out = softmax over the slots with mask != 0 of
    q . k_t (scale 1.0), times v. q / out [M, 8, 2, 256] bf16, k / v [1024, 8, 256] bf16 (the ring
    caches), mask [M, 1024] f32."""
    M = _rows(q, QS, "q")
    args = [
        _ptr(q, "q", _BF16), _ptr(k, "k", _BF16, TS * NS * DS), _ptr(v, "v", _BF16, TS * NS * DS),
        _ptr(mask, "mask", _F32, M * TS), _ptr(out, "out", _BF16, M * QS),
    ]
    _call("moa_sliding_attention", *args, M, _stream(q))


GF, DF, QF, PF, TF = 16, 512, 8192, 512, 512  # full-attention layers (FO/src/axes.rs)


def full_project_qkv(x, q_weight, k_weight, q_weight_scale, k_weight_scale, input_rms_weight, q_rms_weight,
                     k_rms_weight, kv_offset, rope_offset, cos, sin, k_cache, v_cache, q_out) -> None:
    """ops::full_project_qkv (FO/src/ops.rs:78-116). k_cache / v_cache are the position's page
    [512, 512]; V is the unweighted norm of the raw K projection. bf16 per-row weight scales."""
    M = _rows(x, H, "x")
    args = [
        _ptr(x, "x", _BF16), _ptr(q_weight, "q_weight", _U8, QF * H), _ptr(k_weight, "k_weight", _U8, PF * H),
        _ptr(q_weight_scale, "q_weight_scale", _BF16, QF), _ptr(k_weight_scale, "k_weight_scale", _BF16, PF),
        _ptr(input_rms_weight, "input_rms_weight", _BF16, H), _ptr(q_rms_weight, "q_rms_weight", _BF16, DF),
        _ptr(k_rms_weight, "k_rms_weight", _BF16, DF), _ptr(kv_offset, "kv_offset", _I32, 1),
        _ptr(rope_offset, "rope_offset", _I32, 1), _ptr(cos, "cos", _BF16, E * DF), _ptr(sin, "sin", _BF16, E * DF),
        _ptr(k_cache, "k_cache", _BF16, TF * DF), _ptr(v_cache, "v_cache", _BF16, TF * DF),
        _ptr(q_out, "q_out", _BF16, M * QF),
    ]
    _call("moa_full_project_qkv", *args, M, _stream(x))


def _full_page(name, q, k, v, mask, running_max, running_sum, out):
    M = _rows(q, QF, "q")
    args = [
        _ptr(q, "q", _BF16), _ptr(k, "k", _BF16, TF * DF), _ptr(v, "v", _BF16, TF * DF),
        _ptr(mask, "mask", _F32, M * TF), _ptr(running_max, "running_max", _F32, M * GF),
        _ptr(running_sum, "running_sum", _F32, M * GF), _ptr(out, "out", _BF16, M * QF),
    ]
    _call(name, *args, M, _stream(q))


def full_attention_first_page(q, k, v, mask, running_max, running_sum, out) -> None:
    """ops::full_attention_first_page (FO/src/ops.rs:148-160): starts the running softmax state
    (max, sum [M, 16] f32; out [M, 16, 512] bf16, un-normalised) from one 512-slot page."""
    _full_page("moa_full_attention_first_page", q, k, v, mask, running_max, running_sum, out)


def full_attention_page(q, k, v, mask, running_max, running_sum, out) -> None:
    """ops::full_attention_page (FO/src/ops.rs:162-174): folds one more page into the state."""
    _full_page("moa_full_attention_page", q, k, v, mask, running_max, running_sum, out)


def full_attention(q, k_pages, v_pages, masks, running_max, running_sum, out) -> None:
    """The state full_attention_first_page + full_attention_page over pages 1 .. P-1 leave, in two
    launches: k_pages / v_pages [P, 512, 512] bf16 (contiguous), masks [P, M, 512] f32."""
    M = _rows(q, QF, "q")
    P = _rows(k_pages, TF * DF, "k_pages")
    args = [
        _ptr(q, "q", _BF16), _ptr(k_pages, "k_pages", _BF16), _ptr(v_pages, "v_pages", _BF16, P * TF * DF),
        _ptr(masks, "masks", _F32, P * M * TF),
    ]
    tail = [_ptr(running_max, "running_max", _F32, M * GF), _ptr(running_sum, "running_sum", _F32, M * GF),
            _ptr(out, "out", _BF16, M * QF)]
    _call("moa_full_attention", *args, P, *tail, M, _stream(q))


def full_attention_output(x, running_sum, post_attn_rms_weight, o_weight, o_weight_scale, residual) -> None:
    """ops::full_attention_output (FO/src/ops.rs:176-199): x / running_sum, the O projection
    (K = 8192, bf16 per-row scales), post-norm and residual add, in place."""
    M = _rows(x, QF, "x")
    args = [
        _ptr(x, "x", _BF16), _ptr(running_sum, "running_sum", _F32, M * GF),
        _ptr(post_attn_rms_weight, "post_attn_rms_weight", _BF16, H), _ptr(o_weight, "o_weight", _U8, H * QF),
        _ptr(o_weight_scale, "o_weight_scale", _BF16, H), _ptr(residual, "residual", _BF16, M * H),
    ]
    _call("moa_full_attention_output", *args, M, _stream(x))


def final_norm_and_logits(input, rms_weight, lm_head_weight, out) -> None:
    """ops::final_norm_and_logits (FO/src/ops.rs:241-298): out = softcap30(bf16(RMSNorm(input) .
    lm_head_weight^T)). input [M, 3840] bf16, lm_head_weight [262144, 3840] bf16, out [M, 262144] bf16."""
    M = _rows(input, H, "input")
    args = [
        _ptr(input, "input", _BF16), _ptr(rms_weight, "rms_weight", _BF16, H),
        _ptr(lm_head_weight, "lm_head_weight", _BF16, W * H), _ptr(out, "out", _BF16, M * W),
    ]
    _call("moa_final_norm_and_logits", *args, M, _stream(input))


def sliding_attention_output(x, post_attn_rms_weight, o_weight, o_weight_scale, residual) -> None:
    """ops::sliding_attention_output (FO/src/ops.rs:130-146). Updates residual in place."""
    M = _rows(x, QS, "x")
    sd, bf = _scales(o_weight_scale)
    args = [
        _ptr(x, "x", _BF16), _ptr(post_attn_rms_weight, "post_attn_rms_weight", _BF16, H),
        _ptr(o_weight, "o_weight", _U8, H * QS), _ptr(o_weight_scale, "o_weight_scale", sd, H),
        _ptr(residual, "residual", _BF16, M * H),
    ]
    name = "moa_sliding_attention_output_bf16_scales" if bf else "moa_sliding_attention_output"
    _call(name, *args, M, _stream(x))


def decoder_feedforward(residual, pre_ff_rms_weight, up_weight_packed, gate_weight_packed, down_weight_packed,
                        up_weight_scale, gate_weight_scale, down_weight_scale, up_global_scale, gate_global_scale,
                        down_global_scale, post_ff_rms_weight, layer_scalar) -> None:
    """ops::decoder_feedforward (FO/src/ops.rs:201-239), NVFP4 weights. Updates residual in place."""
    M = _rows(residual, H, "residual")
    args = [
        _ptr(residual, "residual", _BF16), _ptr(pre_ff_rms_weight, "pre_ff_rms_weight", _BF16, H),
        _ptr(up_weight_packed, "up_weight_packed", _U8, L * H // 2),
        _ptr(gate_weight_packed, "gate_weight_packed", _U8, L * H // 2),
        _ptr(down_weight_packed, "down_weight_packed", _U8, H * L // 2),
        _ptr(up_weight_scale, "up_weight_scale", _U8, L * H // 16),
        _ptr(gate_weight_scale, "gate_weight_scale", _U8, L * H // 16),
        _ptr(down_weight_scale, "down_weight_scale", _U8, H * L // 16),
        _ptr(up_global_scale, "up_global_scale", _F32, 1), _ptr(gate_global_scale, "gate_global_scale", _F32, 1),
        _ptr(down_global_scale, "down_global_scale", _F32, 1),
        _ptr(post_ff_rms_weight, "post_ff_rms_weight", _BF16, H), _ptr(layer_scalar, "layer_scalar", _BF16, 8),
    ]
    _call("moa_decoder_feedforward", *args, M, _stream(residual))


def decoder_feedforward_fp8(residual, pre_ff_rms_weight, up_weight, gate_weight, down_weight, up_weight_scale,
                            gate_weight_scale, down_weight_scale, post_ff_rms_weight=None, layer_scalar=None) -> None:
    """GeGLU FFN with FP8 E4M3 weights and f32 per-channel scales."""
    M = _rows(residual, H, "residual")
    args = [
        _ptr(residual, "residual", _BF16), _ptr(pre_ff_rms_weight, "pre_ff_rms_weight", _BF16, H),
        _ptr(up_weight, "up_weight", _U8, L * H), _ptr(gate_weight, "gate_weight", _U8, L * H),
        _ptr(down_weight, "down_weight", _U8, H * L), _ptr(up_weight_scale, "up_weight_scale", _F32, L),
        _ptr(gate_weight_scale, "gate_weight_scale", _F32, L), _ptr(down_weight_scale, "down_weight_scale", _F32, H),
        _ptr(post_ff_rms_weight, "post_ff_rms_weight", _BF16, H), _ptr(layer_scalar, "layer_scalar", _BF16, 8),
    ]
    _call("moa_decoder_feedforward_fp8", *args, M, _stream(residual))


def decoder_feedforward_mxfp4(residual, pre_ff_rms_weight, up_weight_packed, gate_weight_packed, down_weight_packed,
                              up_weight_scale, gate_weight_scale, down_weight_scale, post_ff_rms_weight=None,
                              layer_scalar=None) -> None:
    """GeGLU FFN with MXFP4 weights (E2M1 + E8M0 per 32)."""
    M = _rows(residual, H, "residual")
    args = [
        _ptr(residual, "residual", _BF16), _ptr(pre_ff_rms_weight, "pre_ff_rms_weight", _BF16, H),
        _ptr(up_weight_packed, "up_weight_packed", _U8, L * H // 2),
        _ptr(gate_weight_packed, "gate_weight_packed", _U8, L * H // 2),
        _ptr(down_weight_packed, "down_weight_packed", _U8, H * L // 2),
        _ptr(up_weight_scale, "up_weight_scale", _U8, L * H // 32),
        _ptr(gate_weight_scale, "gate_weight_scale", _U8, L * H // 32),
        _ptr(down_weight_scale, "down_weight_scale", _U8, H * L // 32),
        _ptr(post_ff_rms_weight, "post_ff_rms_weight", _BF16, H), _ptr(layer_scalar, "layer_scalar", _BF16, 8),
    ]
    _call("moa_decoder_feedforward_mxfp4", *args, M, _stream(residual))


def _o_args(x, post_attn_rms_weight, o_weight, o_weight_scale, residual, scale_dtypes):
    M = _rows(x, QS, "x")
    return M, [
        _ptr(x, "x", _BF16), _ptr(post_attn_rms_weight, "post_attn_rms_weight", _BF16, H),
        _ptr(o_weight, "o_weight", _U8, H * QS), _ptr(o_weight_scale, "o_weight_scale", scale_dtypes, H),
        _ptr(residual, "residual", _BF16, M * H),
    ]


def sliding_attention_output_feedforward(x, post_attn_rms_weight, o_weight, o_weight_scale, residual,
                                         pre_ff_rms_weight, up_weight_packed, gate_weight_packed, down_weight_packed,
                                         up_weight_scale, gate_weight_scale, down_weight_scale, up_global_scale,
                                         gate_global_scale, down_global_scale, post_ff_rms_weight,
                                         layer_scalar) -> None:
    """The tail of the reference's sliding-layer step (FO/src/host/runtime.rs:440-459, 543-571):
    sliding_attention_output (bf16 O scales, as ops.rs:136) then decoder_feedforward (NVFP4) on the
    same residual, in place. One launch per token row; the same bits as the two calls in turn."""
    M, args = _o_args(x, post_attn_rms_weight, o_weight, o_weight_scale, residual, _BF16)
    args += [
        _ptr(pre_ff_rms_weight, "pre_ff_rms_weight", _BF16, H),
        _ptr(up_weight_packed, "up_weight_packed", _U8, L * H // 2),
        _ptr(gate_weight_packed, "gate_weight_packed", _U8, L * H // 2),
        _ptr(down_weight_packed, "down_weight_packed", _U8, H * L // 2),
        _ptr(up_weight_scale, "up_weight_scale", _U8, L * H // 16),
        _ptr(gate_weight_scale, "gate_weight_scale", _U8, L * H // 16),
        _ptr(down_weight_scale, "down_weight_scale", _U8, H * L // 16),
        _ptr(up_global_scale, "up_global_scale", _F32, 1), _ptr(gate_global_scale, "gate_global_scale", _F32, 1),
        _ptr(down_global_scale, "down_global_scale", _F32, 1),
        _ptr(post_ff_rms_weight, "post_ff_rms_weight", _BF16, H), _ptr(layer_scalar, "layer_scalar", _BF16, 8),
    ]
    _call("moa_sliding_attention_output_feedforward", *args, M, _stream(x))


def sliding_attention_output_feedforward_fp8(x, post_attn_rms_weight, o_weight, o_weight_scale, residual,
                                             pre_ff_rms_weight, up_weight, gate_weight, down_weight, up_weight_scale,
                                             gate_weight_scale, down_weight_scale, post_ff_rms_weight=None,
                                             layer_scalar=None) -> None:
    """sliding_attention_output (f32 O scales) then decoder_feedforward_fp8 on the same residual
    (BASELINE configs 1 then 0), in place: one launch per token row, the same bits as the two calls."""
    M, args = _o_args(x, post_attn_rms_weight, o_weight, o_weight_scale, residual, _F32)
    args += [
        _ptr(pre_ff_rms_weight, "pre_ff_rms_weight", _BF16, H),
        _ptr(up_weight, "up_weight", _U8, L * H), _ptr(gate_weight, "gate_weight", _U8, L * H),
        _ptr(down_weight, "down_weight", _U8, H * L), _ptr(up_weight_scale, "up_weight_scale", _F32, L),
        _ptr(gate_weight_scale, "gate_weight_scale", _F32, L), _ptr(down_weight_scale, "down_weight_scale", _F32, H),
        _ptr(post_ff_rms_weight, "post_ff_rms_weight", _BF16, H), _ptr(layer_scalar, "layer_scalar", _BF16, 8),
    ]
    _call("moa_sliding_attention_output_feedforward_fp8", *args, M, _stream(x))


def sliding_attention_output_feedforward_mxfp4(x, post_attn_rms_weight, o_weight, o_weight_scale, residual,
                                               pre_ff_rms_weight, up_weight_packed, gate_weight_packed,
                                               down_weight_packed, up_weight_scale, gate_weight_scale,
                                               down_weight_scale, post_ff_rms_weight=None,
                                               layer_scalar=None) -> None:
    """sliding_attention_output (f32 O scales) then decoder_feedforward_mxfp4 on the same residual."""
    M, args = _o_args(x, post_attn_rms_weight, o_weight, o_weight_scale, residual, _F32)
    args += [
        _ptr(pre_ff_rms_weight, "pre_ff_rms_weight", _BF16, H),
        _ptr(up_weight_packed, "up_weight_packed", _U8, L * H // 2),
        _ptr(gate_weight_packed, "gate_weight_packed", _U8, L * H // 2),
        _ptr(down_weight_packed, "down_weight_packed", _U8, H * L // 2),
        _ptr(up_weight_scale, "up_weight_scale", _U8, L * H // 32),
        _ptr(gate_weight_scale, "gate_weight_scale", _U8, L * H // 32),
        _ptr(down_weight_scale, "down_weight_scale", _U8, H * L // 32),
        _ptr(post_ff_rms_weight, "post_ff_rms_weight", _BF16, H), _ptr(layer_scalar, "layer_scalar", _BF16, 8),
    ]
    _call("moa_sliding_attention_output_feedforward_mxfp4", *args, M, _stream(x))


def fp8_scaled_projection(x, w, scale, out) -> None:
    """scaled_projection (FO/scripts/generate_references.py:265-274): out = bf16((x . W^T) * scale)."""
    N, K = w.shape
    M = _rows(x, K, "x")
    args = [_ptr(x, "x", _BF16), _ptr(w, "w", _U8, N * K), _ptr(scale, "scale", _F32, N),
            _ptr(out, "out", _BF16, M * N)]
    _call("moa_fp8_scaled_projection", *args, M, N, K, _stream(x))


def device_errors(device: torch.device | None = None) -> int:
    """Synchronise the current stream of `device` (default: the current device); return and clear
    that device's kernel-raised error bits."""
    bits = C.c_uint32(0)
    with torch.cuda.device(device):  # the library reads the bits of the current device
        s = torch.cuda.current_stream().cuda_stream
        _lib.call("moa_device_errors", C.c_void_p(s), C.byref(bits))
    return int(bits.value)


def clear_device_state(device: int = 0) -> None:
    """moa_clear_device_state: acknowledge a tripped device (an expired wait's outputs restored)."""
    _lib.call("moa_clear_device_state", device)


def format_selftest(device="cuda") -> torch.Tensor:
    out = torch.zeros(721924, dtype=torch.int32, device=device)  # layout: moa_decode.hip format_selftest_kernel
    _lib.call("moa_format_selftest", C.c_void_p(out.data_ptr()), _stream(out))
    return out


def init(device: int = 0) -> None:
    _lib.call("moa_init", device)
