"""The reference's checkpoint, loaded onto the GPU (FO/src/host/load.rs).

The file is one safetensors checkpoint of Gemma-4-12B with FP8 attention projections and NVFP4
MLPs. The native reader (include/moa_ckpt.h) maps it, checks each tensor's dtype and shape as
load.rs does, and copies it into device tensors allocated here through two pinned staging
buffers. Field names follow load.rs's structs so that the operators take them unchanged:

    model = checkpoint.load_model()            # MOA_MODEL_DIR or RNGD_MODEL_DIR
    L = model.layers[0]                        # SlidingLayer (layer % 6 != 5) or FullLayer
    ops.sliding_attention_output(x, L.post_attention_norm, L.o_weight, L.o_weight_scale, residual)

Device tensors: bf16 as torch.bfloat16, E4M3 codes as torch.float8_e4m3fn, packed E2M1 pairs as
torch.uint8, global scales as torch.float32 holding 1 / g (load.rs:162-190).
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np
import torch

from . import _lib

H, L, W = 3840, 15360, 262144
QS, PS, DS = 4096, 2048, 256        # sliding layers (FO/src/axes.rs)
QF, PF, DF = 8192, 512, 512         # full-attention layers
LAYERS = 48                         # FO/src/lib.rs:22
MODEL_SUBDIRS = ("Gemma4-12B-it", "gemma-4-12b-it-NVFP4")


def is_full_layer(layer: int) -> bool:
    """Every sixth layer (index 5, 11, ...) attends over the whole context (load.rs:365-369)."""
    return layer % 6 == 5


def model_dir() -> Path:
    """The directory holding model.safetensors (load.rs:192-205): $MOA_MODEL_DIR, else
    $RNGD_MODEL_DIR (the reference's variable), or one of its two known subdirectories."""
    root = os.environ.get("MOA_MODEL_DIR") or os.environ.get("RNGD_MODEL_DIR")
    if not root:
        raise FileNotFoundError("MOA_MODEL_DIR (or RNGD_MODEL_DIR) is not set; point it at the model "
                                "directory or its parent")
    root = Path(root)
    for cand in (root, *(root / s for s in MODEL_SUBDIRS)):
        if (cand / "model.safetensors").is_file():
            return cand
    raise FileNotFoundError(f"no model.safetensors found under {root}")


class Checkpoint:
    """A mapped safetensors file (moa_ckpt_open). Use as a context manager or call close()."""

    def __init__(self, path: str | os.PathLike, device: int | torch.device | None = None):
        self.path = str(path)
        self._device = device
        h = C.c_void_p()
        _lib.call("moa_ckpt_open", self.path.encode(), C.byref(h))
        self._h = h

    def close(self) -> None:
        if self._h:
            _lib.call("moa_ckpt_close", self._h)
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---------------------------------------------------------------- inspection (host only)
    def names(self) -> list[str]:
        n = C.c_int()
        _lib.call("moa_ckpt_count", self._h, C.byref(n))
        out = []
        for i in range(n.value):
            s = C.c_char_p()
            _lib.call("moa_ckpt_name", self._h, i, C.byref(s))
            out.append(s.value.decode())
        return out

    def info(self, name: str) -> tuple[str, tuple[int, ...], int]:
        """(dtype, shape, nbytes) as the header states them."""
        dt, nd, nb = C.c_char_p(), C.c_int(), C.c_uint64()
        shape = (C.c_int64 * 8)()
        _lib.call("moa_ckpt_info", self._h, name.encode(), C.byref(dt), shape, C.byref(nd), C.byref(nb))
        return dt.value.decode(), tuple(shape[: nd.value]), nb.value

    def read(self, name: str) -> np.ndarray:
        """The tensor's raw bytes on the host (uint8)."""
        _, _, nb = self.info(name)
        out = np.empty(nb, np.uint8)
        _lib.call("moa_ckpt_read", self._h, name.encode(), C.c_void_p(out.ctypes.data), nb)
        return out

    def global_scale(self, name: str) -> float:
        """1 / g of an NVFP4 global scale g (load.rs:162-179)."""
        r = C.c_float()
        _lib.call("moa_ckpt_global_scale", self._h, name.encode(), C.byref(r))
        return r.value

    # ---------------------------------------------------------------- typed loads (device)
    @property
    def device(self) -> torch.device:
        d = self._device
        if d is None:
            d = torch.cuda.current_device()
        return torch.device("cuda", d.index if isinstance(d, torch.device) else d)

    def _empty(self, shape, dtype) -> torch.Tensor:
        return torch.empty(shape, dtype=dtype, device=self.device)

    def _stream(self) -> C.c_void_p:
        return C.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)

    def load_bf16(self, name: str, shape) -> torch.Tensor:
        shape = tuple(int(d) for d in shape)
        t = self._empty(shape, torch.bfloat16)
        arr = (C.c_int64 * max(1, len(shape)))(*shape)
        with torch.cuda.device(self.device):
            _lib.call("moa_ckpt_load_bf16", self._h, name.encode(), arr, len(shape), C.c_void_p(t.data_ptr()),
                      self._stream())
        return t

    def load_bf16_column(self, name: str, n: int) -> torch.Tensor:
        t = self._empty((n,), torch.bfloat16)
        with torch.cuda.device(self.device):
            _lib.call("moa_ckpt_load_bf16_column", self._h, name.encode(), n, C.c_void_p(t.data_ptr()),
                      self._stream())
        return t

    def load_f8(self, name: str, rows: int, cols: int) -> torch.Tensor:
        t = self._empty((rows, cols), torch.float8_e4m3fn)
        with torch.cuda.device(self.device):
            _lib.call("moa_ckpt_load_f8", self._h, name.encode(), rows, cols, C.c_void_p(t.data_ptr()), self._stream())
        return t

    def load_f4(self, name: str, rows: int, cols: int) -> torch.Tensor:
        t = self._empty((rows, cols // 2), torch.uint8)
        with torch.cuda.device(self.device):
            _lib.call("moa_ckpt_load_f4", self._h, name.encode(), rows, cols, C.c_void_p(t.data_ptr()), self._stream())
        return t

    def load_scalar_bf16(self, name: str) -> torch.Tensor:
        t = self._empty((8,), torch.bfloat16)
        with torch.cuda.device(self.device):
            _lib.call("moa_ckpt_load_scalar_bf16", self._h, name.encode(), C.c_void_p(t.data_ptr()), self._stream())
        return t

    def load_global_scale(self, name: str) -> torch.Tensor:
        t = self._empty((1,), torch.float32)
        with torch.cuda.device(self.device):
            _lib.call("moa_ckpt_load_global_scale", self._h, name.encode(), C.c_void_p(t.data_ptr()),
                      self._stream())
        return t


# --------------------------------------------------------------------- model structure (load.rs:9-90)

@dataclass
class MlpWeights:
    up_weight_packed: torch.Tensor
    gate_weight_packed: torch.Tensor
    down_weight_packed: torch.Tensor
    up_weight_scale: torch.Tensor
    gate_weight_scale: torch.Tensor
    down_weight_scale: torch.Tensor
    up_global_scale: torch.Tensor
    gate_global_scale: torch.Tensor
    down_global_scale: torch.Tensor


@dataclass
class SlidingLayer:
    input_norm: torch.Tensor
    q_weight: torch.Tensor
    k_weight: torch.Tensor
    v_weight: torch.Tensor
    q_weight_scale: torch.Tensor
    k_weight_scale: torch.Tensor
    v_weight_scale: torch.Tensor
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    post_attention_norm: torch.Tensor
    o_weight: torch.Tensor
    o_weight_scale: torch.Tensor
    pre_feedforward_norm: torch.Tensor
    post_feedforward_norm: torch.Tensor
    layer_scalar: torch.Tensor
    mlp: MlpWeights


@dataclass
class FullLayer:
    input_norm: torch.Tensor
    q_weight: torch.Tensor
    k_weight: torch.Tensor
    q_weight_scale: torch.Tensor
    k_weight_scale: torch.Tensor
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    post_attention_norm: torch.Tensor
    o_weight: torch.Tensor
    o_weight_scale: torch.Tensor
    pre_feedforward_norm: torch.Tensor
    post_feedforward_norm: torch.Tensor
    layer_scalar: torch.Tensor
    mlp: MlpWeights


@dataclass
class Model:
    model_dir: Path | None
    embedding_table: torch.Tensor | None     # [W, H]; also the lm_head (tied, gemma4.py:232-234)
    final_norm: torch.Tensor
    layers: dict = field(default_factory=dict)  # layer index -> SlidingLayer | FullLayer


def _prefix(layer: int) -> str:
    return f"model.language_model.layers.{layer}"


def load_mlp(ck: Checkpoint, prefix: str) -> MlpWeights:
    """load_mlp (load.rs:213-240): three NVFP4 projections, each packed E2M1 + E4M3 block-16 scales
    + the reciprocal of its global scale."""
    def proj(name, rows, cols):
        p = f"{prefix}.{name}"
        return (ck.load_f4(f"{p}.weight_packed", rows, cols), ck.load_f8(f"{p}.weight_scale", rows, cols // 16),
                ck.load_global_scale(f"{p}.weight_global_scale"))
    up, up_s, up_g = proj("up_proj", L, H)
    gate, gate_s, gate_g = proj("gate_proj", L, H)
    down, down_s, down_g = proj("down_proj", H, L)
    return MlpWeights(up, gate, down, up_s, gate_s, down_s, up_g, gate_g, down_g)


def _common(ck: Checkpoint, prefix: str):
    """load_common (load.rs:242-262)."""
    return (ck.load_bf16(f"{prefix}.pre_feedforward_layernorm.weight", (H,)),
            ck.load_bf16(f"{prefix}.post_feedforward_layernorm.weight", (H,)),
            ck.load_bf16(f"{prefix}.input_layernorm.weight", (H,)),
            load_mlp(ck, f"{prefix}.mlp"))


def load_sliding(ck: Checkpoint, layer: int) -> SlidingLayer:
    """load_sliding (load.rs:264-292)."""
    p = _prefix(layer)
    a = f"{p}.self_attn"
    pre, post, inp, mlp = _common(ck, p)
    return SlidingLayer(
        input_norm=inp,
        q_weight=ck.load_f8(f"{a}.q_proj.weight", QS, H), k_weight=ck.load_f8(f"{a}.k_proj.weight", PS, H),
        v_weight=ck.load_f8(f"{a}.v_proj.weight", PS, H),
        q_weight_scale=ck.load_bf16_column(f"{a}.q_proj.weight_scale", QS),
        k_weight_scale=ck.load_bf16_column(f"{a}.k_proj.weight_scale", PS),
        v_weight_scale=ck.load_bf16_column(f"{a}.v_proj.weight_scale", PS),
        q_norm=ck.load_bf16(f"{a}.q_norm.weight", (DS,)), k_norm=ck.load_bf16(f"{a}.k_norm.weight", (DS,)),
        post_attention_norm=ck.load_bf16(f"{p}.post_attention_layernorm.weight", (H,)),
        o_weight=ck.load_f8(f"{a}.o_proj.weight", H, QS),
        o_weight_scale=ck.load_bf16_column(f"{a}.o_proj.weight_scale", H),
        pre_feedforward_norm=pre, post_feedforward_norm=post,
        layer_scalar=ck.load_scalar_bf16(f"{p}.layer_scalar"), mlp=mlp)


def load_full(ck: Checkpoint, layer: int) -> FullLayer:
    """load_full (load.rs:294-320): one K projection (V is the unweighted norm of raw K)."""
    p = _prefix(layer)
    a = f"{p}.self_attn"
    pre, post, inp, mlp = _common(ck, p)
    return FullLayer(
        input_norm=inp,
        q_weight=ck.load_f8(f"{a}.q_proj.weight", QF, H), k_weight=ck.load_f8(f"{a}.k_proj.weight", PF, H),
        q_weight_scale=ck.load_bf16_column(f"{a}.q_proj.weight_scale", QF),
        k_weight_scale=ck.load_bf16_column(f"{a}.k_proj.weight_scale", PF),
        q_norm=ck.load_bf16(f"{a}.q_norm.weight", (DF,)), k_norm=ck.load_bf16(f"{a}.k_norm.weight", (DF,)),
        post_attention_norm=ck.load_bf16(f"{p}.post_attention_layernorm.weight", (H,)),
        o_weight=ck.load_f8(f"{a}.o_proj.weight", H, QF),
        o_weight_scale=ck.load_bf16_column(f"{a}.o_proj.weight_scale", H),
        pre_feedforward_norm=pre, post_feedforward_norm=post,
        layer_scalar=ck.load_scalar_bf16(f"{p}.layer_scalar"), mlp=mlp)


def load_model(path: str | os.PathLike | None = None, device: int | None = None, layers=None,
               embedding: bool = True) -> Model:
    """load_model (load.rs:353-377) for the decoder: the embedding table (the tied lm_head), the
    final norm and every layer, full-attention at index % 6 == 5. `layers` picks a subset of layer
    indices; `embedding=False` skips the 2 GB table. The vision and audio embedders of load.rs are
    not on the decoder path and are not loaded (their tensors stay readable through Checkpoint)."""
    mdir = None
    if path is None:
        mdir = model_dir()
        path = mdir / "model.safetensors"
    with Checkpoint(path, device) as ck:
        emb = ck.load_bf16("model.language_model.embed_tokens.weight", (W, H)) if embedding else None
        final = ck.load_bf16("model.language_model.norm.weight", (H,))
        idx = range(LAYERS) if layers is None else layers
        out = {i: (load_full(ck, i) if is_full_layer(i) else load_sliding(ck, i)) for i in idx}
    return Model(mdir, emb, final, out)
