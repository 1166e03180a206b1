"""Inputs for the three operators (host numpy arrays; bf16 as uint16 bits).

Two families:
  * reference runs -- the exact inputs of the reference harness's run `r`, seeded
    `run{r}.{test}.{tensor}` (FO/src/bin/test_kernels.rs:481-624, generate_references.py:291-414);
  * BASELINE configs -- the measurement workloads (normal weights quantised to FP8 per channel
    or MXFP4, N(0,1) activations), drawn from a generator keyed by
    `cfg{k}.seed{s}.{tensor}` (numpy PCG64 seeded by the name's FNV-1a hash).
"""
from __future__ import annotations

import numpy as np

from . import formats as F
from . import prng

H, L, NS, GS, DS, QS, PS, TS, E, W = 3840, 15360, 8, 2, 256, 4096, 2048, 1024, 32768, 262144

# Reference distributions (test_kernels.rs:147-155; generate_references.py:64-77).
WEIGHT_EXP = (7, 14)
LOCAL_SCALE_EXP = (8, 10)
ROW_SCALE = (0.0, 1e-3)
UNIT = (0.0, 1.0)
RMS_WEIGHT = (0.75, 1.25)
ACTIVATION = (-1.0, 1.0)
GLOBAL_SCALE = (2048.0, 16384.0)
LAYER_SCALAR = 0.375


def rope_row(head_dim: int, theta: float, factor: float, pos: int):
    """cos, sin for one position in f64, narrowed to f32 (generate_references.py:184-197)."""
    angles = int(factor * head_dim // 2)
    inv = 1.0 / (np.float64(theta) ** (np.arange(0, 2 * angles, 2, dtype=np.float64) / head_dim))
    inv = np.concatenate([inv, np.zeros(head_dim // 2 - angles)])
    emb = np.concatenate([pos * inv, pos * inv])
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)


def kernel_sin(sin: np.ndarray) -> np.ndarray:
    """The sin operand the kernel receives: low half negated (generate_references.py:200-210)."""
    out = sin.copy()
    out[: out.size // 2] *= -1.0
    return out


def rope_tables(positions, theta: float = 10_000.0):
    """Full [E, 256] bf16 cos/sin tables with the given rows filled (zeros elsewhere, as the
    reference harness builds them, test_kernels.rs:421-439)."""
    cos = np.zeros((E, DS), np.uint16)
    sin = np.zeros((E, DS), np.uint16)
    for p in positions:
        c, s = rope_row(DS, theta, 1.0, int(p))
        cos[p] = prng.f32_to_bf16_bits(c)
        sin[p] = prng.f32_to_bf16_bits(kernel_sin(s))
    return cos, sin


# ----------------------------------------------------------- reference runs

class RefSynth:
    """One (run, test) pair of the reference harness; records each input's checksum."""

    def __init__(self, test: str, run: int):
        self.test, self.run = test, run
        self.checks: dict[str, int] = {}

    def seed(self, name: str) -> str:
        return f"run{self.run}.{self.test}.{name}"

    def keep(self, name: str, a: np.ndarray) -> np.ndarray:
        self.checks[name] = prng.checksum(a)
        return a

    def bf16(self, name, count, span):
        return self.keep(name, prng.bf16_uniform(self.seed(name), count, *span))

    def f8(self, name, count, band, signed=True):
        return self.keep(name, prng.f8_banded(self.seed(name), count, band[0], band[1], signed))

    def f4(self, name, count):
        return self.keep(name, prng.f4_nibbles(self.seed(name), count))


def ref_qkv_inputs(run: int) -> dict:
    """test_kernels.rs:481-546 / generate_references.py:291-334."""
    s = RefSynth("sliding_project_qkv", run)
    pos = prng.run_pos(run)
    in_rms = s.bf16("input_rms_weight", H, RMS_WEIGHT)
    signs = s.keep("x_signs", prng.bf16_signs(s.seed("x_signs"), H, 1.0))
    # x = bf16(sign / input_rms_weight): normalises to one magnitude with the drawn signs (test_kernels.rs:360-379)
    x = s.keep("x_exact", prng.f32_to_bf16_bits(prng.bf16_bits_to_f32(signs) / prng.bf16_bits_to_f32(in_rms)))
    d = dict(
        x=x, input_rms_weight=in_rms,
        q_weight=s.f8("q_weight", QS * H, WEIGHT_EXP).reshape(QS, H),
        k_weight=s.f8("k_weight", PS * H, WEIGHT_EXP).reshape(PS, H),
        v_weight=s.f8("v_weight", PS * H, WEIGHT_EXP).reshape(PS, H),
        q_weight_scale=s.bf16("q_weight_scale", QS, ROW_SCALE),
        k_weight_scale=s.bf16("k_weight_scale", PS, ROW_SCALE),
        v_weight_scale=s.bf16("v_weight_scale", PS, ROW_SCALE),
        q_rms_weight=s.bf16("q_rms_weight", DS, UNIT),
        k_rms_weight=s.bf16("k_rms_weight", DS, UNIT),
        pos=pos,
    )
    d["cos"], d["sin"] = rope_tables([pos])
    s.keep("cos", d["cos"][pos])
    s.keep("sin", d["sin"][pos])
    d["rope_offset"] = pos * DS * 2
    d["kv_offset"] = (pos % TS) * NS * DS * 2
    d["checks"] = s.checks
    return d


def ref_o_inputs(run: int) -> dict:
    """test_kernels.rs:548-570 / generate_references.py:337-355."""
    s = RefSynth("sliding_attention_output", run)
    d = dict(
        x=s.bf16("x", QS, ACTIVATION),
        post_attn_rms_weight=s.bf16("post_attn_rms_weight", H, UNIT),
        o_weight=s.f8("o_weight", H * QS, WEIGHT_EXP).reshape(H, QS),
        o_weight_scale=s.bf16("o_weight_scale", H, ROW_SCALE),
        residual=s.bf16("residual", H, UNIT),
    )
    d["checks"] = s.checks
    return d


def ref_ffn_inputs(run: int) -> dict:
    """test_kernels.rs:572-624 / generate_references.py:375-414 (NVFP4)."""
    s = RefSynth("decoder_feedforward", run)
    d = dict(
        residual=s.bf16("residual", H, UNIT),
        pre_ff_rms_weight=s.bf16("pre_ff_rms_weight", H, UNIT),
        post_ff_rms_weight=s.bf16("post_ff_rms_weight", H, UNIT),
    )
    for name, rows, cols in (("up", L, H), ("gate", L, H), ("down", H, L)):
        d[f"{name}_weight_packed"] = s.f4(f"{name}_weight_packed", rows * cols).reshape(rows, cols // 2)
        d[f"{name}_weight_scale"] = s.f8(f"{name}_weight_scale", rows * cols // 16, LOCAL_SCALE_EXP, False).reshape(rows, cols // 16)
        g = prng.f32_uniform(f"run{run}.global.{name}_global_scale", 1, *GLOBAL_SCALE)[0]
        d[f"{name}_global_scale"] = np.array([np.float32(1.0) / g], np.float32)
        s.keep(f"{name}_global_scale", d[f"{name}_global_scale"])
    d["layer_scalar"] = s.keep("layer_scalar", prng.f32_to_bf16_bits(np.full(8, LAYER_SCALAR, np.float32)))
    d["checks"] = s.checks
    return d


# --------------------------------------------------------- BASELINE configs

def _gen(name: str) -> np.random.Generator:
    """numpy PCG64 generator seeded by the FNV-1a hash of the tensor's name."""
    return np.random.Generator(np.random.PCG64(prng.name_hash(name)))


def normal(name: str, shape, std: float = 1.0, mean: float = 0.0) -> np.ndarray:
    z = _gen(name).standard_normal(size=shape, dtype=np.float32)
    return (z * np.float32(std) + np.float32(mean)).astype(np.float32)


def bf16_normal(name: str, shape, std: float = 1.0, mean: float = 0.0) -> np.ndarray:
    return prng.f32_to_bf16_bits(normal(name, shape, std, mean))


def rms_weight(name: str, n: int) -> np.ndarray:
    """RMSNorm weight stored as the value 1 + w, w ~ N(0, 0.1)."""
    return prng.f32_to_bf16_bits(np.float32(1.0) + normal(name, (n,), 0.1))


def fp8_weight(name: str, rows: int, cols: int):
    return F.quantize_fp8_rows(normal(name, (rows, cols), 0.02))


def mxfp4_weight(name: str, rows: int, cols: int):
    return F.quantize_mxfp4(normal(name, (rows, cols), 0.02))


def cfg_ffn_fp8(seed: int = 0, M: int = 1, tag: str = "cfg0") -> dict:
    """Config 0: FP8 E4M3 per-channel FFN; post-norm weight and layer scalar included (the
    full FO/src/ops.rs:201-239 contract)."""
    n = lambda t: f"{tag}.seed{seed}.{t}"
    up, su = fp8_weight(n("up"), L, H)
    gate, sg = fp8_weight(n("gate"), L, H)
    down, sd = fp8_weight(n("down"), H, L)
    return dict(residual=bf16_normal(n("residual"), (M, H)), pre_ff_rms_weight=rms_weight(n("pre_rms"), H),
                post_ff_rms_weight=rms_weight(n("post_rms"), H),
                layer_scalar=prng.f32_to_bf16_bits(np.full(8, LAYER_SCALAR, np.float32)),
                up_weight=up, gate_weight=gate, down_weight=down,
                up_weight_scale=su, gate_weight_scale=sg, down_weight_scale=sd)


def cfg_o(seed: int = 0, M: int = 1, tag: str = "cfg1") -> dict:
    """Config 1: attention-output projection, FP8 W_o [3840,4096] per-channel f32 scales."""
    n = lambda t: f"{tag}.seed{seed}.{t}"
    ow, os_ = fp8_weight(n("o"), H, QS)
    return dict(x=bf16_normal(n("x"), (M, QS)), post_attn_rms_weight=rms_weight(n("post_rms"), H),
                o_weight=ow, o_weight_scale=os_, residual=bf16_normal(n("residual"), (M, H)))


def cfg_qkv(seed: int = 0, M: int = 1, tag: str = "cfg2", theta: float = 10_000.0, pos: int | None = None) -> dict:
    """Config 2: fused QKV at a random position p in [0, 8191] (rows p..p+M-1), ring slot p mod 1024,
    every other cache slot pre-filled N(0,1)."""
    n = lambda t: f"{tag}.seed{seed}.{t}"
    if pos is None:
        pos = int(prng.words(n("pos"), 1)[0] % np.uint64(8192))
    qw, qs = fp8_weight(n("q"), QS, H)
    kw, ks = fp8_weight(n("k"), PS, H)
    vw, vs = fp8_weight(n("v"), PS, H)
    cos, sin = rope_tables(range(pos, pos + M), theta)
    return dict(x=bf16_normal(n("x"), (M, H)), q_weight=qw, k_weight=kw, v_weight=vw,
                q_weight_scale=qs, k_weight_scale=ks, v_weight_scale=vs,
                input_rms_weight=rms_weight(n("in_rms"), H), q_rms_weight=rms_weight(n("q_rms"), DS),
                k_rms_weight=rms_weight(n("k_rms"), DS), pos=pos,
                rope_offset=pos * DS * 2, kv_offset=(pos % TS) * NS * DS * 2, cos=cos, sin=sin,
                k_cache=bf16_normal(n("k_cache"), (TS, NS, DS)), v_cache=bf16_normal(n("v_cache"), (TS, NS, DS)))


def cfg_layer_chunk(seed: int = 0, M: int = 256, tag: str = "cfg4") -> dict:
    """Config 4's activations: one decoder-layer chunk of M prefill rows at positions 0..M-1
    (ring slots 0..M-1, other slots pre-filled N(0,1)); the attention output that feeds the
    O-projection is a seeded N(0,1) bf16 input. The FP8 weights are those of configs 0-2 (same
    shapes and distributions)."""
    n = lambda t: f"{tag}.seed{seed}.{t}"
    cos, sin = rope_tables(range(0, M), 10_000.0)
    return dict(x=bf16_normal(n("x"), (M, H)), attn=bf16_normal(n("attn"), (M, QS)), pos=0, rope_offset=0,
                kv_offset=0, cos=cos, sin=sin,
                k_cache=bf16_normal(n("k_cache"), (TS, NS, DS)), v_cache=bf16_normal(n("v_cache"), (TS, NS, DS)))


def attention_mask(M: int, pos) -> np.ndarray:
    """The runtime's mask rows (FO/src/host/runtime.rs:160, 409): row min(pos, 1023) has 1.0 at
    slots <= that row and 0.0 beyond. pos: one position per token row."""
    pos = np.broadcast_to(np.asarray(pos), (M,))
    rows = np.minimum(pos, TS - 1)
    return (np.arange(TS)[None, :] <= rows[:, None]).astype(np.float32)


def cfg_attention(seed: int = 0, M: int = 1, pos=1023, q_std: float = 1.0, tag: str = "attn") -> dict:
    """sliding_attention inputs: q [M, 8, 2, 256] bf16 ~ N(0, q_std) (q after head norm has unit
    RMS, so q_std = 1 gives the real, peaky scores), ring caches [1024, 8, 256] ~ N(0, 1), and the
    runtime's mask rows for the given positions."""
    n = lambda t: f"{tag}.seed{seed}.{t}"
    return dict(q=bf16_normal(n("q"), (M, NS, QS // (NS * DS), DS), q_std),
                k_cache=bf16_normal(n("k_cache"), (TS, NS, DS)), v_cache=bf16_normal(n("v_cache"), (TS, NS, DS)),
                mask=attention_mask(M, pos))


# ------------------------------------------------------------ full-attention layers

GF, DF, QF, PF, TF = 16, 512, 8192, 512, 512


def rope_tables_full(positions, theta: float = 1_000_000.0, rotated: int = 128):
    """[E, 512] bf16 cos / sin of the full-attention layers as the runtime builds them
    (FO/src/host/runtime.rs:298-322): f32 angles pos / theta^(2i / 512) for the first rotated / 2
    entries of each half (25 % of the head), cos 1 and sin 0 beyond, the low half of sin negated.
    Rows outside `positions` stay zero."""
    half, rh = DF // 2, rotated // 2
    i = np.arange(half)
    den = np.power(np.float32(theta), (2 * i).astype(np.float32) / np.float32(DF)).astype(np.float32)
    cos = np.zeros((E, DF), np.uint16)
    sin = np.zeros((E, DF), np.uint16)
    for p in positions:
        freq = (np.float32(p) / den).astype(np.float32)
        c = np.where(i < rh, np.cos(freq), np.float32(1.0)).astype(np.float32)
        lo = np.where(i < rh, -np.sin(freq), np.float32(0.0)).astype(np.float32)
        hi = np.where(i < rh, np.sin(freq), np.float32(0.0)).astype(np.float32)
        cos[p] = prng.f32_to_bf16_bits(np.concatenate([c, c]))
        sin[p] = prng.f32_to_bf16_bits(np.concatenate([lo, hi]))
    return cos, sin


def _bf16_scales(s):
    return prng.f32_to_bf16_bits(np.asarray(s, np.float32))


def cfg_full_qkv(seed: int = 0, M: int = 1, pos: int = 700, tag: str = "full") -> dict:
    """full_project_qkv inputs for rows at positions pos .. pos + M - 1 (one page): FP8 Q [8192, 3840]
    and K [512, 3840] with bf16 per-row scales, N(0, 1) activations, the page pre-filled N(0, 1)."""
    n = lambda t: f"{tag}.seed{seed}.{t}"
    qw, qs = fp8_weight(n("q"), QF, H)
    kw, ks = fp8_weight(n("k"), PF, H)
    cos, sin = rope_tables_full(range(pos, pos + M))
    return dict(x=bf16_normal(n("x"), (M, H)), q_weight=qw, k_weight=kw, q_weight_scale=_bf16_scales(qs),
                k_weight_scale=_bf16_scales(ks), input_rms_weight=rms_weight(n("in_rms"), H),
                q_rms_weight=rms_weight(n("q_rms"), DF), k_rms_weight=rms_weight(n("k_rms"), DF), pos=pos,
                rope_offset=pos * DF * 2, kv_offset=(pos % TF) * DF * 2, cos=cos, sin=sin,
                k_cache=bf16_normal(n("k_page"), (TF, DF)), v_cache=bf16_normal(n("v_page"), (TF, DF)))


def full_masks(P: int, pos) -> np.ndarray:
    """[P, M, 512] mask rows of the runtime (FO/src/host/runtime.rs:159-165, 496-503) for rows at
    positions `pos`: 1.0 over pages before the position's page, its diagonal row on that page
    (slots <= pos % 512), 0.0 on later pages."""
    pos = np.atleast_1d(np.asarray(pos))
    out = np.zeros((P, pos.size, TF), np.float32)
    for m, p in enumerate(pos):
        page, row = int(p) // TF, int(p) % TF
        for pg in range(P):
            if pg < page:
                out[pg, m] = 1.0
            elif pg == page:
                out[pg, m, : row + 1] = 1.0
    return out


def cfg_full_attention(seed: int = 0, M: int = 1, P: int = 2, pos=None, q_std: float = 1.0,
                       tag: str = "fattn") -> dict:
    """Full-attention pages: q [M, 16, 512] ~ N(0, q_std) (1.0: unit-RMS heads, as after the q
    norm), P pages of K and V [512, 512] ~ N(0, 1), and the runtime's masks for positions `pos`
    (default: the last slot of page P - 1)."""
    n = lambda t: f"{tag}.seed{seed}.{t}"
    if pos is None:
        pos = [P * TF - 1] * M
    return dict(q=bf16_normal(n("q"), (M, GF, DF), q_std), k_pages=bf16_normal(n("k"), (P, TF, DF)),
                v_pages=bf16_normal(n("v"), (P, TF, DF)), masks=full_masks(P, pos))


def cfg_full_o(seed: int = 0, M: int = 1, tag: str = "fo") -> dict:
    """full_attention_output inputs: x [M, 16, 512] (un-normalised sums, ~ N(0, 4)), running sums
    [M, 16] in [1, 50), FP8 W_o [3840, 8192] with bf16 per-row scales, post-norm weight, residual."""
    n = lambda t: f"{tag}.seed{seed}.{t}"
    ow, os_ = fp8_weight(n("o"), H, QF)
    rs = (1.0 + 49.0 * _gen(n("sum")).random((M, GF))).astype(np.float32)
    return dict(x=bf16_normal(n("x"), (M, GF, DF), 4.0), running_sum=rs, post_attn_rms_weight=rms_weight(n("post"), H),
                o_weight=ow, o_weight_scale=_bf16_scales(os_), residual=bf16_normal(n("residual"), (M, H)))


def lm_head_bits(r):
    """bf16 lm_head values from random integers r in [0, 65536) (numpy or torch int32): the sign and
    mantissa bits of r, exponent 2^-5 .. 2^-2 from two more bits, so |w| lies in [1/32, 1/2) with an
    RMS of ~0.22. A unit-RMS input row then gives logits of std ~14, which spans the softcap's curve."""
    return (r & 0x807F) | ((122 + ((r >> 7) & 3)) << 7)


def cfg_logits(seed: int = 0, M: int = 1, tag: str = "logits") -> dict:
    """final_norm_and_logits inputs without the lm_head: input [M, 3840] ~ N(0, 1), the final norm's
    weight. The [262144, 3840] lm_head (2 GB) comes from lm_head_device or lm_head_rows."""
    n = lambda t: f"{tag}.seed{seed}.{t}"
    return dict(input=bf16_normal(n("input"), (M, H)), rms_weight=rms_weight(n("rms"), H))


def lm_head_rows(seed: int, rows: int, tag: str = "logits") -> np.ndarray:
    """A host lm_head of `rows` vocabulary rows (bf16 bits [rows, 3840]), for CPU-sized checks."""
    r = _gen(f"{tag}.seed{seed}.lm_head").integers(0, 1 << 16, size=(rows, H), dtype=np.int32)
    return lm_head_bits(r).astype(np.uint16)


def lm_head_device(seed: int, device="cuda"):
    """The full [262144, 3840] lm_head, drawn on the device (torch's generator; host generation of
    2 GB takes a minute), as an int16 tensor of bf16 bits."""
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    out = torch.empty((W, H), dtype=torch.int16, device=device)
    step = 16384
    for r0 in range(0, W, step):
        r = torch.randint(0, 1 << 16, (step, H), dtype=torch.int32, device=device, generator=g)
        b = lm_head_bits(r)
        out[r0:r0 + step] = torch.where(b >= 32768, b - 65536, b).to(torch.int16)
    return out


def cfg_ffn_mxfp4(seed: int = 0, M: int = 1, tag: str = "cfg3") -> dict:
    """Config 3: MXFP4 FFN (E2M1 + E8M0 per 32 along K)."""
    n = lambda t: f"{tag}.seed{seed}.{t}"
    up, su = mxfp4_weight(n("up"), L, H)
    gate, sg = mxfp4_weight(n("gate"), L, H)
    down, sd = mxfp4_weight(n("down"), H, L)
    return dict(residual=bf16_normal(n("residual"), (M, H)), pre_ff_rms_weight=rms_weight(n("pre_rms"), H),
                post_ff_rms_weight=rms_weight(n("post_rms"), H),
                layer_scalar=prng.f32_to_bf16_bits(np.full(8, LAYER_SCALAR, np.float32)),
                up_weight_packed=up, gate_weight_packed=gate, down_weight_packed=down,
                up_weight_scale=su, gate_weight_scale=sg, down_weight_scale=sd)
