"""Known-answer inputs of the reference's probe suites, rebuilt from their coordinate formulas.

Each builder follows the construction named in its docstring (paths under
moa-dev/experiments/candidates/ of the reference); the expected answers are the data files
under tests/golden/ (copied by tests/golden/extract_reference_fixtures.py).
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"
H, L, QS, PS, DS, TS, E = 3840, 15360, 4096, 2048, 256, 1024, 32768


def bf(values) -> np.ndarray:
    """f64/f32 values -> f32 -> bf16 bits, round half to even."""
    b = np.asarray(values, dtype=np.float64).astype(np.float32).view(np.uint32)
    return ((b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def unbf(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def load_json(name: str):
    return json.loads((GOLDEN / name).read_text())


# ------------------------------------------------------- QKV raw projection
def qkv_raw_case(case: int):
    """9 post-pre-RMS projection probes: qkv-fullh-weight-switch/boundary-suite/raw-src/generate.py:14-54.
    Returns x (bf16 bits [3840]) and, per matrix q/k/v, (codes [rows,3840], bf16 scale bits [rows])."""
    cols = 3840
    x = np.zeros(cols, np.float64)
    if case == 0:
        x[1::2] = -0.0
    elif case == 1:
        x[959] = 1.0
    elif case == 2:
        x[960] = -0.5
    elif case == 3:
        x[3839] = 1.5
    elif case in (4, 5):
        x[[0, 959, 960, 1919, 1920, 2879, 2880, 3839]] = [0.125, -0.25, 0.5, -0.75, 1.0, -0.5, 0.25, -0.125]
    elif case == 6:
        x[:] = 2.0 ** -22
        x[0::960] = 1.0
        x[1::960] = -1.0
    elif case == 7:
        x[0] = 1.0
        x[1] = 2.0 ** -8
    elif case == 8:
        x[:] = 129.0 * 2.0 ** -29
        x[0] = 1.0
        x[1] = -1.0
    mats = {}
    for which, (key, rows) in enumerate((("q", 4096), ("k", 2048), ("v", 2048))):
        r = np.arange(rows, dtype=np.int64)[:, None]
        k = np.arange(cols, dtype=np.int64)[None, :]
        local = rows // 128
        code = (0x38 + ((r * 3 + r // local + r // (rows // 2) + k + k // 960 + which) % 16)) | (((r + k // 960 + which) % 2) << 7)
        if case == 5:
            code = np.where(np.isin(r % local, [0, 1, local - 2, local - 1]), code, 0)
        elif case == 6:
            code = np.broadcast_to(np.where(k % 960 < 2, 0x38, 0x77), (rows, cols))
        elif case == 7:
            code = np.broadcast_to(0x38 + 8 * ((r + which) % 2), (rows, cols))
        elif case == 8:
            code = np.where(k < 2, 0x38, 0x77 | (((r // (rows // 2) + r % 2 + which) % 2) << 7))
        rr = np.arange(rows)
        s = np.ldexp(1.0 + ((rr + which) % 4) / 8.0, -(rr // 4 % 5))
        if case == 7:
            s = np.array([1.5, 1.25, 0.5, 0.0, 2.0 ** -10, 3.0, 0.75, 2.0])[(rr + which) % 8]
        if case == 8:
            s = np.ldexp(np.ones(rows), -((rr + which) % 5))
        mats[key] = (np.ascontiguousarray(np.broadcast_to(code, (rows, cols)), dtype=np.uint8), bf(s))
    return bf(x), mats


# --------------------------------------------------------- O raw projection
def o_raw_case(case: int):
    """8 O-projection probes: c09-output-first-npu/validation/probe-v1/generate.py:20-75.
    Returns x (bf16 bits [4096]), codes [3840,4096], bf16 scale bits [3840]."""
    rows = np.arange(H)
    x = np.zeros(QS, np.float64)
    scales = np.ldexp(1.0 + (rows % 4) / 8.0, -(rows // 4 % 5))
    if case == 0:
        x[1::2] = -0.0
    elif case == 1:
        x[255] = 1.0
    elif case == 2:
        x[256] = -0.5
    elif case == 3:
        x[4095] = 1.5
    elif case in (4, 5):
        x[[0, 255, 256, 511, 512, 2047, 2048, 4095]] = [0.125, -0.25, 0.5, -0.75, 1.0, -0.5, 0.25, -0.125]
    elif case == 6:
        x[:] = 2.0 ** -22
        x[0::256] = 1.0
        x[1::256] = -1.0
    else:
        x[0] = 1.0
        x[1] = 2.0 ** -8
        scales = np.array([1.5, 1.25, 0.5, 0.0, 2.0 ** -10, 3.0, 0.75, 2.0])[rows % 8]
    r = np.arange(H, dtype=np.int64)[:, None]
    k = np.arange(QS, dtype=np.int64)[None, :]
    code = (0x38 + ((r * 3 + r // 60 + r // 120 + r // 1920 + k + k // 256) % 16)) | (((r + k // 256) % 2) << 7)
    if case == 5:
        code = np.where(np.isin(r % 120, [0, 58, 59, 60, 61, 118, 119]), code, 0)
    elif case == 6:
        code = np.broadcast_to(np.where(k % 256 < 2, 0x38, 0x77), (H, QS))
    elif case == 7:
        code = np.broadcast_to(0x38 + 8 * (r % 2), (H, QS))
    return bf(x), np.ascontiguousarray(np.broadcast_to(code, (H, QS)), dtype=np.uint8), bf(scales)


# ------------------------------------------------------- O whole-op probes
def o_boundary_case(case: int) -> dict:
    """8 whole-operator O probes: output-boundary-probe-e47/generate_suite.py:37-108."""
    q = np.arange(QS)
    row = np.arange(H)
    scale = bf(np.ldexp(1.0, -(11 + row % 4)))
    gamma = bf((1 + row % 7) / 8.0)
    residual = bf((row % 5) / 8.0)
    x = np.zeros(QS, np.uint16)
    if case == 0:
        x[q % 2 == 1] = 0x8000
    elif case == 1:
        values = np.where((q // 256) % 2 == 0, 0.0, ((q % 17) - 8) / 16.0)
        for col, value in [(0, 0.125), (255, -0.25), (256, 0.5), (511, -0.75), (512, 0.25), (2047, -0.5),
                           (2048, 0.75), (4095, -0.125)]:
            values[col] = value
        x = bf(values)
        scale[[119, 120, 1919, 1920, 3839]] = bf([2.0 ** -10, 2.0 ** -11, 2.0 ** -12, 2.0 ** -13, 2.0 ** -14])
    elif case in (2, 3, 4):
        for group in range(16):
            exponent = -7 + group % 8
            anchor = int(bf([2.0 ** exponent])[0]) + case - 3
            a = float(unbf(np.array([anchor], np.uint16))[0])
            vals = np.array([a * ((i % 15) - 7) / 16 for i in range(256)], dtype=np.float32)
            vals[0] = a
            vals[255] = -a
            x[group * 256:(group + 1) * 256] = bf(vals)
    elif case == 5:
        for group in range(16):
            exponent = -6 + group % 7
            values = np.zeros(256, np.uint16)
            values[0] = bf([2.0 ** exponent])[0]
            for offset, power in ((1, exponent - 13), (7, exponent - 21)):
                middle = int(bf([2.0 ** power])[0])
                for j, delta in enumerate((-1, 0, 1)):
                    values[offset + j] = middle + delta
                    values[offset + j + 3] = (middle + delta) | 0x8000
            values[16:] = np.repeat(values[1:13], 20)
            x[group * 256:(group + 1) * 256] = values
    elif case == 6:
        x = ((q * 37) % 0x400).astype(np.uint16)
        x[q % 2 == 1] |= 0x8000
        x[0], x[1], x[2] = 0x0001, 0x0080, 0x03FF
        gamma[:] = 0x3F80
        residual[:] = 0
    elif case == 7:
        x = bf(np.full(QS, 2.0 ** -22))
        x[0::256], x[1::256] = 0x3F80, 0xBF80
        scale[:] = 0x3A80
        gamma[:] = 0x3F00
        residual[:] = 0x3F00
    r = np.arange(H, dtype=np.int64)[:, None]
    qq = np.arange(QS, dtype=np.int64)[None, :]
    if case == 7:
        codes = np.broadcast_to(np.where(qq % 256 < 2, 0x38, 0x77), (H, QS))
    else:
        exponent = 7 + ((r // 120 + qq // 256 + case) % 8)
        mantissa = (3 * r + qq + qq // 16) % 8
        sign = ((r // 8 + qq // 32 + qq % 3 + case) % 2) << 7
        codes = sign | (exponent << 3) | mantissa
    return dict(x=x, o_weight=np.ascontiguousarray(codes, dtype=np.uint8), o_weight_scale=scale,
                post_attn_rms_weight=gamma, residual=residual)


# --------------------------------------------------------- QKV whole-op probes
def qkv_boundary_case(case: int) -> dict:
    """2 whole-operator QKV probes (qkv-boundary-probe-e53/generate_suite.py:24-105): small inputs
    from the fixture file; weight rows [1,1,478 x 240] repeated per 480 columns."""
    from safetensors.numpy import load_file

    d = load_file(str(GOLDEN / "qkv_boundary.safetensors"))
    g = lambda k: d[f"case{case}.input.{k}"]
    rope_off = int(g("rope_offset").view(np.int32)[0])
    kv_off = int(g("kv_offset").view(np.int32)[0])
    pos = rope_off // (DS * 2)
    cos = np.zeros((E, DS), np.uint16)
    sin = np.zeros((E, DS), np.uint16)
    cos[pos] = g("cos_row").view(np.uint16)
    sin[pos] = g("sin_row").view(np.uint16)
    row = np.where(np.arange(H) % 480 < 2, 0x38, 0x77).astype(np.uint8)
    return dict(
        x=g("x").view(np.uint16).copy(), input_rms_weight=g("input_rms_weight").view(np.uint16).copy(),
        q_rms_weight=g("q_rms_weight").view(np.uint16).copy(), k_rms_weight=g("k_rms_weight").view(np.uint16).copy(),
        q_weight=np.broadcast_to(row, (QS, H)).copy(), k_weight=np.broadcast_to(row, (PS, H)).copy(),
        v_weight=np.broadcast_to(row, (PS, H)).copy(),
        q_weight_scale=g("q_weight_scale").view(np.uint16).copy(),
        k_weight_scale=g("k_weight_scale").view(np.uint16).copy(),
        v_weight_scale=g("v_weight_scale").view(np.uint16).copy(),
        cos=cos, sin=sin, rope_offset=rope_off, kv_offset=kv_off, pos=pos,
        k_cache=np.full((TS, 8, DS), 0x3E80, np.uint16), v_cache=np.full((TS, 8, DS), 0xBF00, np.uint16),
        q_out=np.full(QS, 0x3FC0, np.uint16),
        expected={k: d[f"case{case}.expected.{k}"] for k in ("q", "k", "v")},
        checksums={k.split(".")[-1]: int(v[0]) for k, v in d.items() if k.startswith(f"case{case}.checksum.")},
    )


# ------------------------------------------------------------- FFN stress
def ffn_stress_inputs() -> dict:
    """NVFP4 full-FFN cancellation probe: ffn-native-down-weighted-residual/full-ffn-stress/
    generate_reference.py:34-92. Known answer: 3840 x bf16 0x3ecf (0.404296875)."""
    ones = np.full(H, 0x3F80, np.uint16)
    out = dict(residual=ones.copy(), pre_ff_rms_weight=ones.copy(), post_ff_rms_weight=ones.copy(),
               layer_scalar=np.full(8, 0x3EC0, np.uint16))  # bf16(0.375)
    scale_code = {2.0: 0x40, 4.0: 0x48, 15.0: 0x57}  # E4M3 codes of the local scales
    for name in ("up", "gate", "down"):
        shape = (L, H) if name != "down" else (H, L)
        codes = np.zeros(shape, np.uint8)
        scale = np.full((shape[0], shape[1] // 16), 2.0 if name != "down" else 15.0)
        if name == "up":
            codes[:, 0] = 1
            codes[0, :] = 0
            codes[0, :2730] = 7
            codes[0, 2730] = 6
            codes[7680, :] = 0
            codes[7680, :5] = 7
            codes[7680, 5] = 4
        elif name == "gate":
            codes[:, 0] = 2
            codes[0, :] = 0
            codes[0, :2730] = 7
            codes[0, 2730] = 6
            codes[7680, :] = 0
            codes[7680, :682] = 7
            codes[7680, 682] = 6
        else:
            codes[:1920, 1:7680] = 7
            codes[1920:, 7681:15360] = 7
        if name != "down":
            scale[[0, 7680], :] = 4.0
        out[f"{name}_weight_packed"] = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
        out[f"{name}_weight_scale"] = np.vectorize(scale_code.get)(scale).astype(np.uint8)
        out[f"{name}_global_scale"] = np.array([2.0 ** -11], np.float32)
    return out


def ffn_stress_inputs_fp8() -> dict:
    """The full-FFN stress construction (full-ffn-stress/generate_reference.py:34-92) restated for
    E4M3 weights with per-row f32 scales. Every projection reproduces the NVFP4 case's values:
    ordinary up/gate rows 2^-11 / 2^-10, rows 0 and 7680 up 32 / 2^-4 and gate 32 / 8, so the
    GeGLU row is p[0] = 1024, p[7680] = 0.5 and 2^-22 elsewhere; the down rows skip columns 0 and
    7680 (the large p) and sum 7679 x 2^-22 x 90 x 2^-11 = 691110 x 2^-33, whose bf16 is
    169 x 2^-21, the NVFP4 case's d. Rows 0 and 7680 and the odd down rows carry other scales
    than their neighbours (their codes compensate), so a row-scale index error changes the
    answer. Expected output: 3840 x 0x3ecf, the reference's recorded answer."""
    ones = np.full(H, 0x3F80, np.uint16)
    out = dict(residual=ones.copy(), pre_ff_rms_weight=ones.copy(), post_ff_rms_weight=ones.copy(),
               layer_scalar=np.full(8, 0x3EC0, np.uint16))
    E4 = {1.0: 0x38, 2.0: 0x40, 3.0: 0x44}
    for name, big_row in (("up", 5), ("gate", 682)):
        codes = np.zeros((L, H), np.uint8)
        scale = np.full(L, 2.0 ** -11, np.float32)
        codes[:, 0] = E4[1.0] if name == "up" else E4[2.0]
        # rows 0 and 7680 at scale 2^-8: 2730 x 3 + 2 = 8192 -> 32; 5 x 3 + 1 = 16 -> 2^-4 (up);
        # 682 x 3 + 2 = 2048 -> 8 (gate)
        codes[0, :] = 0
        codes[0, :2730] = E4[3.0]
        codes[0, 2730] = E4[2.0]
        codes[7680, :] = 0
        codes[7680, :big_row] = E4[3.0]
        codes[7680, big_row] = E4[1.0] if name == "up" else E4[2.0]
        scale[[0, 7680]] = 2.0 ** -8
        out[f"{name}_weight"], out[f"{name}_weight_scale"] = codes, scale
    codes = np.zeros((H, L), np.uint8)
    codes[:1920, 1:7680] = E4[1.0]
    codes[1920:, 7681:] = E4[1.0]
    scale = np.full(H, 90 * 2.0 ** -11, np.float32)
    codes[1::2][codes[1::2] != 0] = E4[2.0]  # odd rows: weight 2, scale 45 x 2^-11
    scale[1::2] = 45 * 2.0 ** -11
    out["down_weight"], out["down_weight_scale"] = codes, scale
    return out


def ffn_stress_inputs_mxfp4() -> dict:
    """The full-FFN stress construction restated for E2M1 weights with E8M0 block-32 scales (no
    global scale: proj = bf16(h . W)). Same intermediates as the NVFP4 case (see
    ffn_stress_inputs_fp8). Rows 0 and 7680 of up/gate alternate their block scales 2^-9 / 2^-8
    with codes 6 / 3, so every element is 3 x 2^-8 whichever block it is in; the down rows take
    block scales 2^-7, 2^-6, 2^-5 in turn, each element 3/64 (6274 columns) or 1/32 (1405),
    which sums to exactly 338 x 2^-22 = 169 x 2^-21. A wrong block index or E8M0 bias changes the
    answer. Expected output: 3840 x 0x3ecf."""
    ones = np.full(H, 0x3F80, np.uint16)
    out = dict(residual=ones.copy(), pre_ff_rms_weight=ones.copy(), post_ff_rms_weight=ones.copy(),
               layer_scalar=np.full(8, 0x3EC0, np.uint16))
    pack = lambda c: (c[:, 0::2] | (c[:, 1::2] << 4)).astype(np.uint8)
    for name in ("up", "gate"):
        codes = np.zeros((L, H), np.uint8)
        sc = (127 + (np.arange(H // 32) % 5)[None, :] + np.zeros((L, 1), np.int64)).astype(np.uint8)
        codes[:, 0] = 1 if name == "up" else 2  # 0.5 / 1.0 x 2^-10
        sc[:, 0] = 127 - 10
        for row, n in ((0, 2730), (7680, 5 if name == "up" else 682)):
            codes[row, :] = 0
            blk = np.arange(H) // 32
            sc[row] = np.where(np.arange(H // 32) % 2 == 0, 127 - 9, 127 - 8)
            codes[row, :n] = np.where(blk[:n] % 2 == 0, 7, 5)  # 6 x 2^-9 = 3 x 2^-8
            # the last element: 2^-7 (to 32 / 8) or, up row 7680 (block 0, 2^-9), 2^-8 (to 2^-4)
            codes[row, n] = 4  # 2.0 x the block's scale
        out[f"{name}_weight_packed"], out[f"{name}_weight_scale"] = pack(codes), sc
    codes = np.zeros((H, L), np.uint8)
    e = np.arange(L // 32) % 3  # block scale 2^(-7 + e)
    big, small = np.array([7, 5, 3])[e], np.array([6, 4, 2])[e]  # 3/64 and 1/32 at each scale
    col_blk = np.arange(L) // 32
    for rows, c0 in ((slice(0, 1920), 1), (slice(1920, H), 7681)):
        codes[rows, c0:c0 + 6274] = big[col_blk[c0:c0 + 6274]]
        codes[rows, c0 + 6274:c0 + 7679] = small[col_blk[c0 + 6274:c0 + 7679]]
    out["down_weight_packed"] = pack(codes)
    out["down_weight_scale"] = np.broadcast_to((127 - 7 + e).astype(np.uint8), (H, L // 32)).copy()
    return out


def sign_failures(expected_f32: np.ndarray, actual_f32: np.ndarray, atol: float) -> np.ndarray:
    """BASELINE's "no sign-cancellation failures": where the expected value is at least atol in
    magnitude, the output must carry its sign. (The atol/rtol bound alone lets an output flip sign
    when |e| lies in [atol, atol / (1 - rtol)).) Returns the mask of failing elements."""
    e = np.asarray(expected_f32, np.float32).reshape(-1)
    a = np.asarray(actual_f32, np.float32).reshape(-1)
    return (np.abs(e) >= atol) & (np.signbit(a) != np.signbit(e)) & (a != 0)


def compare(expected_f32: np.ndarray, actual_bits: np.ndarray, atol: float, rtol: float = 1e-2):
    """The reference's gate (FO/src/bin/test_kernels.rs:626-671): every element finite and
    |a - e| <= atol + rtol |e|; plus the sign rule of sign_failures (a non-zero output of the
    wrong sign where |e| >= atol fails, and so does a zero output there: it fails the bound).
    Returns (ok, max_abs_diff, n_exact, n_fail)."""
    e = np.asarray(expected_f32, np.float32).reshape(-1)
    a = unbf(np.asarray(actual_bits).reshape(-1).view(np.uint16))
    if not np.all(np.isfinite(a)):
        return False, float("inf"), 0, int(np.count_nonzero(~np.isfinite(a)))
    diff = np.abs(a - e)
    fail = (diff > atol + rtol * np.abs(e)) | sign_failures(e, a, atol)
    return (not fail.any()), float(diff.max(initial=0.0)), int(np.count_nonzero(diff == 0)), int(fail.sum())
