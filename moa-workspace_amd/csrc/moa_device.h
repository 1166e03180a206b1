// moa_device.h -- device-side helpers shared by the gfx950 kernels.
//
// Number formats follow the reference's oracle exactly:
//   bf16 <-> f32 is round-half-to-even on the raw bits (FO/scripts/fixture_prng.py:80-90);
//   E4M3FN codes widen exactly (FO/scripts/generate_references.py:152);
//   E2M1 nibbles are low-nibble-first, magnitude {0,.5,1,1.5,2,3,4,6} (generate_references.py:69,154-163).
// The file is compiled with -ffp-contract=off: every multiply and add rounds on its own
// unless a kernel calls fmaf() where the product is exact (bf16 x fp8/fp4 products are).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "moa_shapes.h"

namespace moa {

constexpr int kWave = 64;

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ bf16
__device__ __forceinline__ float bf2f(uint32_t b16) { return __uint_as_float(b16 << 16); }

// f32 -> bf16 bits, round half to even: one v_cvt_pk_bf16_f32. For every non-NaN f32 it gives
// the bits of rounding the raw f32 bits, (b + 0x7fff + lsb) >> 16 (fixture_prng.py:80-90; the
// format self-test checks every bf16 high half with ties, near-ties and subnormals); a NaN
// stays a (quiet) NaN.
__device__ __forceinline__ uint32_t f2bf(float v) { return __builtin_bit_cast(uint16_t, (__bf16)v); }

// Two f32 to packed bf16 (lo in the low half), rounded as f2bf: one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2_t));
}

// Round an f32 through bf16 and back (the per-op bf16 commit of a torch bf16 tensor op).
__device__ __forceinline__ float rbf(float v) { return bf2f(f2bf(v)); }

// Eight packed bf16 (one 16-byte load) to f32.
__device__ __forceinline__ void bf16x8_to_f32(const uint4& q, float* o) {
    o[0] = __uint_as_float(q.x << 16); o[1] = __uint_as_float(q.x & 0xffff0000u);
    o[2] = __uint_as_float(q.y << 16); o[3] = __uint_as_float(q.y & 0xffff0000u);
    o[4] = __uint_as_float(q.z << 16); o[5] = __uint_as_float(q.z & 0xffff0000u);
    o[6] = __uint_as_float(q.w << 16); o[7] = __uint_as_float(q.w & 0xffff0000u);
}

// ---------------------------------------------------------- fp8 / fp4 decode
// gfx950 converts OCP E4M3FN in hardware; two codes per instruction.
__device__ __forceinline__ void fp8x4_to_f32(uint32_t w, float* o) {
    f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
    f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(w, true);
    o[0] = lo[0]; o[1] = lo[1]; o[2] = hi[0]; o[3] = hi[1];
}

// Eight E2M1 nibbles of one dword (low nibble = lower element index), each times `scale`.
// The hardware uses only the exponent of `scale` (a power-of-two MX scale); pass 1.0f for
// plain decoding.
__device__ __forceinline__ void fp4x8_to_f32(uint32_t w, float scale, float* o) {
    f32x2 a = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, scale, 0);
    f32x2 b = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, scale, 1);
    f32x2 c = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, scale, 2);
    f32x2 d = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, scale, 3);
    o[0] = a[0]; o[1] = a[1]; o[2] = b[0]; o[3] = b[1];
    o[4] = c[0]; o[5] = c[1]; o[6] = d[0]; o[7] = d[1];
}

// ------------------------------------------------- bf16 dot products (FFN)
// Activations stay bf16, two per dword (lower element in the low half); weights widen to bf16
// exactly (E4M3 and E2M1 values are bf16 values; the conversions run at scale 1) and
// v_dot2c_f32_bf16 accumulates acc + a.lo*b.lo + a.hi*b.hi in f32 -- bf16 x bf16 products are
// exact in f32, so only the accumulation order differs from a chain of fmaf().
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2_bf16(uint32_t x2, bf16x2 w2, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x2), w2, acc, false);
}

// 16 E4M3 codes (a 16-byte chunk) against 16 activations x[0..8) (pairs).
__device__ __forceinline__ float dot_fp8x16_bf16(const uint32_t* x, const uint4& q, float acc) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        acc = dot2_bf16(x[2 * i], __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[i], 1.0f, false), acc);
        acc = dot2_bf16(x[2 * i + 1], __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[i], 1.0f, true), acc);
    }
    return acc;
}

// 8 E2M1 codes (one dword, low nibble first) against 8 activations x[0..4) (pairs).
__device__ __forceinline__ float dot_fp4x8_bf16(const uint32_t* x, uint32_t w, float acc) {
    acc = dot2_bf16(x[0], __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 0), acc);
    acc = dot2_bf16(x[1], __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 1), acc);
    acc = dot2_bf16(x[2], __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 2), acc);
    acc = dot2_bf16(x[3], __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 3), acc);
    return acc;
}

__device__ __forceinline__ float e4m3_to_f32(uint32_t code) {
    return __builtin_amdgcn_cvt_pk_f32_fp8(code & 0xffu, false)[0];
}

// E8M0 exponent -> 2^(e-127) as f32 (0xff is NaN in OCP MX; callers never pass it).
__device__ __forceinline__ float e8m0_to_f32(uint32_t e) {
    e &= 0xffu;
    return e == 0 ? __uint_as_float(0x00400000u) : __uint_as_float(e << 23);
}

// ------------------------------------------------------------- reductions
// xor butterfly: every lane ends with the same bits (f32 add is commutative).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// ----------------------------------------------------------------- loads
// Weights are read exactly once per call: stream them non-temporally.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream(const void* p) {
    u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

// torch.rsqrt on CPU is 1/sqrt with both steps correctly rounded (gemma4.py:86).
__device__ __forceinline__ float rms_inverse(float sum_sq, int n) {
    float mean = __fdiv_rn(sum_sq, (float)n);
    return __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean, kEps)));
}

// tanh(u) = sign(u) (1 - 2 / (1 + e^(2|u|))) in f32 without branches: e^(2|u|) = 2^(2|u| log2 e)
// from v_exp_f32, 1 / (1 + e^(2|u|)) from v_rcp_f32 refined by one Newton step (r + r (1 - d r)).
// A library tanhf branches on |u|, which serialises element-wise loops. For |u| beyond ~9 the
// quotient vanishes next to 1, so the result is exactly +-1 as with f32 tanhf.
__device__ __forceinline__ float tanh_f32(float u) {
    const float d = 1.0f + __builtin_amdgcn_exp2f(fabsf(u) * 2.8853900817779268f);
    const float r0 = __builtin_amdgcn_rcpf(d);
    const float r = __builtin_isinf(d) ? 0.0f : fmaf(r0, fmaf(-d, r0, 1.0f), r0);
    return copysignf(1.0f - 2.0f * r, u);
}

// torch gelu(approximate="tanh") in f32 (gemma4.py:197): 0.5 x (1 + tanh(u)),
// u = sqrt(2/pi) (x + 0.044715 x^3). Over all 65536 bf16 inputs it rounds to the same bf16 as
// the f32 formula with libm tanhf.
__device__ __forceinline__ float gelu_tanh(float x) {
    const float kBeta = 0.7978845608028654f;
    const float kKappa = 0.044715f;
    const float cube = x * x * x;
    const float inner = kBeta * (x + kKappa * cube);
    return 0.5f * x * (1.0f + tanh_f32(inner));
}

// tanh with a small relative error over the whole range: for |u| < 0.25 the odd Taylor series to
// u^11 (truncation below 3e-10 relative), elsewhere tanh_f32, whose 1 - 2 / d loses at most about
// 1e-7 absolute, 5e-7 relative at |u| = 0.25. Both are evaluated; the select is branch-free.
__device__ __forceinline__ float tanh_rel_f32(float u) {
    const float u2 = u * u;
    float p = fmaf(u2, -8.8632355299021966e-3f, 2.1869488536155203e-2f);  // -1382/155925, 62/2835
    p = fmaf(u2, p, -5.3968253968253968e-2f);                              // -17/315
    p = fmaf(u2, p, 1.3333333333333333e-1f);                               // 2/15
    p = fmaf(u2, p, -3.3333333333333333e-1f);                              // -1/3
    p = fmaf(u2 * u, p, u);
    return fabsf(u) < 0.25f ? p : tanh_f32(u);
}

// Gemma's final-logit softcap on a bf16 logit l (FO/src/ops.rs:256-293): l is widened to f32,
// divided by 30, tanh'd, multiplied by 30 and rounded once to bf16. (The torch CPU model,
// gemma4.py:260-261, rounds to bf16 after each of the three ops; the two differ by at most a
// couple of bf16 ulps.)
__device__ __forceinline__ uint32_t softcap30_bf16(float l) {
    return f2bf(tanh_rel_f32(l / 30.0f) * 30.0f);
}

}  // namespace moa
