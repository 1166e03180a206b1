// moa_rows.hip -- decoder_feedforward for 2..16 token rows on the matrix cores (all three formats).
//
// The per-row decode kernels stream every weight once per token row. Here every weight byte is
// read once for all rows of the call: the rows, padded to 16, are the A operand of
// v_mfma_f32_16x16x32_bf16 and 16 weight rows, widened to bf16 in registers, are the B operand.
// The widening is exact: E4M3 and E2M1 values are bf16 values, an E2M1 value times its E8M0
// block scale (MXFP4) is a power-of-two multiple of one, and an E2M1 value times its E4M3 block
// scale (NVFP4) has at most six significant bits -- so the products are exactly those of the
// reference's per-element dequantisation (generate_references.py:383-414) and only the f32
// accumulation order differs. The steps:
//   pre-norm   h = bf16(RMSNorm(x) * w) of the M residual rows (gemma4.py:83-89)
//   up/gate    per workgroup: h into LDS, 64 up and the same 64 gate rows over all of H, and the
//              GeGLU epilogue -> p [M][L] bf16 (gemma4.py:189-197)
//   down       per workgroup: p[:, 3840 q .. +3840] into LDS, 64 down rows over that quarter of
//              L -> f32 partial sums [4][M][H]
//   post       sum of the partials, the format's commit, post-RMSNorm, residual and layer scalar
//              (rmsnorm.rs:204-296, residual.rs:189-241)
// The pre-norm is a launch of its own; up/gate, down and post run in one launch
// (rows_fused_kernel) where its grid fits on the device at once, with tagged flags between the
// steps, else as three launches (rows_kernel twice, then chunk_post_rows_kernel), with the same
// bits. (An earlier one-launch form with grid barriers between the steps, each step's first
// weight loads issued before its barrier, measured no faster than the launches.)
#include <hip/hip_runtime.h>

#include <atomic>

#include "moa_device.h"
#include "moa_internal.h"
#include "moa_post_row.h"
#include "moa_sync.h"

namespace moa {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 rw_bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kRwTile = 16;                    // weight rows per wave (the MFMA's N)
constexpr int kRwGroupRows = 4 * kRwTile;      // weight rows per workgroup
constexpr int kRwK = 3840;                     // k per workgroup: all of H (up/gate), a quarter of L (down)
// 16-byte LDS units per activation row of k range KR, one of them padding (so that 16 rows start on
// distinct LDS banks), and the LDS of 16 such rows
template <int KR>
constexpr int rw_row_units() { return KR / 8 + 1; }
template <int KR>
constexpr int rw_lds_units() { return (kMaxDecodeM * rw_row_units<KR>() + 63) / 64 * 64; }
constexpr int kRwSplits = kL / kRwK;           // down: four k quarters
constexpr int kRwUpGroups = kL / kRwGroupRows;      // 240 up/gate workgroups
constexpr int kRwDownGroups = kH / kRwGroupRows;    // 60 down column groups (x 4 quarters)
constexpr int kRwNH = 2;                       // k parts per workgroup: 8 compute waves
static_assert(kH == kRwK && kL == kRwSplits * kRwK, "one workgroup k range");
static_assert(kL % kRwGroupRows == 0 && kH % kRwGroupRows == 0, "whole weight tiles");
static_assert(kRwDownGroups * kRwSplits == kRwUpGroups, "one grid for both contractions");
static_assert((rw_row_units<kRwK>() * 4) % 64 == 4, "row stride: 16 rows start on distinct LDS banks");

// k covered by one 16-byte weight load of each lane (FP8: 16 codes; FP4: 32 codes), and the
// wave's load step (four lane groups side by side).
template <FfnFormat F>
constexpr int rw_lane_k() { return F == FfnFormat::FP8 ? 16 : 32; }
template <FfnFormat F>
constexpr int rw_step_k() { return 4 * rw_lane_k<F>(); }

// 8 E4M3 codes (two dwords, lower index in the low byte) widened to 8 bf16.
__device__ __forceinline__ bf16x8 rw_fp8x8(uint32_t lo, uint32_t hi) {
    const rw_bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
    const rw_bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
    const rw_bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
    const rw_bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
    return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// Load step `s` of a lane's stream: 16 weight bytes at w + 64 s. Ordinary (not non-temporal) loads:
// each 128-byte line is requested by two steps, and a streaming hint lets the first request's line
// leave the cache before the second arrives (measured: 15-20 % slower).
__device__ __forceinline__ uint4 rw_issue(const uint8_t* w, int s) { return ld16(w + s * 64); }

// The lane's B fragment j (8 consecutive k of its load q) as bf16. sc: MXFP4 the block's E8M0
// code in bits 23-30 (an f32 whose exponent field is the code), NVFP4 the two blocks' E4M3 codes
// (the lower one in the low byte).
template <FfnFormat F>
__device__ __forceinline__ bf16x8 rw_weights(const uint4& d, uint32_t sc, int j) {
    const uint32_t q[4] = {d.x, d.y, d.z, d.w};
    if constexpr (F == FfnFormat::FP8) {
        return rw_fp8x8(q[2 * j], q[2 * j + 1]);
    } else if constexpr (F == FfnFormat::MXFP4) {
        // the conversion applies the exponent field of its f32 scale: E8M0 code e -> 2^(e - 127)
        const float s = __uint_as_float(sc);
        const rw_bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q[j], s, 0);
        const rw_bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q[j], s, 1);
        const rw_bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q[j], s, 2);
        const rw_bf16x2 e = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q[j], s, 3);
        return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], e[0], e[1]};
    } else {
        // E2M1 x E4M3 in f32 (exact), whose low 16 bits are then zero: the bf16 is the high half
        const float s = e4m3_to_f32(sc >> (8 * (j >> 1)));
        float v[8];
        fp4x8_to_f32(q[j], 1.0f, v);
        uint32_t u[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            u[i] = __builtin_amdgcn_perm(__float_as_uint(v[2 * i + 1] * s), __float_as_uint(v[2 * i] * s), 0x07060302u);
        return __builtin_bit_cast(bf16x8, make_uint4(u[0], u[1], u[2], u[3]));
    }
}

template <ScaleKind SK>
__device__ __forceinline__ float rw_row_scale(const void* p, int i) {
    if constexpr (SK == ScaleKind::F32) return static_cast<const float*>(p)[i];
    else return bf2f(static_cast<const uint16_t*>(p)[i]);
}

// Projection commit with the format's rounding rule:
//   FP8:   bf16(dot * s_row)              generate_references.py:265-274
//   NVFP4: bf16(bf16(dot) * inv_global)   generate_references.py:358-372
//   MXFP4: bf16(dot)
template <FfnFormat F>
__device__ __forceinline__ float rw_commit(float dot, float scale) {
    if constexpr (F == FfnFormat::FP8) return rbf(dot * scale);
    else if constexpr (F == FfnFormat::NVFP4) return rbf(rbf(dot) * scale);
    else return rbf(dot);
}

// Workgroup barrier on LDS: this wave's LDS operations are complete and (N >= 0) all but its last
// N global loads have arrived (N = 0: every load, including loads into LDS). With N < 0 global
// loads stay in flight across the barrier (__syncthreads() would wait for them).
template <int N>
__device__ __forceinline__ void rw_lds_barrier() {
    static_assert(N < 64, "vmcnt range");
    if constexpr (N >= 0) __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}

// Launch shape per format and kind: NH parts of the workgroup's k range (4 NH waves: four 16-row
// tiles x NH parts); D, the load steps of each wave's ring; B, the steps refilled at once (every B
// steps, so that B consecutive 64-byte pieces of each weight row are requested back to back).
template <FfnFormat F, bool G>
struct RwShape {
    static constexpr int NH = kRwNH;
    static constexpr int D = 8;
    static constexpr int B = 4;
};

// One wave's weight stream: a 16-row tile (GeGLU: of up and of gate) over one part of the
// workgroup's k range KR, the FP4 block-scale codes of that range, and the ring of loads.
// DD: the ring's depth (the launch shape's by default; the one-launch kernel's down stream issues
// DD - B steps ahead, up to all of them).
template <FfnFormat F, bool G, int KR = kRwK, int DD = RwShape<F, G>::D>
struct RwStream {
    static constexpr int NM = G ? 2 : 1;
    static constexpr int NH = RwShape<F, G>::NH, D = DD, B = RwShape<F, G>::B;
    static constexpr int LK = rw_lane_k<F>(), SKK = rw_step_k<F>();
    static constexpr int KW = KR / NH;    // k per wave
    static constexpr int S = KW / SKK;    // load steps per wave
    static constexpr int EPB = F == FfnFormat::FP8 ? 1 : 2;                                    // elements per byte
    static constexpr int BLK = F == FfnFormat::MXFP4 ? 32 : (F == FfnFormat::NVFP4 ? 16 : 1);  // scale block
    static_assert(KW % SKK == 0 && B >= 1 && D > B, "stream shape");
    const uint8_t* wp[NM];
    uint32_t sd[NM][S];  // FP4: one dword per step (MXFP4: four lane groups' E8M0 codes; NVFP4: this
                         // lane group pair's two pairs of E4M3 codes)
    uint4 ring[D][NM];
};

// The stream of lane (r, g) for weight rows n0 .. n0 + 15 of w0 (and w1), k kb .. kb + KW of rows
// of wk elements: the scale codes, then the first D - B load steps.
template <FfnFormat F, bool G, int KR, int DD>
__device__ __forceinline__ void rw_prefetch(RwStream<F, G, KR, DD>& st, const uint8_t* w0, const uint8_t* w1, const void* s0,
                                            const void* s1, int wk, int n0, int kb, int r, int g) {
    using T = RwStream<F, G, KR, DD>;
#pragma unroll
    for (int k = 0; k < T::NM; ++k) {
        st.wp[k] = (k ? w1 : w0) + (size_t)(n0 + r) * (wk / T::EPB) + kb / T::EPB + 16 * g;
        if constexpr (F != FfnFormat::FP8) {
            const uint8_t* srow = static_cast<const uint8_t*>(k ? s1 : s0) + (size_t)(n0 + r) * (wk / T::BLK) + kb / T::BLK;
#pragma unroll
            for (int s = 0; s < T::S; ++s) {
                if constexpr (F == FfnFormat::MXFP4) st.sd[k][s] = *reinterpret_cast<const uint32_t*>(srow + 4 * s);
                else st.sd[k][s] = *reinterpret_cast<const uint32_t*>(srow + 8 * s + 4 * (g >> 1));
            }
        }
    }
#pragma unroll
    for (int i = 0; i < T::D - T::B; ++i)
        if (i < T::S) {
#pragma unroll
            for (int k = 0; k < T::NM; ++k) st.ring[i][k] = rw_issue(st.wp[k], i);
        }
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rw_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// Activation rows 0 .. M-1 of x (row stride ldx, columns kz ..) staged into LDS by NT threads
// through registers: LDS unit u (16 bytes) is row u / 481, element 8 (u % 481); the padding unit
// and rows past M hold zeros. The loads go out first (rw_rows_load), the weight ring next, and the
// LDS stores (rw_rows_store) then wait for these loads only -- loads complete in order, so the
// ring stays in flight (a load straight into LDS would need a wait for every load).
template <int NT, int KR = kRwK>
struct RwRows {
    static constexpr int RU = rw_row_units<KR>();
    static constexpr int N = (kMaxDecodeM * RU + NT - 1) / NT;
    uint4 v[N];
};

// With div (full-attention output: the running softmax sums [M][16] of the 512-element heads), each
// element becomes bf16(x / sum), or zero where the sum is not positive -- as the per-row kernels'
// o_input_chunk.
template <int NT, int KR>
__device__ __forceinline__ void rw_rows_load(RwRows<NT, KR>& st, const uint16_t* x, int ldx, int kz, int M, int t,
                                             const float* div = nullptr) {
    using R = RwRows<NT, KR>;
    const __amdgpu_buffer_rsrc_t rs = rw_rsrc(x, (uint32_t)(sizeof(uint16_t) * (size_t)M * ldx));
#pragma unroll
    for (int i = 0; i < R::N; ++i) {
        const int u = t + NT * i, m = u / R::RU, c = u % R::RU;
        const bool ok = m < M && c < KR / 8;
        const uint4 v = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, ok ? (int)(sizeof(uint16_t) * (m * ldx + kz + c * 8)) : 0, 0, 0));
        st.v[i] = ok ? v : make_uint4(0, 0, 0, 0);
    }
    if (div) {
#pragma unroll
        for (int i = 0; i < R::N; ++i) {
            const int u = t + NT * i, m = u / R::RU, c = u % R::RU;
            if (m < M && c < KR / 8) {
                const float d = div[m * kGf + (kz + c * 8) / kDf];
                float f[8];
                bf16x8_to_f32(st.v[i], f);
                uint32_t h[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    h[e] = pk_bf16(d > 0.0f ? f[2 * e] / d : 0.0f, d > 0.0f ? f[2 * e + 1] / d : 0.0f);
                st.v[i] = make_uint4(h[0], h[1], h[2], h[3]);
            }
        }
    }
}

template <int NT, int KR>
__device__ __forceinline__ void rw_rows_store(const RwRows<NT, KR>& st, uint4* xs, int t) {
    using R = RwRows<NT, KR>;
#pragma unroll
    for (int i = 0; i < R::N; ++i) {
        const int u = t + NT * i;
        if (u < kMaxDecodeM * R::RU) xs[u] = st.v[i];
    }
    rw_lds_barrier<-1>();
}

// The stream against the LDS rows, unrolled over its S load steps: every B steps, step s first
// refills the ring slots read in steps s - B .. s - 1 (with steps s + D - B .. s + D - 1), then
// each step runs its MFMAs. MFMA j of a step takes the lane's k 8 j .. 8 j + 7 of its load -- for
// A (LDS row r) and B alike, a fixed permutation of the step's k. acc[k][e]: row 4 g + e, weight
// row r of the tile.
template <FfnFormat F, bool G, int KR, int DD>
__device__ __forceinline__ void rw_mma(RwStream<F, G, KR, DD>& st, const uint4* xs, f32x4 (&acc)[G ? 2 : 1], int part, int r,
                                       int g) {
    using T = RwStream<F, G, KR, DD>;
    constexpr int D = T::D, B = T::B, S = T::S;
#pragma unroll
    for (int k = 0; k < T::NM; ++k) acc[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int abase = r * rw_row_units<KR>() + (part * T::KW + g * T::LK) / 8;
    const uint32_t gsh = F == FfnFormat::MXFP4 ? 8 * g : 16 * (g & 1);  // this lane group's code(s) in sd
#pragma unroll
    for (int s = 0; s < S; ++s) {
        if (s % B == 0) {
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const int sn = s + D - B + b;
                if (sn < S) {
#pragma unroll
                    for (int k = 0; k < T::NM; ++k) st.ring[sn % D][k] = rw_issue(st.wp[k], sn);
                }
            }
        }
        uint32_t sc[T::NM];
#pragma unroll
        for (int k = 0; k < T::NM; ++k) {
            sc[k] = 0;
            if constexpr (F == FfnFormat::MXFP4) sc[k] = ((st.sd[k][s] >> gsh) & 0xffu) << 23;
            else if constexpr (F == FfnFormat::NVFP4) sc[k] = (st.sd[k][s] >> gsh) & 0xffffu;
        }
#pragma unroll
        for (int j = 0; j < T::LK / 8; ++j) {
            const bf16x8 av = __builtin_bit_cast(bf16x8, xs[abase + s * (T::SKK / 8) + j]);
#pragma unroll
            for (int k = 0; k < T::NM; ++k)
                acc[k] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, rw_weights<F>(st.ring[s % D][k], sc[k], j), acc[k], 0, 0, 0);
        }
    }
}

// The NH parts' accumulators summed, in part order, into the waves of part 0, through LDS (over the
// rows, which every wave has finished reading). Every wave of the workgroup calls it.
template <int NM, int NH>
__device__ __forceinline__ void rw_reduce(f32x4 (&acc)[NM], uint4* xs, int tile, int part, int lane) {
    if constexpr (NH > 1) {
        rw_lds_barrier<-1>();
        float* red = reinterpret_cast<float*>(xs);
        if (part > 0) {
#pragma unroll
            for (int k = 0; k < NM; ++k)
#pragma unroll
                for (int e = 0; e < 4; ++e) red[((((part - 1) * 4 + tile) * NM + k) * 4 + e) * 64 + lane] = acc[k][e];
        }
        rw_lds_barrier<-1>();
        if (part == 0) {
#pragma unroll
            for (int q = 1; q < NH; ++q)
#pragma unroll
                for (int k = 0; k < NM; ++k)
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[k][e] += red[((((q - 1) * 4 + tile) * NM + k) * 4 + e) * 64 + lane];
        }
    }
}

// GeGLU of the up/gate sums for weight row n: v[e] the bf16 bits of rows 4 g + e.
template <FfnFormat F, ScaleKind SK>
__device__ __forceinline__ void rw_geglu_vals(const f32x4 (&acc)[2], const FfnParams& p, int n, uint32_t (&v)[4]) {
    float su = 1.0f, sg = 1.0f;
    if constexpr (F == FfnFormat::FP8) {
        su = rw_row_scale<SK>(p.up_s, n);
        sg = rw_row_scale<SK>(p.gate_s, n);
    } else if constexpr (F == FfnFormat::NVFP4) {
        su = *p.up_g;
        sg = *p.gate_g;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float up = rw_commit<F>(acc[0][e], su), gate = rw_commit<F>(acc[1][e], sg);
        v[e] = f2bf(rbf(gelu_tanh(gate)) * up);  // gemma4.py:197
    }
}

// The same for rows 4 g + e < M into p [M][L].
template <FfnFormat F, ScaleKind SK>
__device__ __forceinline__ void rw_geglu_out(const f32x4 (&acc)[2], const FfnParams& p, uint16_t* y, int n, int M, int g) {
    uint32_t v[4];
    rw_geglu_vals<F, SK>(acc, p, n, v);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int m = 4 * g + e;
        if (m < M) y[(size_t)m * kL + n] = (uint16_t)v[e];
    }
}

// The down partial sums of weight row n, split z, rows 4 g + e < M into yf [4][M][H].
__device__ __forceinline__ void rw_partial_out(const f32x4& acc, float* yf, int z, int n, int M, int g) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int m = 4 * g + e;
        if (m < M) yf[((size_t)z * M + m) * kH + n] = acc[e];
    }
}

// Workgroup (x, z): weight rows 64 x .. +64 (GeGLU: up and gate rows), k range 3840 z .. +3840;
// wave w: tile w % 4 over part w / 4 of the range.
template <FfnFormat F, ScaleKind SK, bool G>
__global__ __launch_bounds__((256 * RwShape<F, G>::NH)) void rows_kernel(FfnParams p, const uint16_t* x, int ldx, int M,
                                                                          uint16_t* y, float* yf) {
    using T = RwStream<F, G>;
    constexpr int NW = 4 * T::NH;
    __shared__ __attribute__((aligned(16))) uint4 xs[rw_lds_units<kRwK>()];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int tile = wave & 3, part = wave >> 2;
    const int r = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * kRwGroupRows + tile * kRwTile;
    const int kz = blockIdx.z * kRwK;  // first k of the workgroup (weights and activations alike)
    RwRows<64 * NW> rows;
    rw_rows_load<64 * NW>(rows, x, ldx, kz, M, t);
    T st;
    if constexpr (G) rw_prefetch<F, G, kRwK>(st, p.up, p.gate, p.up_s, p.gate_s, kH, n0, kz + part * T::KW, r, g);
    else rw_prefetch<F, G, kRwK>(st, p.down, nullptr, p.down_s, nullptr, kL, n0, kz + part * T::KW, r, g);
    rw_rows_store(rows, xs, t);
    f32x4 acc[T::NM];
    rw_mma<F, G, kRwK>(st, xs, acc, part, r, g);
    rw_reduce<T::NM, T::NH>(acc, xs, tile, part, lane);
    if (part != 0) return;
    if constexpr (G) rw_geglu_out<F, SK>(acc, p, y, n0 + r, M, g);
    else rw_partial_out(acc[0], yf, blockIdx.z, n0 + r, M, g);
}

// ---------------------------------------------------------------- up/gate and down in one launch
// rows_fused_kernel runs the pre-norm, the up/gate and down launches of rows_kernel and the post
// launch as one grid of kRwFusedGrid workgroups, one per CU, all resident at once (the host checks
// the occupancy first): 240 contraction workgroups, then 16 service workgroups.
//   * Service workgroup 240 + m (m < M) normalises residual row m as
//     chunk_rmsnorm_rows_kernel<false> does (four waves, the same arithmetic through
//     rms_row_values), writes it through and flags it; at the end it runs row m's post step as
//     chunk_post_rows_kernel does (post_row), once one contraction workgroup's down flag and then
//     all 240 carry the tag (a poll of one word per round until the end is near).
//   * Contraction workgroup b issues its first up/gate weight loads, waits for the M row flags,
//     stages the rows, and computes the GeGLU block b (L columns 64 b .. +64, all rows) as
//     rows_kernel<GeGLU> does, then the down block (c, z) = (b % 60, b / 60) as rows_kernel<down>
//     does.
// The same arithmetic in the same order as the separate launches, so the same bits.
//
// The hand-off of p: the workgroup writes its 16 x 64 GeGLU block with agent-scope 8-byte stores
// (write-through, coherent across the XCDs' L2s), waits for them to complete, and then publishes
// the launch's tag in its flag word. Down workgroup (c, z) needs the blocks of workgroups
// 60 z .. 60 z + 59 (its quarter of L): one wave polls their 60 flags, then the workgroup stages
// the quarter into LDS with ordinary loads. Those loads cannot meet a stale line: a kernel starts
// with invalidated L2s, each block owns whole 128-byte lines, and no wave reads a block before its
// flag carries the tag. The normalised rows and the down partial sums go the same way: written
// through, flagged, and read with ordinary loads once flagged (the rows by every contraction
// workgroup, row m's partials by service workgroup m). The down weights (rw_down_pre steps per
// wave) go out right after the GeGLU publish (the waves that store no GeGLU value, before it),
// so they stream while the slowest blocks are still being computed.
//
// Tags: epoch counters of this kernel alone (moa_sync.h epoch_tag), 16 workgroups per counter, so
// consecutive launches never share a tag and a flag left by an earlier launch never carries the
// current one. Every poll is bounded by the wall clock (kSpinTicks): on expiry it sets
// kErrSpinTimeout in the device error word and carries on. No wait takes work over (as the
// one-token kernels' do): a grid that could not be resident would end with that error rather than
// hang, and the host takes the separate launches wherever the occupancy check fails. The service
// workgroups' four upper waves end at once; their barriers then wait for the four that remain.
//
// Only calls that include the pre-norm take this kernel. Where the rows arrive normalised (the O ->
// FFN rows path, whose O post rows write them), the separate launches measured faster: 39.8-40.0
// against 40.2-40.4 us for O and the FFN at 16 MXFP4 rows. (The kernel with the post step on
// leader contraction workgroups, 240 workgroups and no service ones, measured 30.3 us at 16 MXFP4
// rows behind a pre-norm launch, 42.1 FP8; the service workgroups polling from the start were no
// faster with longer sleeps between polls: 16 / 64 clocks x 64 cost 0.3 / 1.3 us.)
//
// Down steps per wave issued before p's quarter is staged (of 30 FP8, 15 FP4); the rest stream
// behind the staging through the ring. Measured at 16 rows (graph-replayed): FP8 8 / 16 / 24 /
// 30 steps 43.6 / 42.8 / 43.0 / 44.6 us; MXFP4 4 / 8 / 11 / 15 steps 31.4 / 30.6 / 30.7 / 31.7 us
// (the staging loads return behind the prefetch, so a deeper prefetch delays the first MFMA).
template <FfnFormat F>
constexpr int rw_down_pre() { return F == FfnFormat::FP8 ? 16 : 8; }

// The up/gate ring's depth (D - 4 steps go out before the rows are staged). Measured at 16 rows:
// 8 / 12 / 16 steps FP8 42.8 / 41.1 / 41.0 us, MXFP4 30.0 / 29.6 / 30.7 us. (The pre-norm as a
// launch of its own ahead of this kernel measured 43.4 / 31.6 us at depth 8.)
template <FfnFormat F>
constexpr int rw_ug_depth() { return F == FfnFormat::FP8 ? 16 : 12; }

// The down partial sums of weight row n, split z, rows 4 g + e < M into yf [4][M][H], written
// through (agent scope) for the leaders of the one-launch kernel.
__device__ __forceinline__ void rw_partial_publish(const f32x4& acc, float* yf, int z, int n, int M, int g) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int m = 4 * g + e;
        if (m < M) publish32(yf + ((size_t)z * M + m) * kH + n, __float_as_uint(acc[e]));
    }
}

constexpr int kRwService = kMaxDecodeM;                 // workgroups 240 + m: row m's pre-norm and post step
constexpr int kRwFusedGrid = kRwUpGroups + kRwService;  // after the 240 contraction workgroups
static_assert(kRwFusedGrid == kRowsEpochCounters * kRowsEpochPer, "equal workgroups per epoch counter");
// flag words: the GeGLU blocks, the down blocks, the normalised rows
constexpr int kRwFlagP = 0, kRwFlagDown = kRwUpGroups, kRwFlagNorm = 2 * kRwUpGroups;
static_assert(kRwFlagNorm + kMaxDecodeM <= kRowsFlagWords, "flag words");

// Polls flags[first + i], i < n (n <= 256), until every one carries tag; one wave.
__device__ __forceinline__ void rw_poll(const uint64_t* flags, int first, int n, uint32_t tag, uint32_t* err, int lane) {
    const uint64_t t0 = wall_clock64();
    for (;;) {
        bool ok = true;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int k = lane + 64 * i;
            if (k < n) ok = ok && collect64(flags + first + k) == tag;
        }
        if (__all(ok)) return;
        if (wall_clock64() - t0 > kSpinTicks) {
            if (lane == 0) atomicOr(err, kErrSpinTimeout);
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// O's post step ahead of the FFN (sliding_attention_output then decoder_feedforward on one
// residual): O's split-K partial sums [4][M][H], its row scales and post-norm weight.
struct RwOPost {
    const float* part;
    const void* scale;
    const uint16_t* w_post;
};

// res: the M residual rows; x: their normalised rows, which the service workgroups write. OK: 0, or
// O's scale kind + 1 when the service workgroups first apply O's post step to their row (o).
template <FfnFormat F, ScaleKind SK, int OK = 0>
__global__ __launch_bounds__(256 * kRwNH) void rows_fused_kernel(FfnParams p, RwOPost o, uint16_t* x, int M, uint16_t* y,
                                                                 float* yf, uint16_t* res, uint64_t* flags,
                                                                 uint32_t* tickets, uint32_t* err) {
    using TU = RwStream<F, true, kRwK, rw_ug_depth<F>()>;
    using TD = RwStream<F, false, kRwK, rw_down_pre<F>() + RwShape<F, false>::B>;
    constexpr int NW = 4 * kRwNH;
    static_assert(kRwNH == 2, "grid shape");
    __shared__ __attribute__((aligned(16))) uint4 xs[rw_lds_units<kRwK>()];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int tile = wave & 3, part = wave >> 2;
    const int r = lane & 15, g = lane >> 4;
    // the launch's epoch (its return arrives behind the first loads; wave 0 derives the tag)
    uint64_t ep_old = 0;
    if (t == 0) ep_old = epoch_add(tickets + (kTicketRowsEpoch + blockIdx.x % kRowsEpochCounters) * kTicketStride);

    // ---- service workgroup m: the pre-norm of row m, then its post step (four waves)
    const int b = blockIdx.x;
    if (b >= kRwUpGroups) {
        const int m = b - kRwUpGroups;
        if (m >= M || part != 0) return;
        float* red = reinterpret_cast<float*>(xs);
        const uint32_t tag = epoch_tag<kRowsEpochPer>(__shfl(ep_old, 0));
        {
            // chunk_rmsnorm_rows_kernel's arithmetic, its row written through (agent scope); with O's
            // post step first, chunk_post_pre_rows_kernel's (the new residual row through LDS)
            const int c = min(t, kH / 16 - 1);
            float xv[16], wv[16];
            bf16x8_to_f32(ld16(p.pre_rms + c * 16), wv);
            bf16x8_to_f32(ld16(p.pre_rms + c * 16 + 8), wv + 8);
            if constexpr (OK != 0) {
                uint4 out[2];
                post_row<OK == 1 ? ScaleKind::F32 : ScaleKind::BF16, FfnFormat::FP8, kRwSplits>(
                    o.part, kRwSplits, M, o.scale, nullptr, o.w_post, res, nullptr, m, red, out);
                uint4* row = xs + 64;  // past red; kept until the post step below
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    if (t + 256 * i < kH / 8) row[t + 256 * i] = out[i];
                __syncthreads();
                bf16x8_to_f32(row[2 * c], xv);
                bf16x8_to_f32(row[2 * c + 1], xv + 8);
            } else {
                const uint16_t* xr = res + (size_t)m * kH + c * 16;
                bf16x8_to_f32(ld16(xr), xv);
                bf16x8_to_f32(ld16(xr + 8), xv + 8);
            }
            uint32_t h[8];
            rms_row_values(xv, wv, red, h);
            if (t < kH / 16) {
                uint64_t* dst = reinterpret_cast<uint64_t*>(x + (size_t)m * kH + c * 16);
#pragma unroll
                for (int i = 0; i < 4; ++i) publish64(dst + i, ((uint64_t)h[2 * i + 1] << 32) | h[2 * i]);
            }
            __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (t == 0) publish64(flags + kRwFlagNorm + m, tag);
        }
        // first one contraction workgroup's down flag (one load per round), then all of them
        if (wave == 0) {
            rw_poll(flags, kRwFlagDown + m * (kRwUpGroups / kRwService), 1, tag, err, lane);
            rw_poll(flags, kRwFlagDown, kRwUpGroups, tag, err, lane);
        }
        __syncthreads();
        // with O's post step first, row m's residual is the one in LDS (this workgroup wrote it)
        uint4 out[2];
        post_row<SK, F, kRwSplits>(yf, kRwSplits, M, F == FfnFormat::FP8 ? p.down_s : nullptr,
                                   F == FfnFormat::NVFP4 ? p.down_g : nullptr, p.post_rms, res, p.layer_scalar, m, red,
                                   out, OK != 0 ? xs + 64 : nullptr);
        return;
    }

    // ---- contraction workgroup b: up/gate (rows_kernel<GeGLU>)
    const uint32_t tag = epoch_tag<kRowsEpochPer>(__shfl(ep_old, 0));  // valid in wave 0
    f32x4 acc[2];
    {
        const int n0 = b * kRwGroupRows + tile * kRwTile;
        // the weights first; the rows once the service workgroups have published them
        TU st;
        rw_prefetch<F, true, kRwK>(st, p.up, p.gate, p.up_s, p.gate_s, kH, n0, part * TU::KW, r, g);
        if (wave == 0) rw_poll(flags, kRwFlagNorm, M, tag, err, lane);
        rw_lds_barrier<-1>();
        RwRows<64 * NW> rows;
        rw_rows_load<64 * NW>(rows, x, kH, 0, M, t);
        rw_rows_store(rows, xs, t);
        rw_mma<F, true, kRwK>(st, xs, acc, part, r, g);
    }
    rw_reduce<2, kRwNH>(acc, xs, tile, part, lane);
    // GeGLU block [16][64] into LDS past the reduction's floats, then out as 256 8-byte words
    uint16_t* pb = reinterpret_cast<uint16_t*>(xs + 1024);
    if (part == 0) {
        uint32_t v[4];
        rw_geglu_vals<F, SK>(acc, p, b * kRwGroupRows + tile * kRwTile + r, v);
#pragma unroll
        for (int e = 0; e < 4; ++e) pb[(4 * g + e) * kRwGroupRows + tile * kRwTile + r] = (uint16_t)v[e];
    }
    rw_lds_barrier<-1>();
    // ---- down (rows_kernel<down>): the weights first, then p's quarter once its blocks are in.
    // Waves of part 1 store nothing, so their weights go out at once; waves of part 0 store the
    // block, wait for their stores alone, and issue theirs after the flag.
    constexpr int kPer = kRwUpGroups / kRwSplits;  // GeGLU blocks per quarter of L
    static_assert(kMaxDecodeM * kRwGroupRows / 4 == 64 * (NW / 2), "one 8-byte word per thread of part 0");
    const int c = b % kRwDownGroups, z = b / kRwDownGroups;
    const int nd0 = c * kRwGroupRows + tile * kRwTile;
    TD sd;
    if (part != 0) {
        rw_prefetch<F, false, kRwK>(sd, p.down, nullptr, p.down_s, nullptr, kL, nd0, z * kRwK + part * TD::KW, r, g);
    } else {
        const int m = t / (kRwGroupRows / 4), q = t % (kRwGroupRows / 4);
        if (m < M)
            publish64(reinterpret_cast<uint64_t*>(y + (size_t)m * kL + b * kRwGroupRows) + q,
                      reinterpret_cast<const uint64_t*>(pb)[t]);
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
    if (t == 0) publish64(flags + kRwFlagP + b, tag);
    if (part == 0)
        rw_prefetch<F, false, kRwK>(sd, p.down, nullptr, p.down_s, nullptr, kL, nd0, z * kRwK + part * TD::KW, r, g);
    if (wave == 0) rw_poll(flags, kRwFlagP + z * kPer, kPer, tag, err, lane);
    rw_lds_barrier<-1>();
    f32x4 dacc[1];
    {
        RwRows<64 * NW> rows;
        rw_rows_load<64 * NW>(rows, y, kL, z * kRwK, M, t);
        rw_rows_store(rows, xs, t);
    }
    rw_mma<F, false, kRwK>(sd, xs, dacc, part, r, g);
    rw_reduce<1, kRwNH>(dacc, xs, tile, part, lane);
    // ---- the partial sums out (written through), then the block's down flag
    if (part == 0) {
        rw_partial_publish(dacc[0], yf, z, nd0 + r, M, g);
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
    if (t == 0) publish64(flags + kRwFlagDown + b, tag);
}

// ---------------------------------------------------------------- host
template <FfnFormat F, ScaleKind SK, bool G>
hipError_t rw_launch(dim3 grid, hipStream_t s, const FfnParams& p, const uint16_t* x, int ldx, int M, uint16_t* y, float* yf) {
    hipLaunchKernelGGL((rows_kernel<F, SK, G>), grid, dim3(256 * RwShape<F, G>::NH), 0, s, p, x, ldx, M, y, yf);
    return hipGetLastError();
}

std::atomic<int> g_rows_one_launch{1};

// Whether rows_fused_kernel<F, SK, OK> runs: its hand-off words exist, tests have not switched it
// off, and its grid fits on the device at once (checked once per device and instantiation).
template <FfnFormat F, ScaleKind SK, int OK = 0>
bool rows_fused_fits(DevCtx* ctx) {
    if (!ctx->rows_flag || !g_rows_one_launch.load()) return false;
    int8_t& known = ctx->rows_fused[((int)F * 2 + (int)SK) * 3 + OK];
    if (known < 0) {
        int per_cu = 0;
        const hipError_t e =
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, rows_fused_kernel<F, SK, OK>, 256 * kRwNH, 0);
        known = (e == hipSuccess && per_cu * ctx->cus >= kRwFusedGrid) ? 1 : 0;
    }
    return known == 1;
}

// One launch of rows_fused_kernel for rows m0 .. m0 + M - 1 (with O's post step first when OK != 0).
template <FfnFormat F, ScaleKind SK, int OK>
hipError_t launch_rows_fused(const FfnParams& p, const RwOPost& o, int m0, int M, hipStream_t s, DevCtx* ctx) {
    hipLaunchKernelGGL((rows_fused_kernel<F, SK, OK>), dim3(kRwFusedGrid), dim3(256 * kRwNH), 0, s, p, o, ctx->hbuf, M,
                       ctx->pbuf, ctx->fbuf, p.residual + (size_t)m0 * kH, ctx->rows_flag, ctx->tickets, ctx->err);
    return hipGetLastError();
}

// normed: the pre-norm's rows are already in ctx->hbuf (launch_o_ffn_rows)
template <FfnFormat F, ScaleKind SK>
hipError_t rows_ffn_impl(const FfnParams& p, int m0, int M, hipStream_t s, DevCtx* ctx, bool normed = false) {
    if (!normed && rows_fused_fits<F, SK>(ctx)) return launch_rows_fused<F, SK, 0>(p, RwOPost{}, m0, M, s, ctx);
    hipError_t e = normed ? hipSuccess : launch_rmsnorm_rows(p.residual + (size_t)m0 * kH, p.pre_rms, ctx->hbuf, M, s);
    if (e != hipSuccess) return e;
    e = rw_launch<F, SK, true>(dim3(kRwUpGroups, 1, 1), s, p, ctx->hbuf, kH, M, ctx->pbuf, nullptr);
    if (e != hipSuccess) return e;
    e = rw_launch<F, SK, false>(dim3(kRwDownGroups, 1, kRwSplits), s, p, ctx->pbuf, kL, M, nullptr, ctx->fbuf);
    if (e != hipSuccess) return e;
    return launch_ffn_post_rows(p, ctx->fbuf, kRwSplits, M, p.residual + (size_t)m0 * kH, s);
}

// ---------------------------------------------------------------- FP8 projections (QKV, O)
// Y[M][N] = X[M][K] . W[N][K]^T as split-K f32 partial sums [gridDim.z][M][N]; column n of the
// output uses weight matrix w[i] (its row n - nseg[i]); a workgroup's 64 columns never straddle two
// matrices. The scales are applied by the row kernels that sum the partials.
struct ProjRows {
    const uint16_t* x;  // [M][K] bf16 rows
    const float* div;   // full-attention output: running sums [M][16] dividing x (or null)
    int M, K, N;
    const uint8_t* w[3];
    int nseg[4];
    int nsegs;
    float* yf;
};

template <int KR>
__global__ __launch_bounds__((256 * kRwNH)) void rows_proj_kernel(ProjRows a) {
    using T = RwStream<FfnFormat::FP8, false, KR>;
    constexpr int NW = 4 * T::NH;
    __shared__ __attribute__((aligned(16))) uint4 xs[rw_lds_units<KR>()];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int tile = wave & 3, part = wave >> 2;
    const int r = lane & 15, g = lane >> 4;
    const int c0 = blockIdx.x * kRwGroupRows;
    int seg = 0;
    while (seg + 1 < a.nsegs && c0 >= a.nseg[seg + 1]) ++seg;
    const int n0 = c0 - a.nseg[seg] + tile * kRwTile;  // row of w[seg]
    const int kz = blockIdx.z * KR;
    RwRows<64 * NW, KR> rows;
    rw_rows_load<64 * NW>(rows, a.x, a.K, kz, a.M, t, a.div);
    T st;
    rw_prefetch<FfnFormat::FP8, false, KR>(st, a.w[seg], nullptr, nullptr, nullptr, a.K, n0, kz + part * T::KW, r, g);
    rw_rows_store(rows, xs, t);
    f32x4 acc[1];
    rw_mma<FfnFormat::FP8, false, KR>(st, xs, acc, part, r, g);
    rw_reduce<1, T::NH>(acc, xs, tile, part, lane);
    if (part != 0) return;
    const int n = c0 + tile * kRwTile + r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int m = 4 * g + e;
        if (m < a.M) a.yf[((size_t)blockIdx.z * a.M + m) * a.N + n] = acc[0][e];
    }
}

template <int KR>
hipError_t rw_proj(const ProjRows& a, hipStream_t s) {
    if (a.N % kRwGroupRows || a.K % KR) return hipErrorInvalidValue;
    hipLaunchKernelGGL((rows_proj_kernel<KR>), dim3(a.N / kRwGroupRows, 1, a.K / KR), dim3(256 * kRwNH), 0, s, a);
    return hipGetLastError();
}

constexpr int kRwQkvKR = 1920;  // QKV: 128 column groups x 2 halves of H
constexpr int kRwOKR = 1024;    // O: 60 column groups x 4 quarters of the 4096 inputs
constexpr int kRwFoKR = 2048;   // full-attention O: 60 column groups x 4 quarters of the 8192 inputs
static_assert((rw_row_units<kRwQkvKR>() * 4) % 64 == 4 && (rw_row_units<kRwOKR>() * 4) % 64 == 4 &&
                  (rw_row_units<kRwFoKR>() * 4) % 64 == 4, "LDS banks");

// Block sum over the workgroup's NW waves, in wave order.
template <int NW>
__device__ __forceinline__ float rw_block_sum(float v, float* red, int lane, int wave) {
    v = wave_sum(v);
    if (lane == 0) red[wave] = v;
    rw_lds_barrier<-1>();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) tot += red[w];
    rw_lds_barrier<-1>();
    return tot;
}

// full_project_qkv heads after the split-K contraction: workgroup (head, row), head < 16 a query
// head, head 16 the one KV head; thread t owns elements t and t + 256 of the head's 512. raw =
// bf16(sum of the partials * scale), then as the per-row kernels' head epilogue (full/rmsnorm.rs,
// rope.rs; generate_references.py:265-274): RMSNorm over the head (weighted for q and k; V is the
// unweighted norm of the same raw K), RoPE (the table's sin has its low half negated: plain half
// swap), q_out / page-slot stores. A row whose offsets are bad writes nothing, and its head-0
// workgroup reports them.
template <ScaleKind SK>
__global__ __launch_bounds__(256) void rows_fqkv_heads_kernel(QkvParams p, int m0, int M, const float* __restrict__ part,
                                                              int splits, uint32_t* err) {
    constexpr int Hf = kDf / 2, N = kQf + kPf;
    __shared__ float red[4];
    const int head = blockIdx.x, m = blockIdx.y, t = threadIdx.x;
    const int mm = m0 + m;
    const int32_t rope_off = *p.rope_off, kv_off = *p.kv_off;
    const bool rope_ok = rope_off >= 0 && (rope_off % (kDf * 2)) == 0 && rope_off / (kDf * 2) + mm < kE;
    const bool kv_ok = kv_off >= 0 && (kv_off % (kDf * 2)) == 0 && kv_off / (kDf * 2) + mm < kTf;
    if (!rope_ok || !kv_ok) {
        if (head == 0 && t == 0) atomicOr(err, (rope_ok ? 0u : kErrRopeOffset) | (kv_ok ? 0u : kErrKvOffset));
        return;
    }
    const int slot = kv_off / (kDf * 2) + mm;
    const int trow = rope_off / (kDf * 2) + mm;
    float raw[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int col = head * kDf + t + h * Hf;
        float a = 0.0f;
        for (int z = 0; z < splits; ++z) a = z == 0 ? part[((size_t)z * M + m) * N + col] : a + part[((size_t)z * M + m) * N + col];
        const float sc = head < kGf ? rw_row_scale<SK>(p.qs, col) : rw_row_scale<SK>(p.ks, col - kQf);
        raw[h] = rbf(a * sc);
    }
    const uint16_t* wn = head < kGf ? p.q_rms : p.k_rms;
    const float w0 = bf2f(wn[t]), w1 = bf2f(wn[t + Hf]);
    const float c0 = bf2f(p.cos[(size_t)trow * kDf + t]), c1 = bf2f(p.cos[(size_t)trow * kDf + t + Hf]);
    const float s0 = bf2f(p.sin[(size_t)trow * kDf + t]), s1 = bf2f(p.sin[(size_t)trow * kDf + t + Hf]);
    const float inv = rms_inverse(rw_block_sum<4>(raw[0] * raw[0] + raw[1] * raw[1], red, t & 63, t >> 6), kDf);
    const float u0 = raw[0] * inv, u1 = raw[1] * inv;
    if (head == kGf) {  // V: the unweighted norm
        p.v_cache[(size_t)slot * kDf + t] = (uint16_t)f2bf(u0);
        p.v_cache[(size_t)slot * kDf + t + Hf] = (uint16_t)f2bf(u1);
    }
    const float n0 = rbf(u0 * w0), n1 = rbf(u1 * w1);
    uint16_t* dst = head < kGf ? p.q_out + (size_t)mm * kQf + head * kDf : p.k_cache + (size_t)slot * kDf;
    dst[t] = (uint16_t)f2bf(rbf(n0 * c0) + rbf(n1 * s0));
    dst[t + Hf] = (uint16_t)f2bf(rbf(n1 * c1) + rbf(n0 * s1));
}

}  // namespace

hipError_t launch_full_qkv_rows(const QkvParams& p, int m0, int M, hipStream_t s, DevCtx* ctx) {
    if (M < 1 || M > kMaxDecodeM) return hipErrorInvalidValue;
    hipError_t e = launch_rmsnorm_rows(p.x + (size_t)m0 * kH, p.in_rms, ctx->hbuf, M, s);
    if (e != hipSuccess) return e;
    ProjRows a{};
    a.x = ctx->hbuf; a.M = M; a.K = kH; a.N = kQf + kPf;
    a.w[0] = p.qw; a.w[1] = p.kw;
    a.nseg[0] = 0; a.nseg[1] = kQf; a.nseg[2] = kQf + kPf; a.nsegs = 2;
    a.yf = ctx->fbuf;
    e = rw_proj<kRwQkvKR>(a, s);
    if (e != hipSuccess) return e;
    const int sp = kH / kRwQkvKR;
    if (p.scale_kind == ScaleKind::F32)
        hipLaunchKernelGGL((rows_fqkv_heads_kernel<ScaleKind::F32>), dim3(kGf + 1, M), dim3(256), 0, s, p, m0, M,
                           (const float*)ctx->fbuf, sp, ctx->err);
    else
        hipLaunchKernelGGL((rows_fqkv_heads_kernel<ScaleKind::BF16>), dim3(kGf + 1, M), dim3(256), 0, s, p, m0, M,
                           (const float*)ctx->fbuf, sp, ctx->err);
    return hipGetLastError();
}

hipError_t launch_qkv_rows(const QkvParams& p, int m0, int M, hipStream_t s, DevCtx* ctx) {
    if (M < 1 || M > kMaxDecodeM) return hipErrorInvalidValue;
    hipError_t e = launch_rmsnorm_rows(p.x + (size_t)m0 * kH, p.in_rms, ctx->hbuf, M, s);
    if (e != hipSuccess) return e;
    ProjRows a{};
    a.x = ctx->hbuf; a.M = M; a.K = kH; a.N = kQkvRowsTotal;
    a.w[0] = p.qw; a.w[1] = p.kw; a.w[2] = p.vw;
    a.nseg[0] = 0; a.nseg[1] = kQs; a.nseg[2] = kQs + kPs; a.nseg[3] = kQkvRowsTotal; a.nsegs = 3;
    a.yf = ctx->fbuf;
    e = rw_proj<kRwQkvKR>(a, s);
    if (e != hipSuccess) return e;
    return launch_qkv_heads(p, m0, M, ctx->fbuf, kH / kRwQkvKR, s, ctx);
}

hipError_t launch_o_rows(const OParams& p, int m0, int M, hipStream_t s, DevCtx* ctx) {
    if (M < 1 || M > kMaxDecodeM) return hipErrorInvalidValue;
    const bool full = p.div != nullptr;  // full-attention layer: 8192 inputs divided by the running sums
    const int K = full ? kQf : kQs;
    ProjRows a{};
    a.x = p.x + (size_t)m0 * K; a.div = full ? p.div + (size_t)m0 * kGf : nullptr; a.M = M; a.K = K; a.N = kH;
    a.w[0] = p.ow; a.nseg[0] = 0; a.nseg[1] = kH; a.nsegs = 1;
    a.yf = ctx->fbuf;
    const hipError_t e = full ? rw_proj<kRwFoKR>(a, s) : rw_proj<kRwOKR>(a, s);
    if (e != hipSuccess) return e;
    return launch_post_rows(ctx->fbuf, K / (full ? kRwFoKR : kRwOKR), M, p.os, p.scale_kind, p.post_rms,
                            p.residual + (size_t)m0 * kH, nullptr, s);
}

static hipError_t ffn_rows_dispatch(const FfnParams& p, int m0, int M, hipStream_t s, DevCtx* ctx, bool normed) {
    switch (p.fmt) {
        case FfnFormat::FP8:
            return p.scale_kind == ScaleKind::F32 ? rows_ffn_impl<FfnFormat::FP8, ScaleKind::F32>(p, m0, M, s, ctx, normed)
                                                  : rows_ffn_impl<FfnFormat::FP8, ScaleKind::BF16>(p, m0, M, s, ctx, normed);
        case FfnFormat::NVFP4: return rows_ffn_impl<FfnFormat::NVFP4, ScaleKind::F32>(p, m0, M, s, ctx, normed);
        case FfnFormat::MXFP4: return rows_ffn_impl<FfnFormat::MXFP4, ScaleKind::F32>(p, m0, M, s, ctx, normed);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_ffn_rows(const FfnParams& p, int m0, int M, hipStream_t s, DevCtx* ctx) {
    if (M < 1 || M > kMaxDecodeM) return hipErrorInvalidValue;
    return ffn_rows_dispatch(p, m0, M, s, ctx, false);
}

// O's contraction as launch_o_rows runs it, then O's post rows and the FFN's pre-norm (the bits of
// chunk_post_rows_kernel, then of chunk_rmsnorm_rows_kernel<false>) and the FFN: in one launch on
// rows_fused_kernel's service workgroups where its grid fits, else as one row kernel
// (chunk_post_pre_rows_kernel) and the FFN's rows path from its up/gate contraction on.
static_assert(kQs / kRwOKR == kRwSplits, "O's split-K partial sums: as many as the down projection's");

// O's post step and the FFN in one launch (rows_fused_kernel with O's post on its service
// workgroups), for the formats and O scale kinds the fused kernel is instantiated for.
template <FfnFormat F, ScaleKind SK>
static bool o_ffn_rows_fused(const OParams& o, const FfnParams& p, const float* opart, int m0, int M, hipStream_t s,
                             DevCtx* ctx, hipError_t* e) {
    const RwOPost op{opart, o.os, o.post_rms};
    if (o.scale_kind == ScaleKind::F32) {
        if (!rows_fused_fits<F, SK, 1>(ctx)) return false;
        *e = launch_rows_fused<F, SK, 1>(p, op, m0, M, s, ctx);
    } else {
        if (!rows_fused_fits<F, SK, 2>(ctx)) return false;
        *e = launch_rows_fused<F, SK, 2>(p, op, m0, M, s, ctx);
    }
    return true;
}

hipError_t launch_o_ffn_rows(const OParams& o, const FfnParams& p, int m0, int M, hipStream_t s, DevCtx* ctx) {
    if (M < 1 || M > kMaxDecodeM || o.div || o.residual != p.residual) return hipErrorInvalidValue;
    ProjRows a{};
    a.x = o.x + (size_t)m0 * kQs; a.M = M; a.K = kQs; a.N = kH;
    a.w[0] = o.ow; a.nseg[0] = 0; a.nseg[1] = kH; a.nsegs = 1;
    // O's partial sums past the FFN's own (the one launch reads the first while it writes the second)
    float* opart = ctx->fbuf + (size_t)kRwSplits * kMaxDecodeM * kH;
    a.yf = opart;
    hipError_t e = rw_proj<kRwOKR>(a, s);
    if (e != hipSuccess) return e;
    bool done = false;
    switch (p.fmt) {
        case FfnFormat::FP8:
            done = p.scale_kind == ScaleKind::F32 ? o_ffn_rows_fused<FfnFormat::FP8, ScaleKind::F32>(o, p, opart, m0, M, s, ctx, &e)
                                                  : o_ffn_rows_fused<FfnFormat::FP8, ScaleKind::BF16>(o, p, opart, m0, M, s, ctx, &e);
            break;
        case FfnFormat::NVFP4: done = o_ffn_rows_fused<FfnFormat::NVFP4, ScaleKind::F32>(o, p, opart, m0, M, s, ctx, &e); break;
        case FfnFormat::MXFP4: done = o_ffn_rows_fused<FfnFormat::MXFP4, ScaleKind::F32>(o, p, opart, m0, M, s, ctx, &e); break;
    }
    if (done) return e;
    e = launch_post_pre_rows(opart, kQs / kRwOKR, M, o.os, o.scale_kind, o.post_rms, o.residual + (size_t)m0 * kH,
                             p.pre_rms, ctx->hbuf, s);
    if (e != hipSuccess) return e;
    return ffn_rows_dispatch(p, m0, M, s, ctx, true);
}

void set_rows_one_launch(bool on) { g_rows_one_launch.store(on ? 1 : 0); }

}  // namespace moa
