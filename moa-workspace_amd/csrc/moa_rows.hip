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
// run as one launch whose phases are separated by grid barriers when the 240 workgroups fit on
// the device at once (each phase's weight loads are issued before the barrier that precedes it),
// and otherwise as four launches.
#include <hip/hip_runtime.h>

#include "moa_device.h"
#include "moa_internal.h"
#include "moa_sync.h"

namespace moa {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 rw_bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kRwTile = 16;                    // weight rows per wave (the MFMA's N)
constexpr int kRwGroupRows = 4 * kRwTile;      // weight rows per workgroup
constexpr int kRwK = 3840;                     // k per workgroup: all of H (up/gate), a quarter of L (down)
constexpr int kRwRowUnits = kRwK / 8 + 1;      // 16-byte LDS units per activation row, one of them padding
constexpr int kRwLdsUnits = (kMaxDecodeM * kRwRowUnits + 63) / 64 * 64;  // whole 1 KB blocks
constexpr int kRwSplits = kL / kRwK;           // down: four k quarters
constexpr int kRwUpGroups = kL / kRwGroupRows;      // 240 up/gate workgroups
constexpr int kRwDownGroups = kH / kRwGroupRows;    // 60 down column groups (x 4 quarters)
constexpr int kRwNH = 2;                       // k parts per workgroup: 8 compute waves
constexpr int kRwCompute = 4 * kRwNH;
constexpr int kRwFusedBlock = 64 * (kRwCompute + 1);  // the single launch adds a control wave
static_assert(kH == kRwK && kL == kRwSplits * kRwK, "one workgroup k range");
static_assert(kL % kRwGroupRows == 0 && kH % kRwGroupRows == 0, "whole weight tiles");
static_assert(kRwDownGroups * kRwSplits == kRwUpGroups, "one grid for both contractions");
static_assert((kRwRowUnits * 4) % 64 == 4, "row stride: 16 rows start on distinct LDS banks");
static_assert(kH / 8 <= kRwCompute * 64, "a row's 16-byte units fit the compute waves");

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
// workgroup's k range, the FP4 block-scale codes of that range, and the ring of loads.
template <FfnFormat F, bool G>
struct RwStream {
    static constexpr int NM = G ? 2 : 1;
    static constexpr int NH = RwShape<F, G>::NH, D = RwShape<F, G>::D, B = RwShape<F, G>::B;
    static constexpr int LK = rw_lane_k<F>(), SKK = rw_step_k<F>();
    static constexpr int KW = kRwK / NH;  // k per wave
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
template <FfnFormat F, bool G>
__device__ __forceinline__ void rw_prefetch(RwStream<F, G>& st, const uint8_t* w0, const uint8_t* w1, const void* s0,
                                            const void* s1, int wk, int n0, int kb, int r, int g) {
    using T = RwStream<F, G>;
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
#pragma unroll
        for (int k = 0; k < T::NM; ++k) st.ring[i][k] = rw_issue(st.wp[k], i);
}

// Activation rows 0 .. M-1 of x (row stride ldx, columns kz ..) into LDS, 1 KB per wave
// instruction by nw waves (unit u: row u / 481, 16 bytes u % 481; the padding unit and the last
// block's tail load a valid chunk that is not read). AUX: the loads' cache policy (16 = sc1, for
// rows written by other workgroups of the same launch).
template <int AUX>
__device__ __forceinline__ void rw_stage_issue(uint4* xs, const uint16_t* x, int ldx, int kz, int M, int wave, int nw,
                                               int lane) {
    for (int b = wave; b * 64 < M * kRwRowUnits; b += nw) {
        const int u = b * 64 + lane;
        const int m = min(u / kRwRowUnits, M - 1), c = min(u % kRwRowUnits, kRwK / 8 - 1);
        __builtin_amdgcn_global_load_lds((glb_void*)(x + (size_t)m * ldx + kz + c * 8), (lds_void*)(xs + b * 64), 16, 0,
                                         AUX);
    }
}

// Staging complete in every wave (vmcnt(0): the compiler may merge or reorder the loads issued
// after the staging, so no count of them is relied on); rows past M become zeros.
__device__ __forceinline__ void rw_stage_finish(uint4* xs, int M, int t, int nthreads) {
    rw_lds_barrier<0>();
    for (int u = M * kRwRowUnits + t; u < kMaxDecodeM * kRwRowUnits; u += nthreads) xs[u] = make_uint4(0, 0, 0, 0);
    rw_lds_barrier<-1>();
}

// The stream against the LDS rows, unrolled over its S load steps: every B steps, step s first
// refills the ring slots read in steps s - B .. s - 1 (with steps s + D - B .. s + D - 1), then
// each step runs its MFMAs. MFMA j of a step takes the lane's k 8 j .. 8 j + 7 of its load -- for
// A (LDS row r) and B alike, a fixed permutation of the step's k. acc[k][e]: row 4 g + e, weight
// row r of the tile.
template <FfnFormat F, bool G>
__device__ __forceinline__ void rw_mma(RwStream<F, G>& st, const uint4* xs, f32x4 (&acc)[G ? 2 : 1], int part, int r,
                                       int g) {
    using T = RwStream<F, G>;
    constexpr int D = T::D, B = T::B, S = T::S;
#pragma unroll
    for (int k = 0; k < T::NM; ++k) acc[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int abase = r * kRwRowUnits + (part * T::KW + g * T::LK) / 8;
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
// rows, which every wave has finished reading). Every wave of the workgroup calls it (a wave
// without a part passes -1).
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

// GeGLU of the up/gate sums for weight row n and rows 4 g + e < M into p [M][L] (PUB: agent-scope
// stores, read by other workgroups of the same launch).
template <FfnFormat F, ScaleKind SK, bool PUB>
__device__ __forceinline__ void rw_geglu_out(const f32x4 (&acc)[2], const FfnParams& p, uint16_t* y, int n, int M, int g) {
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
        const int m = 4 * g + e;
        if (m < M) {
            const float up = rw_commit<F>(acc[0][e], su), gate = rw_commit<F>(acc[1][e], sg);
            const uint32_t v = f2bf(rbf(gelu_tanh(gate)) * up);  // gemma4.py:197
            if constexpr (PUB) publish(y + (size_t)m * kL + n, v);
            else y[(size_t)m * kL + n] = (uint16_t)v;
        }
    }
}

// The down partial sums of weight row n, split z, rows 4 g + e < M into yf [4][M][H].
template <bool PUB>
__device__ __forceinline__ void rw_partial_out(const f32x4& acc, float* yf, int z, int n, int M, int g) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int m = 4 * g + e;
        if (m < M) {
            float* dst = yf + ((size_t)z * M + m) * kH + n;
            if constexpr (PUB) publish32(dst, __float_as_uint(acc[e]));
            else *dst = acc[e];
        }
    }
}

// ---------------------------------------------------------------- four launches
// Workgroup (x, z): weight rows 64 x .. +64 (GeGLU: up and gate rows), k range 3840 z .. +3840;
// wave w: tile w % 4 over part w / 4 of the range.
template <FfnFormat F, ScaleKind SK, bool G>
__global__ __launch_bounds__((256 * RwShape<F, G>::NH)) void rows_kernel(FfnParams p, const uint16_t* x, int ldx, int M,
                                                                          uint16_t* y, float* yf) {
    using T = RwStream<F, G>;
    constexpr int NW = 4 * T::NH;
    __shared__ __attribute__((aligned(16))) uint4 xs[kRwLdsUnits];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int tile = wave & 3, part = wave >> 2;
    const int r = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * kRwGroupRows + tile * kRwTile;
    const int kz = blockIdx.z * kRwK;  // first k of the workgroup (weights and activations alike)
    rw_stage_issue<0>(xs, x, ldx, kz, M, wave, NW, lane);
    T st;
    if constexpr (G) rw_prefetch<F, G>(st, p.up, p.gate, p.up_s, p.gate_s, kH, n0, kz + part * T::KW, r, g);
    else rw_prefetch<F, G>(st, p.down, nullptr, p.down_s, nullptr, kL, n0, kz + part * T::KW, r, g);
    rw_stage_finish(xs, M, t, 64 * NW);
    f32x4 acc[T::NM];
    rw_mma<F, G>(st, xs, acc, part, r, g);
    rw_reduce<T::NM, T::NH>(acc, xs, tile, part, lane);
    if (part != 0) return;
    if constexpr (G) rw_geglu_out<F, SK, false>(acc, p, y, n0 + r, M, g);
    else rw_partial_out<false>(acc[0], yf, blockIdx.z, n0 + r, M, g);
}

// ---------------------------------------------------------------- one launch
struct RowsFused {
    FfnParams p;
    int m0, M;
    uint16_t* hbuf;     // [M][H] pre-normed rows
    uint16_t* pbuf;     // [M][L] GeGLU output
    float* fbuf;        // [4][M][H] down partial sums
    uint32_t* tickets;
    uint32_t* err;
};

// Block sum over the workgroup's waves, in wave order.
__device__ __forceinline__ float rw_block_sum(float v, float* red, int lane, int wave) {
    v = wave_sum(v);
    if (lane == 0) red[wave] = v;
    rw_lds_barrier<-1>();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w <= kRwCompute; ++w) tot += red[w];
    rw_lds_barrier<-1>();
    return tot;
}

// Every wave: the workgroup's published results are complete (each wave waited for its own
// stores), then the control wave's first lane arrives on the grid barrier and waits for `target`.
__device__ __forceinline__ void rw_grid_sync(bool ctl, int lane, uint32_t* tickets, uint32_t target, uint32_t* err) {
    rw_lds_barrier<-1>();
    if (ctl && lane == 0)
        grid_barrier(tickets + kTicketRowsBar * kTicketStride, tickets + kTicketRowsGen * kTicketStride, target, err);
    rw_lds_barrier<-1>();
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rw_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// Workgroups 0 .. M-1 of the single launch; workgroup b: row b. Thread t < 480 owns the row's
// 16-byte unit t (8 elements).
// Pre-norm: h = bf16((x * inv) * w), published (gemma4.py:83-89).
__device__ __forceinline__ void rw_norm_row(const RowsFused& f, int b, float* red, int t, int lane, int wave) {
    const bool act = t < kH / 8;
    const int c = min(t, kH / 8 - 1);
    float xv[8], wv[8];
    bf16x8_to_f32(ld16(f.p.residual + (size_t)(f.m0 + b) * kH + c * 8), xv);
    bf16x8_to_f32(ld16(f.p.pre_rms + c * 8), wv);
    float ss = 0.0f;
    if (act) {
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(xv[e], xv[e], ss);  // x*x is exact in f32
    }
    const float inv = rms_inverse(rw_block_sum(ss, red, lane, wave), kH);
    if (act) {
        uint32_t h[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = f2bf((xv[2 * e] * inv) * wv[2 * e]) | (f2bf((xv[2 * e + 1] * inv) * wv[2 * e + 1]) << 16);
        uint64_t* dst = reinterpret_cast<uint64_t*>(f.hbuf + (size_t)b * kH + c * 8);
        publish64(dst, ((uint64_t)h[1] << 32) | h[0]);
        publish64(dst + 1, ((uint64_t)h[3] << 32) | h[2]);
    }
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // published before the workgroup arrives
}

// Post: d = commit(sum of the four partials), out = bf16(bf16(r + N(d)) * ls) with N the post-RMSNorm
// (identity when the weight is null) and ls skipped when null.
template <FfnFormat F, ScaleKind SK>
__device__ __forceinline__ void rw_post_row(const RowsFused& f, int b, float* red, int t, int lane, int wave) {
    const FfnParams& p = f.p;
    const bool act = t < kH / 8;
    const int c = min(t, kH / 8 - 1);
    uint16_t* rr = p.residual + (size_t)(f.m0 + b) * kH + c * 8;
    const uint4 rq = ld16(rr);
    const uint4 wq = p.post_rms ? ld16(p.post_rms + c * 8) : make_uint4(0, 0, 0, 0);
    const __amdgpu_buffer_rsrc_t rs = rw_rsrc(f.fbuf, (uint32_t)(sizeof(float) * kRwSplits * f.M * kH));
    float4 u[kRwSplits][2];
#pragma unroll
    for (int z = 0; z < kRwSplits; ++z) {
        const int off = (int)(sizeof(float) * (((size_t)z * f.M + b) * kH + c * 8));
        u[z][0] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 16 /* sc1 */));
        u[z][1] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16, 0, 16 /* sc1 */));
    }
    float gs = 1.0f;
    if constexpr (F == FfnFormat::NVFP4) gs = *p.down_g;
    float d[8];
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        float a = 0.0f;
#pragma unroll
        for (int z = 0; z < kRwSplits; ++z) {
            const float4& v = u[z][e >> 2];
            const float x = (e & 3) == 0 ? v.x : ((e & 3) == 1 ? v.y : ((e & 3) == 2 ? v.z : v.w));
            a = z == 0 ? x : a + x;
        }
        if constexpr (F == FfnFormat::FP8) d[e] = rbf(a * rw_row_scale<SK>(p.down_s, c * 8 + e));
        else if constexpr (F == FfnFormat::NVFP4) d[e] = rbf(rbf(a) * gs);
        else d[e] = rbf(a);
        if (act) ss = fmaf(d[e], d[e], ss);
    }
    const float tot = rw_block_sum(ss, red, lane, wave);
    const float inv = p.post_rms ? rms_inverse(tot, kH) : 1.0f;
    if (!act) return;
    const float lsv = p.layer_scalar ? bf2f(p.layer_scalar[0]) : 1.0f;
    float rv[8], wv[8];
    bf16x8_to_f32(rq, rv);
    bf16x8_to_f32(wq, wv);
    uint32_t pk[4];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        float n = d[e];
        if (p.post_rms) n = rbf((n * inv) * wv[e]);
        float sres = rbf(rv[e] + n);
        if (p.layer_scalar) sres = rbf(sres * lsv);
        const uint32_t bb = f2bf(sres);
        if (e & 1) pk[e >> 1] |= bb << 16; else pk[e >> 1] = bb;
    }
    *reinterpret_cast<uint4*>(rr) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
}

// The four steps in one launch of 240 workgroups (all resident at once), eight compute waves and
// a control wave each. Phases: 0 pre-norm (workgroups 0 .. M-1) | 1 up/gate (workgroup b: L-rows
// 64 b ..) | 2 down (workgroup b: columns 64 (b % 60) .., k quarter b / 60) | 3 post (workgroups
// 0 .. M-1), separated by grid barriers. Each compute wave issues its next phase's weight loads
// before the barrier; the control wave, which loads no weights, is the one that waits on the
// barrier's counters (a wave's wait for an atomic's result waits for all of its earlier loads).
template <FfnFormat F, ScaleKind SK>
__global__ __launch_bounds__(kRwFusedBlock) void rows_fused_kernel(RowsFused f) {
    using TU = RwStream<F, true>;
    using TD = RwStream<F, false>;
    static_assert(TU::NH == kRwNH && TD::NH == kRwNH, "one workgroup shape for both contractions");
    __shared__ __attribute__((aligned(16))) uint4 xs[kRwLdsUnits];
    __shared__ float red[kRwCompute + 1];
    const FfnParams& p = f.p;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const bool ctl = wave == kRwCompute;
    const int tile = wave & 3, part = ctl ? -1 : wave >> 2;
    const int r = lane & 15, g = lane >> 4;
    const int M = f.M, b = blockIdx.x;
    uint32_t g0 = 0;
    if (ctl) g0 = __hip_atomic_load(f.tickets + kTicketRowsGen * kTicketStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    // phase 0: pre-norm; every compute wave's up/gate loads go out
    if (b < M) rw_norm_row(f, b, red, t, lane, wave);
    TU us;
    const int un0 = b * kRwGroupRows + tile * kRwTile;
    if (!ctl) rw_prefetch<F, true>(us, p.up, p.gate, p.up_s, p.gate_s, kH, un0, part * TU::KW, r, g);
    rw_grid_sync(ctl, lane, f.tickets, g0 + 1u, f.err);

    // phase 1: up/gate and GeGLU; then the down loads go out
    rw_stage_issue<16>(xs, f.hbuf, kH, 0, M, wave, kRwCompute + 1, lane);
    rw_stage_finish(xs, M, t, kRwFusedBlock);
    {
        f32x4 acc[2];
        if (!ctl) rw_mma<F, true>(us, xs, acc, part, r, g);
        rw_reduce<2, kRwNH>(acc, xs, tile, part, lane);
        if (part == 0) rw_geglu_out<F, SK, true>(acc, p, f.pbuf, un0 + r, M, g);
    }
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // p published
    TD dst;
    const int dx = b % kRwDownGroups, dz = b / kRwDownGroups;
    const int dn0 = dx * kRwGroupRows + tile * kRwTile;
    if (!ctl) rw_prefetch<F, false>(dst, p.down, nullptr, p.down_s, nullptr, kL, dn0, dz * kRwK + part * TD::KW, r, g);
    rw_grid_sync(ctl, lane, f.tickets, g0 + 2u, f.err);

    // phase 2: down partial sums
    rw_stage_issue<16>(xs, f.pbuf, kL, dz * kRwK, M, wave, kRwCompute + 1, lane);
    rw_stage_finish(xs, M, t, kRwFusedBlock);
    {
        f32x4 acc[1];
        if (!ctl) rw_mma<F, false>(dst, xs, acc, part, r, g);
        rw_reduce<1, kRwNH>(acc, xs, tile, part, lane);
        if (part == 0) rw_partial_out<true>(acc[0], f.fbuf, dz, dn0 + r, M, g);
    }
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // partial sums published
    rw_grid_sync(ctl, lane, f.tickets, g0 + 3u, f.err);

    // phase 3: post
    if (b < M) rw_post_row<F, SK>(f, b, red, t, lane, wave);
}

// ---------------------------------------------------------------- host
template <FfnFormat F, ScaleKind SK, bool G>
hipError_t rw_launch(dim3 grid, hipStream_t s, const FfnParams& p, const uint16_t* x, int ldx, int M, uint16_t* y, float* yf) {
    hipLaunchKernelGGL((rows_kernel<F, SK, G>), grid, dim3(256 * RwShape<F, G>::NH), 0, s, p, x, ldx, M, y, yf);
    return hipGetLastError();
}

// Whether the single launch's 240 workgroups fit on the device at once (checked once per device).
template <FfnFormat F, ScaleKind SK>
bool rows_fused_fits(DevCtx* ctx) {
    int8_t& known = ctx->rows_fused[(int)F * 2 + (int)SK];
    if (known < 0) {
        int per_cu = 0;
        const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, rows_fused_kernel<F, SK>, kRwFusedBlock, 0);
        known = (e == hipSuccess && per_cu * ctx->cus >= kRwUpGroups) ? 1 : 0;
    }
    return known == 1;
}

template <FfnFormat F, ScaleKind SK>
hipError_t rows_ffn_impl(const FfnParams& p, int m0, int M, hipStream_t s, DevCtx* ctx) {
    if (rows_fused_fits<F, SK>(ctx)) {
        const RowsFused f{p, m0, M, ctx->hbuf, ctx->pbuf, ctx->fbuf, ctx->tickets, ctx->err};
        hipLaunchKernelGGL((rows_fused_kernel<F, SK>), dim3(kRwUpGroups), dim3(kRwFusedBlock), 0, s, f);
        return hipGetLastError();
    }
    hipError_t e = launch_rmsnorm_rows(p.residual + (size_t)m0 * kH, p.pre_rms, ctx->hbuf, M, s);
    if (e != hipSuccess) return e;
    e = rw_launch<F, SK, true>(dim3(kRwUpGroups, 1, 1), s, p, ctx->hbuf, kH, M, ctx->pbuf, nullptr);
    if (e != hipSuccess) return e;
    e = rw_launch<F, SK, false>(dim3(kRwDownGroups, 1, kRwSplits), s, p, ctx->pbuf, kL, M, nullptr, ctx->fbuf);
    if (e != hipSuccess) return e;
    return launch_ffn_post_rows(p, ctx->fbuf, kRwSplits, M, p.residual + (size_t)m0 * kH, s);
}

}  // namespace

hipError_t launch_ffn_rows(const FfnParams& p, int m0, int M, hipStream_t s, DevCtx* ctx) {
    if (M < 1 || M > kMaxDecodeM) return hipErrorInvalidValue;
    switch (p.fmt) {
        case FfnFormat::FP8:
            return p.scale_kind == ScaleKind::F32 ? rows_ffn_impl<FfnFormat::FP8, ScaleKind::F32>(p, m0, M, s, ctx)
                                                  : rows_ffn_impl<FfnFormat::FP8, ScaleKind::BF16>(p, m0, M, s, ctx);
        case FfnFormat::NVFP4: return rows_ffn_impl<FfnFormat::NVFP4, ScaleKind::F32>(p, m0, M, s, ctx);
        case FfnFormat::MXFP4: return rows_ffn_impl<FfnFormat::MXFP4, ScaleKind::F32>(p, m0, M, s, ctx);
    }
    return hipErrorInvalidValue;
}

}  // namespace moa
