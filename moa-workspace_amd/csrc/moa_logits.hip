// moa_logits.hip -- ops::final_norm_and_logits (FO/src/ops.rs:241-298): the final RMSNorm, the
// lm_head GEMV over 262144 bf16 vocabulary rows (2.01 GB, the largest byte mover per token), and
// Gemma's logit softcap (gemma4.py:256-261, torch bf16 semantics: one rounding per op).
//
// Streaming GEMV, HBM-bound: each wave takes 8 vocabulary rows at a time, 8 lanes per row, each
// lane 16 bytes (8 bf16) per load. Those are units j, j + 8, ... of the row's 480 units, and for
// the 8 lanes of a row one load moves 128 contiguous bytes. The normalised input rows sit in LDS;
// the 8 row groups of a wave read the same x units (LDS broadcast). Loads run kLgDepth units
// ahead through a register ring, across row boundaries. The 8 partial sums of a row meet in three
// lane exchanges; lane 0 of the row group applies the softcap and stores the bf16 logit.
#include <hip/hip_runtime.h>

#include "moa_device.h"
#include "moa_internal.h"

namespace moa {
namespace {

constexpr int kLgBlock = 256;                       // four waves
constexpr int kLgUnits = kH / 8;                    // 480 units of 16 bytes per row
constexpr int kLgUnitsLane = kLgUnits / 8;          // 60 per lane
constexpr int kLgDepth = 10;                        // units in flight per lane (60 % 10 == 0)
constexpr int kLgRowsWg = 256;                      // vocabulary rows per workgroup
constexpr int kLgGrid = kW / kLgRowsWg;             // 1024 workgroups
constexpr int kLgIters = kLgRowsWg / (4 * 8);       // 8 row groups of 8 rows per wave
static_assert(kLgUnitsLane % kLgDepth == 0 && kW % kLgRowsWg == 0, "logits tiling");

// MB: token rows per launch (1, or up to 16 with the rest masked).
template <int MB>
__global__ __launch_bounds__(kLgBlock) void logits_kernel(const uint16_t* __restrict__ input, const uint16_t* __restrict__ rms_w,
                                                          const uint16_t* __restrict__ w, uint16_t* __restrict__ out, int M) {
    __shared__ __attribute__((aligned(16))) uint16_t xs[MB][kH];
    __shared__ float red[4];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int j = lane & 7, grp = lane >> 3;

    // first row group's loads go out before the input norm
    const int row_base = blockIdx.x * kLgRowsWg + wave * 8 + grp;  // + 32 it
    auto wptr = [&](int it, int i) { return w + (size_t)(row_base + 32 * it) * kH + (j + 8 * i) * 8; };
    uint4 ring[kLgDepth];
#pragma unroll
    for (int d = 0; d < kLgDepth; ++d) ring[d] = ld_stream(wptr(0, d));

    // RMSNorm of the token rows into LDS (FO/src/device/shared/rmsnorm.rs; gemma4.py:83-89):
    // thread t < 240 owns elements 16 t .. 16 t + 15
    for (int m = 0; m < M && m < MB; ++m) {
        const bool act = t < kH / 16;
        const int c = min(t, kH / 16 - 1);
        float xv[16], wv[16];
        bf16x8_to_f32(ld16(input + (size_t)m * kH + c * 16), xv);
        bf16x8_to_f32(ld16(input + (size_t)m * kH + c * 16 + 8), xv + 8);
        bf16x8_to_f32(ld16(rms_w + c * 16), wv);
        bf16x8_to_f32(ld16(rms_w + c * 16 + 8), wv + 8);
        float ss = 0.0f;
        if (act) {
#pragma unroll
            for (int i = 0; i < 16; ++i) ss = fmaf(xv[i], xv[i], ss);
        }
        ss = wave_sum(ss);
        __syncthreads();
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        const float inv = rms_inverse(((red[0] + red[1]) + red[2]) + red[3], kH);
        if (act) {
            uint32_t h[8];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                h[i] = pk_bf16((xv[2 * i] * inv) * wv[2 * i], (xv[2 * i + 1] * inv) * wv[2 * i + 1]);
            *reinterpret_cast<uint4*>(&xs[m][c * 16]) = make_uint4(h[0], h[1], h[2], h[3]);
            *reinterpret_cast<uint4*>(&xs[m][c * 16 + 8]) = make_uint4(h[4], h[5], h[6], h[7]);
        }
    }
    __syncthreads();

    for (int it = 0; it < kLgIters; ++it) {
        float acc[MB];
#pragma unroll
        for (int m = 0; m < MB; ++m) acc[m] = 0.0f;
#pragma unroll
        for (int i = 0; i < kLgUnitsLane; ++i) {
            const uint4 q = ring[i % kLgDepth];
            // refill: unit i + kLgDepth of this row, or unit i + kLgDepth - 60 of the next row
            // group (the last group re-reads its own row, in bounds and unused)
            if (i + kLgDepth < kLgUnitsLane) ring[i % kLgDepth] = ld_stream(wptr(it, i + kLgDepth));
            else ring[i % kLgDepth] = ld_stream(wptr(min(it + 1, kLgIters - 1), i + kLgDepth - kLgUnitsLane));
            const uint32_t wq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int m = 0; m < MB; ++m) {
                if (m < M) {
                    const uint4 xq = *reinterpret_cast<const uint4*>(&xs[m][(j + 8 * i) * 8]);
                    const uint32_t xw[4] = {xq.x, xq.y, xq.z, xq.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[m] = dot2_bf16(xw[e], __builtin_bit_cast(bf16x2, wq[e]), acc[m]);
                }
            }
        }
        const int row = row_base + 32 * it;
#pragma unroll
        for (int m = 0; m < MB; ++m) {
            if (m < M) {
                float a = acc[m];
                a += __shfl_xor(a, 1);
                a += __shfl_xor(a, 2);
                a += __shfl_xor(a, 4);
                // the lm_head linear's output is bf16 (FO/src/ops.rs:252, cast to f32 at :264)
                if (j == 0) out[(size_t)m * kW + row] = (uint16_t)softcap30_bf16(rbf(a));
            }
        }
    }
}

}  // namespace

hipError_t launch_final_norm_and_logits(const uint16_t* input, const uint16_t* rms_w, const uint16_t* w, uint16_t* out,
                                        int M, hipStream_t s) {
    for (int m0 = 0; m0 < M; m0 += 16) {
        const int mm = M - m0 < 16 ? M - m0 : 16;
        if (mm == 1)
            hipLaunchKernelGGL(logits_kernel<1>, dim3(kLgGrid), dim3(kLgBlock), 0, s, input + (size_t)m0 * kH, rms_w, w,
                               out + (size_t)m0 * kW, mm);
        else
            hipLaunchKernelGGL(logits_kernel<16>, dim3(kLgGrid), dim3(kLgBlock), 0, s, input + (size_t)m0 * kH, rms_w, w,
                               out + (size_t)m0 * kW, mm);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace moa
