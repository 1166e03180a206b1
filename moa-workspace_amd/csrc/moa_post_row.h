// moa_post_row.h -- the last row step of a split-K contraction whose output is added to the
// residual (the FFN's down projection, O): the partial sums, the format's commit, post-RMSNorm,
// residual and layer scalar for one row, by four waves. Shared by the chunk and rows paths, so
// that every path that ends in it gives the same bits.
#pragma once

#include <hip/hip_runtime.h>

#include "moa_device.h"
#include "moa_internal.h"

namespace moa {
namespace {

template <ScaleKind SK>
__device__ __forceinline__ float chunk_scale(const void* p, int i) {
    if constexpr (SK == ScaleKind::F32) return static_cast<const float*>(p)[i];
    else return bf2f(static_cast<const uint16_t*>(p)[i]);
}

// Block sum over the four waves, in wave order.
__device__ __forceinline__ float ck_block_sum(float v, float* red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return ((red[0] + red[1]) + red[2]) + red[3];
}

// Row RMSNorm by four waves: thread t < kH / 16 holds elements 16 t .. 16 t + 15 of the row (xv)
// and their weights (wv); h receives the 8 bf16 pairs of bf16(x * inv * w) (gemma4.py:83-89).
// Threads past the row take part in the sum with nothing.
__device__ __forceinline__ void rms_row_values(const float (&xv)[16], const float (&wv)[16], float* red, uint32_t (&h)[8]) {
    const bool act = threadIdx.x < kH / 16;
    float ss = 0.0f;
    if (act) {
#pragma unroll
        for (int i = 0; i < 16; ++i) ss = fmaf(xv[i], xv[i], ss);
    }
    const float inv = rms_inverse(ck_block_sum(ss, red), kH);
#pragma unroll
    for (int i = 0; i < 8; ++i)
        h[i] = pk_bf16((xv[2 * i] * inv) * wv[2 * i], (xv[2 * i + 1] * inv) * wv[2 * i + 1]);
}

// Per row: d = bf16((sum of the split-K partials) * s[n]), then out = bf16(bf16(r + N(d)) * ls)
// with N the post-RMSNorm (identity when w_post is null) and ls skipped when null
// (shared/rmsnorm.rs:204-296, residual.rs:189-241; generate_references.py:411-413).
// ZS: the most splits a call may have (the loads of all of them are in flight at once).
// Row m; out[i] returns thread t's stored chunk t + 256 i (8 bf16 values) of the new residual.
// rlds: the row's current residual in LDS (480 chunks of 8), read instead of res when given (a
// caller that has just written the row itself).
template <ScaleKind SK, FfnFormat F, int ZS>
__device__ __forceinline__ void post_row(const float* __restrict__ part, int splits, int M, const void* scale,
                                         const float* __restrict__ gscale, const uint16_t* __restrict__ w_post,
                                         uint16_t* __restrict__ res, const uint16_t* __restrict__ ls, int m, float* red,
                                         uint4 (&out)[2], const uint4* rlds = nullptr) {
    const int t = threadIdx.x;
    const float gs = F == FfnFormat::NVFP4 ? *gscale : 1.0f;
    constexpr int NC = kH / 8;  // 480 chunks of 8; thread t owns t and t + 256
    float d[2][8];
    float ss = 0.0f;
    // the residual and post-norm weight chunks are loaded first, in flight during the partial sums
    uint4 rq[2], wq[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = min(t + 256 * i, NC - 1);
        rq[i] = rlds ? rlds[c] : ld16(res + (size_t)m * kH + c * 8);
        wq[i] = w_post ? ld16(w_post + c * 8) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = min(t + 256 * i, NC - 1);
        const bool act = t + 256 * i < NC;
        // all partial loads in flight at once (index clamped), then summed in split order
        float4 u[ZS], v[ZS];
#pragma unroll
        for (int z = 0; z < ZS; ++z) {
            const float* src = part + ((size_t)min(z, splits - 1) * M + m) * kH + c * 8;
            u[z] = *reinterpret_cast<const float4*>(src);
            v[z] = *reinterpret_cast<const float4*>(src + 4);
        }
        float a[8] = {u[0].x, u[0].y, u[0].z, u[0].w, v[0].x, v[0].y, v[0].z, v[0].w};
#pragma unroll
        for (int z = 1; z < ZS; ++z) {
            const bool on = z < splits;
            a[0] = on ? a[0] + u[z].x : a[0]; a[1] = on ? a[1] + u[z].y : a[1];
            a[2] = on ? a[2] + u[z].z : a[2]; a[3] = on ? a[3] + u[z].w : a[3];
            a[4] = on ? a[4] + v[z].x : a[4]; a[5] = on ? a[5] + v[z].y : a[5];
            a[6] = on ? a[6] + v[z].z : a[6]; a[7] = on ? a[7] + v[z].w : a[7];
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            // the format's commit: FP8 bf16(sum * s[n]); NVFP4 bf16(bf16(sum) * 1/g); MXFP4 bf16(sum)
            if constexpr (F == FfnFormat::FP8) d[i][e] = rbf(a[e] * chunk_scale<SK>(scale, c * 8 + e));
            else if constexpr (F == FfnFormat::NVFP4) d[i][e] = rbf(rbf(a[e]) * gs);
            else d[i][e] = rbf(a[e]);
            if (act) ss = fmaf(d[i][e], d[i][e], ss);
        }
    }
    const float inv = w_post ? rms_inverse(ck_block_sum(ss, red), kH) : 1.0f;
    const float lsv = ls ? bf2f(ls[0]) : 1.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = t + 256 * i;
        if (c >= NC) continue;
        uint16_t* rr = res + (size_t)m * kH + c * 8;
        float rv[8], wv[8];
        bf16x8_to_f32(rq[i], rv);
        bf16x8_to_f32(wq[i], wv);
        uint32_t pk[4];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float n = d[i][e];
            if (w_post) n = rbf((n * inv) * wv[e]);
            float sres = rbf(rv[e] + n);
            if (ls) sres = rbf(sres * lsv);
            const uint32_t b = f2bf(sres);
            if (e & 1) pk[e >> 1] |= b << 16; else pk[e >> 1] = b;
        }
        out[i] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        *reinterpret_cast<uint4*>(rr) = out[i];
    }
}

}  // namespace
}  // namespace moa
