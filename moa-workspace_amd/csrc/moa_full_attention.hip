// moa_full_attention.hip -- ops::full_attention_first_page / ops::full_attention_page
// (FO/src/ops.rs:148-174; FO/src/device/full/attention.rs): decode attention of a full-attention
// layer over one 512-slot page of its cache, folded into a running softmax state.
//
// The layer has 16 query heads and one KV head of 512 (FO/src/axes.rs: Gf, Df, Tf). For token row
// m and head h the state after pages 0..p is
//   running_max[h] = the largest score q_h . k_t (scale 1.0) over the valid slots seen so far,
//   running_sum[h] = sum of exp(s_t - running_max[h]) over them,
//   out[h]         = bf16(sum of exp(s_t - running_max[h]) v_t),
// where a slot is valid when its mask value is non-zero. The first page starts the state; each
// later page rescales the old state by exp(old max - new max) and adds its own terms, as
// attend_next_page does. full_attention_output divides out by running_sum. This is the softmax
// of the CPU reference over the valid slots (gemma4.py:180-184, causal SDPA with scale 1.0); the
// RNGD kernel takes its page max over every slot, rounds scores and weights to bf16 and adds 1e-6
// to each page sum, which moves results within rounding.
//
// Two launches per page:
//  1. fattn_partial_kernel, grid (8 slot chunks, 4 dim blocks, M): workgroup (c, b, m) scores the
//     64 slots of chunk c against all 16 heads on the matrix cores (v_mfma_f32_16x16x32_bf16: the
//     heads as A rows, K rows as B columns, 512 = 16 steps of 32), takes each head's max and the
//     f32 exp weights, and multiplies them into its 128 dims of V (V staged through LDS, where the
//     B operand's slot-major gather is cheap). A weight enters the MFMA as two bf16 parts, high
//     and low (about 16 significant bits; one bf16 part alone would put a 2^-9 relative error on
//     every weight). It writes the chunk's per-head max, sum and partial out (f32).
//  2. fattn_combine_kernel, grid (16 heads, M): merges the 8 chunks with the old state and writes
//     the new one. One workgroup owns a head's state, so no other reads it while it is replaced.
#include <hip/hip_runtime.h>

#include "moa_device.h"
#include "moa_internal.h"

namespace moa {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int kFaBlock = 256;
constexpr int kFaChunk = 64;                  // slots per workgroup
constexpr int kFaDims = kDf / kFaDimBlocks;   // 128 dims of V per workgroup
constexpr int kFaVStride = kFaDims + 4;       // LDS row of the V slice, in elements (8-byte aligned rows)
constexpr int kFaPStride = kFaChunk + 8;      // LDS row of the weights, in elements (16-byte aligned rows)
static_assert(kFaChunks * kFaChunk == kTf && kFaRec == 2 * kGf + kGf * kDf, "full attention tiling");

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4& v) { return __builtin_bit_cast(bf16x8, v); }

__global__ __launch_bounds__(kFaBlock) void fattn_partial_kernel(const uint16_t* __restrict__ q,
                                                                 const uint16_t* __restrict__ kc,
                                                                 const uint16_t* __restrict__ vc,
                                                                 const float* __restrict__ mask, float* part) {
    __shared__ __attribute__((aligned(16))) uint16_t vs[kFaChunk * kFaVStride];
    __shared__ __attribute__((aligned(16))) uint16_t ps[2][kGf * kFaPStride];  // exp weights: bf16 high, low parts
    __shared__ float red_m[4][kGf], red_l[4][kGf];
    const int c = blockIdx.x, b = blockIdx.y, m = blockIdx.z;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int slot0 = c * kFaChunk;

    // Wave w scores slots 16 w .. 16 w + 15 of the chunk. Lane l feeds K row (l % 16) and query
    // head (l % 16), k 32 j + 8 (l / 16) .. + 7 of step j.
    const int sl = slot0 + 16 * wave + l16;
    uint4 kb[kDf / 32], qa[kDf / 32];
#pragma unroll
    for (int j = 0; j < kDf / 32; ++j) kb[j] = ld16(kc + (size_t)sl * kDf + 32 * j + 8 * g);
#pragma unroll
    for (int j = 0; j < kDf / 32; ++j) qa[j] = ld16(q + (size_t)m * kQf + l16 * kDf + 32 * j + 8 * g);
    // the chunk's V slice: 64 rows x 128 dims = 1024 units of 16 bytes, thread t takes t + 256 i
    uint4 vv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int u = t + kFaBlock * i, row = u >> 4, cu = u & 15;
        vv[i] = ld16(vc + (size_t)(slot0 + row) * kDf + b * kFaDims + cu * 8);
    }
    const bool valid = mask[(size_t)m * kTf + sl] != 0.0f;

    f32x4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < kDf / 32; ++j)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(qa[j]), as_bf16x8(kb[j]), acc, 0, 0, 0);
    // acc[r]: score of head 4 (l / 16) + r at slot sl
    float sc[4], mx[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        sc[r] = valid ? acc[r] : -INFINITY;
        mx[r] = sc[r];
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) mx[r] = fmaxf(mx[r], __shfl_xor(mx[r], o));
    }
    if (l16 == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) red_m[wave][4 * g + r] = mx[r];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int u = t + kFaBlock * i, row = u >> 4, cu = u & 15;
        uint2* dst = reinterpret_cast<uint2*>(vs + row * kFaVStride + cu * 8);
        dst[0] = make_uint2(vv[i].x, vv[i].y);
        dst[1] = make_uint2(vv[i].z, vv[i].w);
    }
    __syncthreads();
    float ls[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int h = 4 * g + r;
        const float mh = fmaxf(fmaxf(red_m[0][h], red_m[1][h]), fmaxf(red_m[2][h], red_m[3][h]));
        const float pv = sc[r] == -INFINITY ? 0.0f : __expf(sc[r] - mh);
        const uint32_t hi = f2bf(pv);
        ps[0][h * kFaPStride + 16 * wave + l16] = (uint16_t)hi;
        ps[1][h * kFaPStride + 16 * wave + l16] = (uint16_t)f2bf(pv - bf2f(hi));
        ls[r] = pv;
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) ls[r] += __shfl_xor(ls[r], o);
    }
    if (l16 == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) red_l[wave][4 * g + r] = ls[r];
    }
    __syncthreads();

    // out[h][d] = sum_s p[h][s] v[s][d]: wave w takes dims 32 w .. 32 w + 31 of the block (two
    // 16-column tiles), the 64 slots as two k steps of 32. A: weights of head l % 16, slots
    // 32 kk + 8 (l / 16) .. + 7; B: V at those slots, dim l % 16 of the tile.
    f32x4v o[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
        const uint4 a = *reinterpret_cast<const uint4*>(ps[0] + l16 * kFaPStride + 32 * kk + 8 * g);
        const uint4 al = *reinterpret_cast<const uint4*>(ps[1] + l16 * kFaPStride + 32 * kk + 8 * g);
#pragma unroll
        for (int dd = 0; dd < 2; ++dd) {
            const int col = 32 * wave + 16 * dd + l16;
            const uint16_t* vp = vs + (32 * kk + 8 * g) * kFaVStride + col;
            uint32_t w[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) w[i] = (uint32_t)vp[(2 * i) * kFaVStride] | ((uint32_t)vp[(2 * i + 1) * kFaVStride] << 16);
            const bf16x8 bv = as_bf16x8(make_uint4(w[0], w[1], w[2], w[3]));
            o[dd] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), bv, o[dd], 0, 0, 0);
            o[dd] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(al), bv, o[dd], 0, 0, 0);
        }
    }
    float* pc = part + ((size_t)m * kFaChunks + c) * kFaRec;
    if (b == 0 && t < kGf) {
        pc[t] = fmaxf(fmaxf(red_m[0][t], red_m[1][t]), fmaxf(red_m[2][t], red_m[3][t]));
        pc[kGf + t] = ((red_l[0][t] + red_l[1][t]) + red_l[2][t]) + red_l[3][t];
    }
#pragma unroll
    for (int dd = 0; dd < 2; ++dd)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            pc[2 * kGf + (4 * g + r) * kDf + b * kFaDims + 32 * wave + 16 * dd + l16] = o[dd][r];
}

// Workgroup (h, m) merges head h's 8 chunk partials into the row's state; thread t owns dims
// 2 t, 2 t + 1.
__global__ __launch_bounds__(kFaBlock) void fattn_combine_kernel(const float* __restrict__ part, float* rmax,
                                                                 float* rsum, uint16_t* out, int first) {
    const int h = blockIdx.x, m = blockIdx.y, t = threadIdx.x;
    const float* pm = part + (size_t)m * kFaChunks * kFaRec;
    float mc[kFaChunks], lc[kFaChunks];
    float2 oc[kFaChunks];
#pragma unroll
    for (int c = 0; c < kFaChunks; ++c) {
        mc[c] = pm[c * kFaRec + h];
        lc[c] = pm[c * kFaRec + kGf + h];
        oc[c] = *reinterpret_cast<const float2*>(pm + c * kFaRec + 2 * kGf + h * kDf + 2 * t);
    }
    const size_t sh = (size_t)m * kGf + h;
    uint32_t* op = reinterpret_cast<uint32_t*>(out + sh * kDf) + t;
    const float om = first ? -INFINITY : rmax[sh];
    const float os = first ? 0.0f : rsum[sh];
    const uint32_t ob = first ? 0u : *op;
    __syncthreads();  // every wave has read the old state before thread 0 replaces it

    float mp = -INFINITY;
#pragma unroll
    for (int c = 0; c < kFaChunks; ++c) mp = fmaxf(mp, mc[c]);
    const float mn = fmaxf(om, mp);
    float l = 0.0f, o0 = 0.0f, o1 = 0.0f;
    if (mn != -INFINITY) {
        const float ro = om == -INFINITY ? 0.0f : __expf(om - mn);
        l = ro * os;
        o0 = ro * bf2f(ob & 0xffffu);
        o1 = ro * bf2f(ob >> 16);
#pragma unroll
        for (int c = 0; c < kFaChunks; ++c) {
            const float f = mc[c] == -INFINITY ? 0.0f : __expf(mc[c] - mn);
            l = fmaf(f, lc[c], l);
            o0 = fmaf(f, oc[c].x, o0);
            o1 = fmaf(f, oc[c].y, o1);
        }
    }
    *op = f2bf(o0) | (f2bf(o1) << 16);
    if (t == 0) {
        rmax[sh] = mn;
        rsum[sh] = l;
    }
}

}  // namespace

hipError_t launch_full_attention_page(const uint16_t* q, const uint16_t* k_page, const uint16_t* v_page,
                                      const float* mask, float* running_max, float* running_sum, uint16_t* out,
                                      int M, bool first, hipStream_t s, DevCtx* ctx) {
    for (int m0 = 0; m0 < M; m0 += kMaxDecodeM) {
        const int mm = M - m0 < kMaxDecodeM ? M - m0 : kMaxDecodeM;
        hipLaunchKernelGGL(fattn_partial_kernel, dim3(kFaChunks, kFaDimBlocks, mm), dim3(kFaBlock), 0, s,
                           q + (size_t)m0 * kQf, k_page, v_page, mask + (size_t)m0 * kTf, ctx->fattn_part);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(fattn_combine_kernel, dim3(kGf, mm), dim3(kFaBlock), 0, s, (const float*)ctx->fattn_part,
                           running_max + (size_t)m0 * kGf, running_sum + (size_t)m0 * kGf, out + (size_t)m0 * kQf,
                           first ? 1 : 0);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace moa
