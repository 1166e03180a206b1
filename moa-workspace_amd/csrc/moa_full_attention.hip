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
//     heads as A rows, K rows as B columns, each wave a quarter of the 512 dims), takes each
//     head's max and the f32 exp weights, and multiplies them into its 128 dims of V (V staged
//     through LDS, where the B operand's slot-major gather is cheap). A weight enters the MFMA as two bf16 parts, high
//     and low (about 16 significant bits; one bf16 part alone would put a 2^-9 relative error on
//     every weight). It writes the chunk's per-head max, sum and partial out (f32).
//  2. fattn_combine_kernel, grid (16 heads, M): merges the 8 chunks with the old state and writes
//     the new one. One workgroup owns a head's state, so no other reads it while it is replaced.
//
// moa_full_attention computes the same state over pages 0 .. P - 1 in two launches instead of 2 P:
// the partial pass runs over every page at once -- up to 8 pages with the dim-split kernel (one
// chunk per workgroup), beyond with fattn_span_kernel (a workgroup takes a span of chunks over all
// dims with an online softmax; at most 256 records per row) -- and fattn_merge_kernel merges the
// records with a grid of (16 heads, 8 dim blocks): no old state is read, so the split is free of
// races.
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

// Workgroup (x, b, m) of the partial pass: chunks u = x * cpw .. min(x * cpw + cpw, nchunks) - 1 of
// the row's slots (chunk u = slots 64 (u % 8) .. + 63 of page u / 8; pages lie kTf * kDf apart),
// dims 128 b .. 128 b + 127 of V. Across its chunks it keeps an online softmax per head: the
// running max, the sum of exp and out for its dims, rescaled whenever the max grows. Its record
// of part (record x of row m, kFaRec floats): max[16], sum[16], out[16][512] (its 128 dims).
//
// Scores are split by dims: wave w multiplies dims 128 w .. 128 w + 127 of the chunk's 64 K rows
// (four 16-slot tiles) with the 16 heads, so each wave loads a quarter of q once; the four partial
// score tiles meet in LDS. Two register stages hold a chunk's K rows and V slice: the next chunk's
// loads go out at the top of each step, ahead of the current chunk's work.
__global__ __launch_bounds__(kFaBlock) void fattn_partial_kernel(const uint16_t* __restrict__ q,
                                                                 const uint16_t* __restrict__ kc,
                                                                 const uint16_t* __restrict__ vc,
                                                                 const float* __restrict__ mask, int mask_page_stride,
                                                                 int nchunks, int cpw, float* part) {
    __shared__ __attribute__((aligned(16))) uint16_t vs[kFaChunk * kFaVStride];
    __shared__ __attribute__((aligned(16))) uint16_t ps[2][kGf * kFaPStride];  // exp weights: bf16 high, low parts
    __shared__ float sp[4][kGf * kFaChunk];                                   // per-wave partial scores [head][slot]
    __shared__ float red_m[4][kGf], red_l[4][kGf];
    const int b = blockIdx.y, m = blockIdx.z;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int u0 = blockIdx.x * cpw, u1 = min(u0 + cpw, nchunks);

    // Lane l feeds head l % 16 and, of tile st, slot 16 st + l % 16, k 128 w + 32 j + 8 (l / 16) .. + 7
    // of step j. The V slice (64 rows x 128 dims = 1024 units of 16 bytes) is spread as units
    // t + 256 i. The lane's softmax slot is 16 w + l % 16 (its mask value rides with the stage).
    uint4 qa[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) qa[j] = ld16(q + (size_t)m * kQf + l16 * kDf + 128 * wave + 32 * j + 8 * g);
    auto issue = [&](int u, uint4 (&kr)[4][4], uint4 (&vr)[4], float& mk) {
        const int page = u / kFaChunks, s0 = (u % kFaChunks) * kFaChunk;
        const uint16_t* kp = kc + ((size_t)page * kTf + s0 + l16) * kDf + 128 * wave + 8 * g;
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
            for (int j = 0; j < 4; ++j) kr[st][j] = ld16(kp + (size_t)16 * st * kDf + 32 * j);
        const uint16_t* vp = vc + ((size_t)page * kTf + s0) * kDf + b * kFaDims;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int un = t + kFaBlock * i, row = un >> 4, cu = un & 15;
            vr[i] = ld16(vp + (size_t)row * kDf + cu * 8);
        }
        mk = mask[(size_t)page * mask_page_stride + (size_t)m * kTf + s0 + 16 * wave + l16];
    };

    float m_run[4], l_run[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        m_run[r] = -INFINITY;
        l_run[r] = 0.0f;
    }
    f32x4v o[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
    auto step = [&](int u, const uint4 (&kr)[4][4], const uint4 (&vr)[4], float mk, uint4 (&kn)[4][4], uint4 (&vn)[4],
                    float& mkn) {
        __syncthreads();                              // the previous chunk's LDS reads are done
        if (u + 1 < u1) issue(u + 1, kn, vn, mkn);    // the next chunk's loads go out first
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            f32x4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(qa[j]), as_bf16x8(kr[st][j]), acc, 0, 0, 0);
            // acc[r]: the wave's part of the score of head 4 (l / 16) + r at slot 16 st + l % 16
#pragma unroll
            for (int r = 0; r < 4; ++r) sp[wave][(4 * g + r) * kFaChunk + 16 * st + l16] = acc[r];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int un = t + kFaBlock * i, row = un >> 4, cu = un & 15;
            uint2* dst = reinterpret_cast<uint2*>(vs + row * kFaVStride + cu * 8);
            dst[0] = make_uint2(vr[i].x, vr[i].y);
            dst[1] = make_uint2(vr[i].z, vr[i].w);
        }
        __syncthreads();
        const bool valid = mk != 0.0f;
        float sc[4], mx[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int at = (4 * g + r) * kFaChunk + 16 * wave + l16;
            const float sv = ((sp[0][at] + sp[1][at]) + sp[2][at]) + sp[3][at];
            sc[r] = valid ? sv : -INFINITY;
            mx[r] = sc[r];
#pragma unroll
            for (int sh = 1; sh < 16; sh <<= 1) mx[r] = fmaxf(mx[r], __shfl_xor(mx[r], sh));
        }
        if (l16 == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) red_m[wave][4 * g + r] = mx[r];
        }
        __syncthreads();
        float scale[4], ls[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int h = 4 * g + r;
            const float mc = fmaxf(fmaxf(red_m[0][h], red_m[1][h]), fmaxf(red_m[2][h], red_m[3][h]));
            const float mn = fmaxf(m_run[r], mc);
            scale[r] = m_run[r] == -INFINITY ? 0.0f : __expf(m_run[r] - mn);
            m_run[r] = mn;
            const float pv = sc[r] == -INFINITY ? 0.0f : __expf(sc[r] - mn);
            const uint32_t hi = f2bf(pv);
            ps[0][h * kFaPStride + 16 * wave + l16] = (uint16_t)hi;
            ps[1][h * kFaPStride + 16 * wave + l16] = (uint16_t)f2bf(pv - bf2f(hi));
            ls[r] = pv;
#pragma unroll
            for (int sh = 1; sh < 16; sh <<= 1) ls[r] += __shfl_xor(ls[r], sh);
        }
        if (l16 == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) red_l[wave][4 * g + r] = ls[r];
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int h = 4 * g + r;
            l_run[r] = fmaf(l_run[r], scale[r], ((red_l[0][h] + red_l[1][h]) + red_l[2][h]) + red_l[3][h]);
#pragma unroll
            for (int dd = 0; dd < 2; ++dd) o[dd][r] *= scale[r];
        }
        // out[h][d] += sum_s p[h][s] v[s][d]: wave w takes dims 32 w .. 32 w + 31 of the block (two
        // 16-column tiles), the 64 slots as two k steps of 32. A: weights of head l % 16, slots
        // 32 kk + 8 (l / 16) .. + 7; B: V at those slots, dim l % 16 of the tile.
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
                for (int i = 0; i < 4; ++i)
                    w[i] = (uint32_t)vp[(2 * i) * kFaVStride] | ((uint32_t)vp[(2 * i + 1) * kFaVStride] << 16);
                const bf16x8 bv = as_bf16x8(make_uint4(w[0], w[1], w[2], w[3]));
                o[dd] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), bv, o[dd], 0, 0, 0);
                o[dd] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(al), bv, o[dd], 0, 0, 0);
            }
        }
    };
    uint4 kA[4][4], vA[4], kB[4][4], vB[4];
    float mA = 0.0f, mB = 0.0f;
    issue(u0, kA, vA, mA);
    for (int u = u0; u < u1; u += 2) {
        step(u, kA, vA, mA, kB, vB, mB);
        if (u + 1 < u1) step(u + 1, kB, vB, mB, kA, vA, mA);
    }
    float* pc = part + ((size_t)m * gridDim.x + blockIdx.x) * kFaRec;
    if (b == 0 && l16 == 0 && wave == 0) {  // every wave holds the same per-head values
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            pc[4 * g + r] = m_run[r];
            pc[kGf + 4 * g + r] = l_run[r];
        }
    }
#pragma unroll
    for (int dd = 0; dd < 2; ++dd)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            pc[2 * kGf + (4 * g + r) * kDf + b * kFaDims + 32 * wave + 16 * dd + l16] = o[dd][r];
}

// The span kernel of moa_full_attention for more than 8 pages: workgroup (x, 0, m) takes chunks
// x * cpw .. of row m over all 512 dims, so every K row and V row is read from memory once (the
// dim-split partial kernel above reads a chunk's K rows in each of its 4 dim-block workgroups).
// The chunk's V rows (64 KB) go straight to LDS (global_load_lds, no registers) in rows of 1040
// bytes; the next chunk's K rows are requested before this chunk's products, its V rows once
// they are done. Scores are split by dims as above. Record x of row m holds all 512 dims.
constexpr int kFsVRow = kDf + 8;  // LDS row of the V chunk, in elements (1040 bytes)
typedef __attribute__((address_space(3))) void fa_lds_void;
typedef __attribute__((address_space(1))) void fa_glb_void;

__global__ __launch_bounds__(kFaBlock) void fattn_span_kernel(const uint16_t* __restrict__ q,
                                                              const uint16_t* __restrict__ kc,
                                                              const uint16_t* __restrict__ vc,
                                                              const float* __restrict__ mask, int mask_page_stride,
                                                              int nchunks, int cpw, float* part) {
    __shared__ __attribute__((aligned(16))) uint16_t vsm[kFaChunk * kFsVRow];
    __shared__ __attribute__((aligned(16))) uint16_t ps[2][kGf * kFaPStride];
    __shared__ float sp[4][kGf * kFaChunk];
    __shared__ float red_m[4][kGf], red_l[4][kGf];
    const int m = blockIdx.z;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int u0 = blockIdx.x * cpw, u1 = min(u0 + cpw, nchunks);

    uint4 qa[4], kr[4][4];
    float mk = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) qa[j] = ld16(q + (size_t)m * kQf + l16 * kDf + 128 * wave + 32 * j + 8 * g);
    auto issue_k = [&](int u) {
        const int page = u / kFaChunks, s0 = (u % kFaChunks) * kFaChunk;
        const uint16_t* kp = kc + ((size_t)page * kTf + s0 + l16) * kDf + 128 * wave + 8 * g;
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
            for (int j = 0; j < 4; ++j) kr[st][j] = ld16(kp + (size_t)16 * st * kDf + 32 * j);
        mk = mask[(size_t)page * mask_page_stride + (size_t)m * kTf + s0 + 16 * wave + l16];
    };
    auto issue_v = [&](int u) {  // wave w moves rows 16 w .. 16 w + 15, one 1 KB row per instruction
        const int page = u / kFaChunks, s0 = (u % kFaChunks) * kFaChunk;
        const uint16_t* vp = vc + ((size_t)page * kTf + s0) * kDf;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int row = 16 * wave + i;
            __builtin_amdgcn_global_load_lds((fa_glb_void*)(vp + (size_t)row * kDf + lane * 8),
                                             (fa_lds_void*)(vsm + row * kFsVRow), 16, 0, 0);
        }
    };
    issue_k(u0);
    issue_v(u0);

    float m_run[4], l_run[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        m_run[r] = -INFINITY;
        l_run[r] = 0.0f;
    }
    f32x4v o[8];
#pragma unroll
    for (int dd = 0; dd < 8; ++dd) o[dd] = f32x4v{0.0f, 0.0f, 0.0f, 0.0f};
    for (int u = u0; u < u1; ++u) {
        __syncthreads();  // the previous chunk's score and weight reads are done
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            f32x4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(qa[j]), as_bf16x8(kr[st][j]), acc, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) sp[wave][(4 * g + r) * kFaChunk + 16 * st + l16] = acc[r];
        }
        const bool valid = mk != 0.0f;
        __syncthreads();
        float sc[4], mx[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int at = (4 * g + r) * kFaChunk + 16 * wave + l16;
            const float sv = ((sp[0][at] + sp[1][at]) + sp[2][at]) + sp[3][at];
            sc[r] = valid ? sv : -INFINITY;
            mx[r] = sc[r];
#pragma unroll
            for (int sh = 1; sh < 16; sh <<= 1) mx[r] = fmaxf(mx[r], __shfl_xor(mx[r], sh));
        }
        if (l16 == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) red_m[wave][4 * g + r] = mx[r];
        }
        __syncthreads();
        float scale[4], ls[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int h = 4 * g + r;
            const float mc = fmaxf(fmaxf(red_m[0][h], red_m[1][h]), fmaxf(red_m[2][h], red_m[3][h]));
            const float mn = fmaxf(m_run[r], mc);
            scale[r] = m_run[r] == -INFINITY ? 0.0f : __expf(m_run[r] - mn);
            m_run[r] = mn;
            const float pv = sc[r] == -INFINITY ? 0.0f : __expf(sc[r] - mn);
            const uint32_t hi = f2bf(pv);
            ps[0][h * kFaPStride + 16 * wave + l16] = (uint16_t)hi;
            ps[1][h * kFaPStride + 16 * wave + l16] = (uint16_t)f2bf(pv - bf2f(hi));
            ls[r] = pv;
#pragma unroll
            for (int sh = 1; sh < 16; sh <<= 1) ls[r] += __shfl_xor(ls[r], sh);
        }
        if (l16 == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) red_l[wave][4 * g + r] = ls[r];
        }
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's V rows have landed in LDS
        __syncthreads();                                     // and every other wave's
        if (u + 1 < u1) issue_k(u + 1);                      // K registers are free
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int h = 4 * g + r;
            l_run[r] = fmaf(l_run[r], scale[r], ((red_l[0][h] + red_l[1][h]) + red_l[2][h]) + red_l[3][h]);
#pragma unroll
            for (int dd = 0; dd < 8; ++dd) o[dd][r] *= scale[r];
        }
        // out[h][d] += sum_s p[h][s] v[s][d]: wave w takes dims 128 w .. 128 w + 127 (eight 16-column
        // tiles), the 64 slots as two k steps of 32.
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const uint4 a = *reinterpret_cast<const uint4*>(ps[0] + l16 * kFaPStride + 32 * kk + 8 * g);
            const uint4 al = *reinterpret_cast<const uint4*>(ps[1] + l16 * kFaPStride + 32 * kk + 8 * g);
#pragma unroll
            for (int dd = 0; dd < 8; ++dd) {
                const uint16_t* vp = vsm + (32 * kk + 8 * g) * kFsVRow + 128 * wave + 16 * dd + l16;
                uint32_t w[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    w[i] = (uint32_t)vp[(2 * i) * kFsVRow] | ((uint32_t)vp[(2 * i + 1) * kFsVRow] << 16);
                const bf16x8 bv = as_bf16x8(make_uint4(w[0], w[1], w[2], w[3]));
                o[dd] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), bv, o[dd], 0, 0, 0);
                o[dd] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(al), bv, o[dd], 0, 0, 0);
            }
        }
        __syncthreads();  // the V chunk's reads are done
        if (u + 1 < u1) issue_v(u + 1);
    }
    float* pc = part + ((size_t)m * gridDim.x + blockIdx.x) * kFaRec;
    if (l16 == 0 && wave == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            pc[4 * g + r] = m_run[r];
            pc[kGf + 4 * g + r] = l_run[r];
        }
    }
#pragma unroll
    for (int dd = 0; dd < 8; ++dd)
#pragma unroll
        for (int r = 0; r < 4; ++r) pc[2 * kGf + (4 * g + r) * kDf + 128 * wave + 16 * dd + l16] = o[dd][r];
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
    *op = pk_bf16(o0, o1);
    if (t == 0) {
        rmax[sh] = mn;
        rsum[sh] = l;
    }
}

// The fused pass (state from scratch): workgroup (h, db, m) merges the nrec records of row m for
// head h, dims 64 db .. 64 db + 63. Thread t takes records t / 32, t / 32 + 8, ... (up to 32) and dims
// 2 (t % 32), + 1 of the block, every load issued before any is used; the 8 record groups meet in
// LDS in a fixed order. Records of chunks with no valid slot hold max -inf and add nothing.
constexpr int kFmGroups = 8;
constexpr int kFmDims = 64;
constexpr int kFmRpg = kFaMaxRecords / kFmGroups;

__global__ __launch_bounds__(kFaBlock) void fattn_merge_kernel(const float* __restrict__ part, int nrec, float* rmax,
                                                               float* rsum, uint16_t* out) {
    __shared__ float wm[kFmGroups], wl[kFmGroups];
    __shared__ float2 wo[kFmGroups][kFmDims / 2];
    const int h = blockIdx.x, db = blockIdx.y, m = blockIdx.z;
    const int t = threadIdx.x, rg = t / (kFmDims / 2), dp = t % (kFmDims / 2);
    const float* pm = part + (size_t)m * nrec * kFaRec;
    const int d = db * kFmDims + 2 * dp;
    float mr[kFmRpg], lr[kFmRpg];
    float2 ov[kFmRpg];
#pragma unroll
    for (int i = 0; i < kFmRpg; ++i) {
        const int x = rg + kFmGroups * i;
        const float* rec = pm + (size_t)min(x, nrec - 1) * kFaRec;
        mr[i] = x < nrec ? rec[h] : -INFINITY;
        lr[i] = rec[kGf + h];
        ov[i] = *reinterpret_cast<const float2*>(rec + 2 * kGf + h * kDf + d);
    }
    float mw = -INFINITY;
#pragma unroll
    for (int i = 0; i < kFmRpg; ++i) mw = fmaxf(mw, mr[i]);
    if (dp == 0) wm[rg] = mw;
    __syncthreads();
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < kFmGroups; ++k) mx = fmaxf(mx, wm[k]);
    float l = 0.0f, o0 = 0.0f, o1 = 0.0f;
    if (mx != -INFINITY) {
#pragma unroll
        for (int i = 0; i < kFmRpg; ++i) {
            const float f = mr[i] == -INFINITY ? 0.0f : __expf(mr[i] - mx);
            l = fmaf(f, lr[i], l);
            o0 = fmaf(f, ov[i].x, o0);
            o1 = fmaf(f, ov[i].y, o1);
        }
    }
    if (dp == 0) wl[rg] = l;
    wo[rg][dp] = make_float2(o0, o1);
    __syncthreads();
    if (rg != 0) return;
    float s0 = 0.0f, s1 = 0.0f, sl = 0.0f;
#pragma unroll
    for (int k = 0; k < kFmGroups; ++k) {
        s0 += wo[k][dp].x;
        s1 += wo[k][dp].y;
        sl += wl[k];
    }
    const size_t sh = (size_t)m * kGf + h;
    *reinterpret_cast<uint32_t*>(out + sh * kDf + d) = pk_bf16(s0, s1);
    if (db == 0 && dp == 0) {
        rmax[sh] = mx;
        rsum[sh] = sl;
    }
}

}  // namespace

hipError_t launch_full_attention(const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages,
                                 const float* masks, int P, float* running_max, float* running_sum, uint16_t* out,
                                 int M, hipStream_t s, DevCtx* ctx) {
    const int nchunks = P * kFaChunks;
    // Up to kFaSplitPages pages: one chunk per dim-split workgroup (P x 32 workgroups). More: spans
    // of chunks over all dims, at most kFaMaxRecords workgroups per row.
    const bool split = P <= kFaSplitPages;
    const int cpw = split ? 1 : (nchunks + kFaMaxRecords - 1) / kFaMaxRecords;
    const int nrec = (nchunks + cpw - 1) / cpw;
    const int rows = kFattnRecords / nrec;  // rows per launch (scratch)
    for (int m0 = 0; m0 < M; m0 += rows) {
        const int mm = M - m0 < rows ? M - m0 : rows;
        if (split)
            hipLaunchKernelGGL(fattn_partial_kernel, dim3(nrec, kFaDimBlocks, mm), dim3(kFaBlock), 0, s,
                               q + (size_t)m0 * kQf, k_pages, v_pages, masks + (size_t)m0 * kTf, M * kTf, nchunks,
                               cpw, ctx->fattn_part);
        else
            hipLaunchKernelGGL(fattn_span_kernel, dim3(nrec, 1, mm), dim3(kFaBlock), 0, s, q + (size_t)m0 * kQf,
                               k_pages, v_pages, masks + (size_t)m0 * kTf, M * kTf, nchunks, cpw, ctx->fattn_part);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(fattn_merge_kernel, dim3(kGf, kDf / kFmDims, mm), dim3(kFaBlock), 0, s,
                           (const float*)ctx->fattn_part, nrec, running_max + (size_t)m0 * kGf,
                           running_sum + (size_t)m0 * kGf, out + (size_t)m0 * kQf);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_full_attention_page(const uint16_t* q, const uint16_t* k_page, const uint16_t* v_page,
                                      const float* mask, float* running_max, float* running_sum, uint16_t* out,
                                      int M, bool first, hipStream_t s, DevCtx* ctx) {
    for (int m0 = 0; m0 < M; m0 += kMaxDecodeM) {
        const int mm = M - m0 < kMaxDecodeM ? M - m0 : kMaxDecodeM;
        hipLaunchKernelGGL(fattn_partial_kernel, dim3(kFaChunks, kFaDimBlocks, mm), dim3(kFaBlock), 0, s,
                           q + (size_t)m0 * kQf, k_page, v_page, mask + (size_t)m0 * kTf, 0, kFaChunks, 1,
                           ctx->fattn_part);
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
