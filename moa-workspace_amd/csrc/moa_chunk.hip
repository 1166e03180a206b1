// moa_chunk.hip -- the MFMA path for calls of more than 16 token rows (prefill chunks).
//
// A chunk of M <= kMaxChunkM rows turns each projection into a dense contraction
// Y[M, N] = X[M, K] . W[N, K]^T, computed on the matrix cores: v_mfma_f32_32x32x16_bf16 with the
// bf16 activations as A and the FP8 weights widened to bf16 (exact: every E4M3 value is a bf16
// value) as B, f32 accumulation. The operators' row-wise steps run as small kernels around it:
//   QKV: RMSNorm rows -> one GEMM over [Wq; Wk; Wv] (bf16(acc * s)) -> per-head RMSNorm + RoPE +
//        q_out / ring-cache stores
//   O:   GEMM (split-K, f32 partials) -> d = bf16(sum * s) -> post-RMSNorm + residual
//   FFN: RMSNorm rows -> up and gate GEMMs in one kernel with the GeGLU epilogue -> down GEMM
//        (split-K) -> post-RMSNorm + residual + layer scalar
// Rounding points are those of the oracle (FO/scripts/generate_references.py:265-274, 337-414;
// FO/scripts/reference/gemma4.py:83-89, 189-197); only the f32 accumulation order differs.
#include <hip/hip_runtime.h>

#include "moa_device.h"
#include "moa_internal.h"

namespace moa {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kCkBlock = 256;        // four waves, 2 (rows) x 2 (columns)
constexpr int kCkBM = 64;            // rows per workgroup
constexpr int kCkBN = 128;           // columns per workgroup (64 per wave: two 32-column MFMA blocks)
constexpr int kCkBK = 64;            // k per pipeline step
constexpr int kCkXStride = kCkBK + 8;  // LDS row stride (elements): padding spreads the rows over banks

// 8 E4M3 codes (two dwords, lower index in the low byte) widened to 8 bf16.
__device__ __forceinline__ bf16x8 fp8x8_to_bf16(uint32_t lo, uint32_t hi) {
    const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
    const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
    const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
    const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
    return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4& v) { return __builtin_bit_cast(bf16x8, v); }

template <ScaleKind SK>
__device__ __forceinline__ float chunk_scale(const void* p, int i) {
    if constexpr (SK == ScaleKind::F32) return static_cast<const float*>(p)[i];
    else return bf2f(static_cast<const uint16_t*>(p)[i]);
}

enum class Epi { Bf16Scaled, F32Partial, GeGLU };

// The contraction of one chunk. Columns [nseg[i], nseg[i+1]) use weight matrix w[i] (rows
// n - nseg[i]) and scales s[i]; a workgroup's 128 columns never straddle two matrices.
struct GemmArgs {
    const uint16_t* x;  // bf16 [M][ldx]
    int ldx;
    int M, N, K;        // K: full reduction length; each of gridDim.z splits takes K / gridDim.z
    const uint8_t* w[3];
    const void* s[3];
    int nseg[4];
    int nsegs;
    const uint8_t* w2;  // GeGLU: the gate matrix (w[0] is up)
    const void* s2;
    uint16_t* y;        // Bf16Scaled, GeGLU: bf16 [M][ldy]
    int ldy;
    float* yf;          // F32Partial: [gridDim.z][M][N]
};

// Workgroup (bx, by, bz): rows 64 by .. +64, columns 128 bx .. +128, k split bz. Wave w covers
// rows 32 (w >> 1) .. +32 and columns 64 (w & 1) .. +64 (two 32 x 32 MFMA blocks). Per 64-k step
// the workgroup stages the X tile in LDS (double-buffered); each wave loads its own weight rows
// (16 bytes per lane per 32 k). Within a 32-k block the k order fed to the two MFMAs is
// permuted identically for A and B (lane half h takes k 16h .. 16h+7 in the first MFMA and
// 16h+8 .. 16h+15 in the second), so one 16-byte weight load feeds both.
template <Epi E, ScaleKind SK>
__global__ __launch_bounds__(kCkBlock) void chunk_gemm_kernel(GemmArgs g) {
    __shared__ __attribute__((aligned(16))) uint16_t xs[2][kCkBM * kCkXStride];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int hf = lane >> 5, l32 = lane & 31;
    const int mb0 = blockIdx.y * kCkBM;
    const int n_wave = blockIdx.x * kCkBN + wn * 64;
    const int kz = g.K / gridDim.z, kbeg = blockIdx.z * kz, nsteps = kz / kCkBK;

    int seg = 0;
    while (seg + 1 < g.nsegs && blockIdx.x * kCkBN >= g.nseg[seg + 1]) ++seg;
    const uint8_t* W = g.w[seg];
    const uint8_t* wr[2];
    const uint8_t* wr2[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        const size_t row = (size_t)(n_wave - g.nseg[seg] + nb * 32 + l32);
        wr[nb] = W + row * g.K + 16 * hf + kbeg;
        wr2[nb] = E == Epi::GeGLU ? g.w2 + row * g.K + 16 * hf + kbeg : nullptr;
    }
    // X staging: 64 rows x 64 k = 512 chunks of 8; thread t moves chunks t and t + 256
    const uint16_t* xr[2];
    bool xok[2];
    int xoff[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = t + 256 * i, row = c >> 3, kc = (c & 7) * 8;
        xok[i] = mb0 + row < g.M;
        xr[i] = g.x + (size_t)min(mb0 + row, g.M - 1) * g.ldx + kbeg + kc;
        xoff[i] = row * kCkXStride + kc;
    }

    f32x16 acc[2], acc2[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[nb][r] = acc2[nb][r] = 0.0f;

    uint4 wq[2][2], wq2[2][2];  // [n block][32-k block]
    auto load_w = [&](int step, uint4 (&dst)[2][2], uint4 (&dst2)[2][2]) {
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                dst[nb][kb] = ld_stream(wr[nb] + step * kCkBK + kb * 32);
                if constexpr (E == Epi::GeGLU) dst2[nb][kb] = ld_stream(wr2[nb] + step * kCkBK + kb * 32);
            }
    };
    uint4 xq[2];
    auto load_x = [&](int step) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint4 v = ld16(xr[i] + step * kCkBK);
            xq[i] = xok[i] ? v : make_uint4(0, 0, 0, 0);
        }
    };
    auto store_x = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 2; ++i) *reinterpret_cast<uint4*>(&xs[buf][xoff[i]]) = xq[i];
    };

    load_x(0);
    load_w(0, wq, wq2);
    store_x(0);
    __syncthreads();
    for (int s = 0; s < nsteps; ++s) {
        const int cur = s & 1;
        uint4 wn[2][2], wn2[2][2];
        if (s + 1 < nsteps) {
            load_x(s + 1);
            load_w(s + 1, wn, wn2);
        }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const uint16_t* ap = &xs[cur][(wm * 32 + l32) * kCkXStride + kb * 32 + 16 * hf];
            const bf16x8 a0 = as_bf16x8(*reinterpret_cast<const uint4*>(ap));
            const bf16x8 a1 = as_bf16x8(*reinterpret_cast<const uint4*>(ap + 8));
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                const uint4 q = wq[nb][kb];
                acc[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, fp8x8_to_bf16(q.x, q.y), acc[nb], 0, 0, 0);
                acc[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, fp8x8_to_bf16(q.z, q.w), acc[nb], 0, 0, 0);
                if constexpr (E == Epi::GeGLU) {
                    const uint4 q2 = wq2[nb][kb];
                    acc2[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, fp8x8_to_bf16(q2.x, q2.y), acc2[nb], 0, 0, 0);
                    acc2[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, fp8x8_to_bf16(q2.z, q2.w), acc2[nb], 0, 0, 0);
                }
            }
        }
        if (s + 1 < nsteps) {
            store_x(cur ^ 1);
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    wq[nb][kb] = wn[nb][kb];
                    if constexpr (E == Epi::GeGLU) wq2[nb][kb] = wn2[nb][kb];
                }
        }
        __syncthreads();
    }

    // Accumulator element r of lane l: row 8 (r / 4) + 4 (l / 32) + r % 4 of the wave's 32-row
    // block, column l % 32 of the 32-column block.
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        const int n = n_wave + nb * 32 + l32;
        float sc = 1.0f, sc2 = 1.0f;
        if constexpr (E != Epi::F32Partial) sc = chunk_scale<SK>(g.s[seg], n - g.nseg[seg]);
        if constexpr (E == Epi::GeGLU) sc2 = chunk_scale<SK>(g.s2, n);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = mb0 + wm * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
            if (m >= g.M) continue;
            if constexpr (E == Epi::Bf16Scaled) {
                g.y[(size_t)m * g.ldy + n] = (uint16_t)f2bf(acc[nb][r] * sc);  // generate_references.py:265-274
            } else if constexpr (E == Epi::F32Partial) {
                g.yf[((size_t)blockIdx.z * g.M + m) * g.N + n] = acc[nb][r];
            } else {
                const float up = rbf(acc[nb][r] * sc), gate = rbf(acc2[nb][r] * sc2);
                g.y[(size_t)m * g.ldy + n] = (uint16_t)f2bf(rbf(gelu_tanh(gate)) * up);  // gemma4.py:197
            }
        }
    }
}

// Block sum over the four waves, in wave order.
__device__ __forceinline__ float ck_block_sum(float v, float* red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return ((red[0] + red[1]) + red[2]) + red[3];
}

// out[m] = bf16(x[m] * rsqrt(mean(x[m]^2) + eps) * w) (gemma4.py:83-89). One workgroup per row;
// thread t < 240 owns elements 16t .. 16t+15.
__global__ __launch_bounds__(kCkBlock) void chunk_rmsnorm_rows_kernel(const uint16_t* __restrict__ x,
                                                                      const uint16_t* __restrict__ w,
                                                                      uint16_t* __restrict__ out) {
    __shared__ float red[4];
    const int t = threadIdx.x, m = blockIdx.x;
    const bool act = t < kH / 16;
    const int c = min(t, kH / 16 - 1);
    const uint16_t* xr = x + (size_t)m * kH + c * 16;
    float xv[16], wv[16];
    bf16x8_to_f32(ld16(xr), xv);
    bf16x8_to_f32(ld16(xr + 8), xv + 8);
    bf16x8_to_f32(ld16(w + c * 16), wv);
    bf16x8_to_f32(ld16(w + c * 16 + 8), wv + 8);
    float ss = 0.0f;
    if (act) {
#pragma unroll
        for (int i = 0; i < 16; ++i) ss = fmaf(xv[i], xv[i], ss);
    }
    const float inv = rms_inverse(ck_block_sum(ss, red), kH);
    if (!act) return;
    uint32_t h[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
        h[i] = f2bf((xv[2 * i] * inv) * wv[2 * i]) | (f2bf((xv[2 * i + 1] * inv) * wv[2 * i + 1]) << 16);
    uint16_t* o = out + (size_t)m * kH + c * 16;
    *reinterpret_cast<uint4*>(o) = make_uint4(h[0], h[1], h[2], h[3]);
    *reinterpret_cast<uint4*>(o + 8) = make_uint4(h[4], h[5], h[6], h[7]);
}

// Per (head, row): RMSNorm over the head's 256 raw values (q, k weighted; v plain), RoPE on q
// and k, and the q_out / ring-cache stores (sliding/rmsnorm.rs:22-153, rope.rs:9-211,
// ops.rs:72-75). Thread t owns head element t; RoPE partners (t, t ^ 128) meet in LDS. A bad
// offset writes nothing; workgroup (0, 0) reports it.
__global__ __launch_bounds__(kCkBlock) void chunk_qkv_heads_kernel(QkvParams p, int m0, const uint16_t* __restrict__ raw,
                                                                   uint32_t* err) {
    __shared__ float red[4];
    __shared__ float xch[kDs];
    const int head = blockIdx.x, m = blockIdx.y, t = threadIdx.x;
    const int32_t rope_off = *p.rope_off, kv_off = *p.kv_off;
    const int mm = m0 + m;
    const bool rope_ok = rope_off >= 0 && (rope_off % (kDs * 2)) == 0 && rope_off / (kDs * 2) + mm < kE;
    const bool kv_ok = kv_off >= 0 && (kv_off % (kNs * kDs * 2)) == 0 && kv_off / (kNs * kDs * 2) < kTs;
    if (!rope_ok || !kv_ok) {
        if (head == 0 && m == 0 && t == 0) atomicOr(err, (rope_ok ? 0u : kErrRopeOffset) | (kv_ok ? 0u : kErrKvOffset));
        return;
    }
    const int slot = (kv_off / (kNs * kDs * 2) + mm) % kTs;
    const int trow = rope_off / (kDs * 2) + mm;
    const uint16_t* wn = head < 16 ? p.q_rms : (head < 24 ? p.k_rms : nullptr);
    const float wv = wn ? bf2f(wn[t]) : 1.0f;
    const float cv = bf2f(p.cos[(size_t)trow * kDs + t]);
    const float sv = bf2f(p.sin[(size_t)trow * kDs + t]);
    const float v = bf2f(raw[(size_t)m * kQkvRowsTotal + head * kDs + t]);
    const float inv = rms_inverse(ck_block_sum(v * v, red), kDs);
    float n = v * inv;
    if (wn) n = n * wv;
    n = rbf(n);
    if (head >= 24) {
        p.v_cache[(size_t)slot * (kNs * kDs) + (head - 24) * kDs + t] = (uint16_t)f2bf(n);
        return;
    }
    xch[t] = n;
    __syncthreads();
    const float partner = xch[t ^ (kDs / 2)];
    // the table's sin has its low half negated (generate_references.py:200-210): plain half swap
    const float a = rbf(n * cv);
    const float b = rbf(partner * sv);
    uint16_t* dst = head < 16 ? p.q_out + (size_t)mm * kQs + head * kDs
                              : p.k_cache + (size_t)slot * (kNs * kDs) + (head - 16) * kDs;
    dst[t] = (uint16_t)f2bf(a + b);
}

// Per row: d = bf16((sum of the split-K partials) * s[n]), then out = bf16(bf16(r + N(d)) * ls)
// with N the post-RMSNorm (identity when w_post is null) and ls skipped when null
// (shared/rmsnorm.rs:204-296, residual.rs:189-241; generate_references.py:411-413).
template <ScaleKind SK>
__global__ __launch_bounds__(kCkBlock) void chunk_post_rows_kernel(const float* __restrict__ part, int splits, int M,
                                                                   const void* scale, const uint16_t* __restrict__ w_post,
                                                                   uint16_t* __restrict__ res, const uint16_t* __restrict__ ls) {
    __shared__ float red[4];
    const int t = threadIdx.x, m = blockIdx.x;
    constexpr int NC = kH / 8;  // 480 chunks of 8; thread t owns t and t + 256
    float d[2][8];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = min(t + 256 * i, NC - 1);
        const bool act = t + 256 * i < NC;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int n = c * 8 + e;
            float a = 0.0f;
            for (int z = 0; z < splits; ++z) a += part[((size_t)z * M + m) * kH + n];
            d[i][e] = rbf(a * chunk_scale<SK>(scale, n));
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
        bf16x8_to_f32(ld16(rr), rv);
        if (w_post) bf16x8_to_f32(ld16(w_post + c * 8), wv);
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
        *reinterpret_cast<uint4*>(rr) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    }
}

template <typename K, typename... A>
hipError_t ck_launch(K kernel, dim3 grid, hipStream_t s, A... args) {
    hipLaunchKernelGGL(kernel, grid, dim3(kCkBlock), 0, s, args...);
    return hipGetLastError();
}

template <Epi E>
hipError_t gemm(const GemmArgs& g, int splits, ScaleKind sk, hipStream_t s) {
    const dim3 grid(g.N / kCkBN, (g.M + kCkBM - 1) / kCkBM, splits);
    return sk == ScaleKind::F32 ? ck_launch(chunk_gemm_kernel<E, ScaleKind::F32>, grid, s, g)
                                : ck_launch(chunk_gemm_kernel<E, ScaleKind::BF16>, grid, s, g);
}

}  // namespace

hipError_t launch_qkv_chunk(const QkvParams& p, int m0, int M, hipStream_t s, DevCtx* ctx) {
    hipError_t e = ck_launch(chunk_rmsnorm_rows_kernel, dim3(M), s, p.x + (size_t)m0 * kH, p.in_rms, ctx->hbuf);
    if (e != hipSuccess) return e;
    GemmArgs g{};
    g.x = ctx->hbuf; g.ldx = kH; g.M = M; g.N = kQkvRowsTotal; g.K = kH;
    g.w[0] = p.qw; g.w[1] = p.kw; g.w[2] = p.vw;
    g.s[0] = p.qs; g.s[1] = p.ks; g.s[2] = p.vs;
    g.nseg[0] = 0; g.nseg[1] = kQs; g.nseg[2] = kQs + kPs; g.nseg[3] = kQkvRowsTotal; g.nsegs = 3;
    g.y = ctx->raw_qkv; g.ldy = kQkvRowsTotal;
    e = gemm<Epi::Bf16Scaled>(g, 1, p.scale_kind, s);
    if (e != hipSuccess) return e;
    return ck_launch(chunk_qkv_heads_kernel, dim3(32, M), s, p, m0, (const uint16_t*)ctx->raw_qkv, ctx->err);
}

hipError_t launch_o_chunk(const OParams& p, int m0, int M, hipStream_t s, DevCtx* ctx) {
    GemmArgs g{};
    g.x = p.x + (size_t)m0 * kQs; g.ldx = kQs; g.M = M; g.N = kH; g.K = kQs;
    g.w[0] = p.ow; g.s[0] = p.os; g.nseg[0] = 0; g.nseg[1] = kH; g.nsegs = 1;
    g.yf = ctx->fbuf;
    hipError_t e = gemm<Epi::F32Partial>(g, kChunkSplitK, p.scale_kind, s);
    if (e != hipSuccess) return e;
    uint16_t* res = p.residual + (size_t)m0 * kH;
    return p.scale_kind == ScaleKind::F32
        ? ck_launch(chunk_post_rows_kernel<ScaleKind::F32>, dim3(M), s, (const float*)ctx->fbuf, kChunkSplitK, M, p.os,
                    p.post_rms, res, (const uint16_t*)nullptr)
        : ck_launch(chunk_post_rows_kernel<ScaleKind::BF16>, dim3(M), s, (const float*)ctx->fbuf, kChunkSplitK, M, p.os,
                    p.post_rms, res, (const uint16_t*)nullptr);
}

hipError_t launch_ffn_chunk(const FfnParams& p, int m0, int M, hipStream_t s, DevCtx* ctx) {
    if (p.fmt != FfnFormat::FP8) return hipErrorInvalidValue;
    uint16_t* res = p.residual + (size_t)m0 * kH;
    hipError_t e = ck_launch(chunk_rmsnorm_rows_kernel, dim3(M), s, (const uint16_t*)res, p.pre_rms, ctx->hbuf);
    if (e != hipSuccess) return e;
    GemmArgs g{};
    g.x = ctx->hbuf; g.ldx = kH; g.M = M; g.N = kL; g.K = kH;
    g.w[0] = p.up; g.s[0] = p.up_s; g.nseg[0] = 0; g.nseg[1] = kL; g.nsegs = 1;
    g.w2 = p.gate; g.s2 = p.gate_s;
    g.y = ctx->pbuf; g.ldy = kL;
    e = gemm<Epi::GeGLU>(g, 1, p.scale_kind, s);
    if (e != hipSuccess) return e;
    GemmArgs d{};
    d.x = ctx->pbuf; d.ldx = kL; d.M = M; d.N = kH; d.K = kL;
    d.w[0] = p.down; d.s[0] = p.down_s; d.nseg[0] = 0; d.nseg[1] = kH; d.nsegs = 1;
    d.yf = ctx->fbuf;
    e = gemm<Epi::F32Partial>(d, kChunkSplitK, p.scale_kind, s);
    if (e != hipSuccess) return e;
    return p.scale_kind == ScaleKind::F32
        ? ck_launch(chunk_post_rows_kernel<ScaleKind::F32>, dim3(M), s, (const float*)ctx->fbuf, kChunkSplitK, M, p.down_s,
                    p.post_rms, res, p.layer_scalar)
        : ck_launch(chunk_post_rows_kernel<ScaleKind::BF16>, dim3(M), s, (const float*)ctx->fbuf, kChunkSplitK, M, p.down_s,
                    p.post_rms, res, p.layer_scalar);
}

}  // namespace moa
