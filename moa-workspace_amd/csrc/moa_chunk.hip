// moa_chunk.hip -- the MFMA path for calls of more than 16 token rows (prefill chunks).
//
// A chunk of M <= kMaxChunkM rows turns each projection into a dense contraction
// Y[M, N] = X[M, K] . W[N, K]^T, computed on the matrix cores: v_mfma_f32_32x32x16_bf16 with the
// bf16 activations as A and the weights widened to bf16 as B, f32 accumulation. The widening is
// exact in every format: E4M3 values are bf16 values; an MXFP4 weight is an E2M1 value times a
// power of two (its E8M0 block scale); an NVFP4 weight, E2M1 times its E4M3 block scale, has at
// most six significant bits (generate_references.py:383-414 folds the same product into bf16). The operators' row-wise steps run as small kernels around it:
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
#include "moa_post_row.h"

namespace moa {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kCkBlock = 256;          // four waves
constexpr int kCkBM = 256;             // rows per workgroup: wave w takes rows 64 w .. 64 w + 63
constexpr int kCkBN = 128;             // weight rows per workgroup (GeGLU: 64 up + the same 64 gate)
constexpr int kCkBK = 64;              // k per pipeline step
constexpr int kCkWStride = 2 * kCkBK + 16;  // LDS bytes per staged (bf16) weight row: 144 puts 16 rows on distinct banks
constexpr int kCkTilesTarget = 264;    // split-K aims at about one workgroup per CU
constexpr int kCkSplitMax = 8;

// 8 E4M3 codes (two dwords, lower index in the low byte) widened to 8 bf16.
__device__ __forceinline__ bf16x8 fp8x8_to_bf16(uint32_t lo, uint32_t hi) {
    const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
    const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
    const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
    const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
    return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// 8 E2M1 codes (one dword, lower index in the low nibble) widened to 8 bf16 with their block
// scale: MXFP4 -- the conversion applies the exponent field of its f32 scale, so the E8M0 code goes
// into bits 23-30; NVFP4 -- each value times the E4M3 scale in f32 (exact: at most six significant
// bits), whose high half is then the bf16.
template <FfnFormat F>
__device__ __forceinline__ bf16x8 fp4x8_to_bf16(uint32_t q, uint32_t sc) {
    if constexpr (F == FfnFormat::MXFP4) {
        const float s = __uint_as_float((sc & 0xffu) << 23);
        const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, s, 0);
        const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, s, 1);
        const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, s, 2);
        const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, s, 3);
        return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
    } else {
        const float s = e4m3_to_f32(sc);
        float v[8];
        fp4x8_to_f32(q, 1.0f, v);
        uint32_t u[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            u[i] = __builtin_amdgcn_perm(__float_as_uint(v[2 * i + 1] * s), __float_as_uint(v[2 * i] * s), 0x07060302u);
        return __builtin_bit_cast(bf16x8, make_uint4(u[0], u[1], u[2], u[3]));
    }
}

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4& v) { return __builtin_bit_cast(bf16x8, v); }

// Activation layout of the MFMA path ("A tiles"): a row-major [M][K] bf16 matrix is stored as
// 4 KB tiles of 32 rows x 64 k, ordered [row block][k step]. Inside a tile the 16-byte unit
// (i, lane), at element 512 i + 8 lane, holds row lane % 32, k 32 (lane / 32) + 8 i .. + 7: what
// lane `lane` feeds to the step's MFMA i. One 16-byte load per lane then reads 1 KB contiguous
// (eight cache lines) instead of touching 32 rows. Rows are padded to a multiple of 32.
__host__ __device__ __forceinline__ size_t atile_off(int m, int k, int K) {
    const int kk = k & 63;
    return ((size_t)(m >> 5) * (K >> 6) + (k >> 6)) * 2048 + ((kk >> 3) & 3) * 512 + ((m & 31) + 32 * (kk >> 5)) * 8 +
           (k & 7);
}


enum class Epi { F32Partial, GeGLU };

// The contraction of one chunk. Columns [nseg[i], nseg[i+1]) use weight matrix w[i] (rows
// n - nseg[i]); a workgroup's 128 columns never straddle two matrices.
struct GemmArgs {
    const uint16_t* x;  // bf16 A tiles of [M][K]
    int M, N, K;        // K: full reduction length; each of gridDim.z splits takes K / gridDim.z
    const uint8_t* w[3];
    int nseg[4];
    int nsegs;
    const uint8_t* w2;  // GeGLU: the gate matrix (w[0] is up); s[0], s2 their scales
    const void* s0;
    const void* s2;
    const uint8_t* wsc[3];  // FP4 weights: block-scale codes of w[i] ([rows][K/16] NVFP4, [rows][K/32] MXFP4)
    const uint8_t* wsc2;    // ... and of w2
    const float* g0;        // NVFP4 GeGLU: reciprocal global scales of up (w[0]) and gate (w2), device
    const float* g2;
    uint16_t* y;        // GeGLU: bf16 A tiles of [M][N] (the down projection's input)
    float* yf;          // F32Partial: [gridDim.z][M][N]
};

template <int V>
struct Par {
    static constexpr int value = V;
};

// Buffer resource over [base, base + bytes): loads past the end return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t ck_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// Cache policy of the weight loads: the default. Non-temporal loads (policy 2) measured 6 us slower
// per M = 256 layer (177.9 -> 171.9 us), as they were in the rows path.
constexpr int kCkNt = 0;

// Workgroup (bx, by, bz): rows 256 by .. +256, a 128-row weight tile (columns 128 bx .. +128,
// or for GeGLU up and gate rows 64 bx .. +64), k split bz. Wave w computes rows 64 w .. +64 of
// the tile against all 128 weight rows: 2 x 4 blocks of v_mfma_f32_32x32x16_bf16, 128 f32
// accumulators per lane.
//   Activations (A tiles) go from memory straight into the registers of the lanes that feed them
//   to the MFMA (no other wave needs them): per 64-k step lane (l32, h) holds 32 bf16 of row l32
//   of each 32-row block, k 32 h .. 32 h + 31, in four 1 KB-contiguous loads. MFMA j (j = 0..3)
//   of the step takes k 32 h + 8 j .. + 7 from lane half h, for A and B alike, which is a fixed
//   permutation of the step's 64 k. Row blocks past M read zeros (the buffer ends there); rows
//   past M are not stored.
//   Weights (FP8) are staged once per workgroup through LDS, widened to bf16 on the way (exact for
//   E4M3; once per workgroup instead of once per wave): each thread moves two 16-byte chunks per
//   step, loaded eight steps ahead (HBM latency at the rate the whole chip streams weights) and
//   written two steps ahead; a wave reads 64 bytes (bf16) per lane per 32-column block.
//   All loads are buffer loads whose per-lane offsets are fixed: the step moves the scalar
//   offset only. Prefetches past the last step repeat the last step (harmless), so the loop body
//   has no branches.
template <Epi E, ScaleKind SK, FfnFormat F = FfnFormat::FP8, int BN = kCkBN>
__global__ __launch_bounds__(kCkBlock) __attribute__((amdgpu_waves_per_eu(1, 1))) void chunk_gemm_kernel(GemmArgs g) {
    static_assert(BN == 128 || (BN == 64 && E == Epi::F32Partial), "128 weight rows, or 64 for split-K partials");
    constexpr int NB = BN / 32;   // 32-column blocks per wave
    constexpr int RPT = BN / 64;  // staged weight rows per thread
    constexpr bool FP4 = F != FfnFormat::FP8;
    // bytes per weight row and per 64-k step; FP4 block-scale bytes per row and per step
    const int rb = FP4 ? g.K / 2 : g.K;
    constexpr int kStepB = FP4 ? kCkBK / 2 : kCkBK;
    const int sb = F == FfnFormat::NVFP4 ? g.K / 16 : (F == FfnFormat::MXFP4 ? g.K / 32 : 0);
    constexpr int kStepS = F == FfnFormat::NVFP4 ? 4 : 2;
    // three weight buffers during the loop; the GeGLU epilogue reuses the space for its transpose
    constexpr int kWsBytes = BN * kCkWStride, kTpStride = 72;
    constexpr int kLds = 3 * kWsBytes > 4 * 64 * kTpStride * 2 ? 3 * kWsBytes : 4 * 64 * kTpStride * 2;
    __shared__ __attribute__((aligned(16))) uint8_t smem[kLds];
    uint8_t(*ws)[kWsBytes] = reinterpret_cast<uint8_t(*)[kWsBytes]>(smem);
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int hf = lane >> 5, l32 = lane & 31;
    const int m_blk = blockIdx.y * kCkBM;
    const int m_wave = m_blk + wave * 64;
    const int kz = g.K / gridDim.z, kbeg = blockIdx.z * kz, nsteps = kz / kCkBK;

    // staged weight rows of this thread: tile row r0 (and r0 + 64 when BN = 128), k 16 q .. 16 q + 15 of each step
    // (FP8: 16 bytes; FP4: 8 bytes of codes and the one block-scale code covering them)
    const int r0 = t >> 2, q = t & 3;
    __amdgpu_buffer_rsrc_t wrs[2], srs[2];
    int wvo[2], svo[2] = {0, 0};
    const int kcol = FP4 ? (kbeg + 16 * q) / 2 : kbeg + 16 * q;
    const int scol = F == FfnFormat::NVFP4 ? kbeg / 16 + q : kbeg / 32 + q / 2;
    int seg = 0;
    if constexpr (E == Epi::GeGLU) {
        const size_t off = (size_t)blockIdx.x * 64 * rb;
        wrs[0] = ck_rsrc(g.w[0] + off, 64u * rb);
        wrs[1] = ck_rsrc(g.w2 + off, 64u * rb);
        wvo[0] = wvo[1] = r0 * rb + kcol;
        if constexpr (FP4) {
            const size_t so = (size_t)blockIdx.x * 64 * sb;
            srs[0] = ck_rsrc(g.wsc[0] + so, 64u * sb);
            srs[1] = ck_rsrc(g.wsc2 + so, 64u * sb);
            svo[0] = svo[1] = r0 * sb + scol;
        }
    } else {
        const int n0 = blockIdx.x * BN;
        while (seg + 1 < g.nsegs && n0 >= g.nseg[seg + 1]) ++seg;
        wrs[0] = wrs[1] = ck_rsrc(g.w[seg] + (size_t)(n0 - g.nseg[seg]) * rb, (uint32_t)BN * rb);
        wvo[0] = r0 * rb + kcol;
        wvo[1] = (r0 + 64) * rb + kcol;
        if constexpr (FP4) {
            srs[0] = srs[1] = ck_rsrc(g.wsc[seg] + (size_t)(n0 - g.nseg[seg]) * sb, (uint32_t)BN * sb);
            svo[0] = r0 * sb + scol;
            svo[1] = (r0 + 64) * sb + scol;
        }
    }
    const int wdst0 = r0 * kCkWStride + 32 * q, wdst1 = (r0 + 64) * kCkWStride + 32 * q;

    const int kst = g.K / kCkBK;  // 64-k steps (A tiles) per row block
    const int rblks = (min(g.M - m_blk, kCkBM) + 31) >> 5;
    const __amdgpu_buffer_rsrc_t ars = ck_rsrc(g.x + (size_t)(m_blk >> 5) * kst * 2048, (uint32_t)rblks * kst * 4096u);
    int avo[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) avo[mb] = ((wave * 2 + mb) * kst * 2048 + lane * 8) * 2 + (kbeg / kCkBK) * 4096;

    f32x16 acc[2][NB];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mb][nb][r] = 0.0f;

    constexpr int WD = 6;  // weight register sets: W(s + 2) is loaded six steps before it is staged
    uint4 wr[WD][2];       // [set][row pair]
    uint4 ar[3][2][4];     // [set][32-row block][16 bytes]: A(s) in set s mod 3, loaded two steps ahead
    bf16x8 bb[2][4];       // B fragments: [set][MFMA j]
    const int last = nsteps - 1;
    // FP4: .x, .y the 16 codes, .z the block-scale code
    auto load_w = [&](uint4 (&dst)[2], int s) {
        const int so = min(s, last) * kStepB;
        if constexpr (FP4) {
#pragma unroll
            for (int i = 0; i < RPT; ++i) {
                const auto v = __builtin_amdgcn_raw_buffer_load_b64(wrs[i], wvo[i], so, kCkNt);
                dst[i].x = v[0];
                dst[i].y = v[1];
                dst[i].z = __builtin_amdgcn_raw_buffer_load_b8(srs[i], svo[i], min(s, last) * kStepS, 0);
            }
        } else {
#pragma unroll
            for (int i = 0; i < RPT; ++i)
                dst[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wrs[i], wvo[i], so, kCkNt));
        }
    };
    auto store_w = [&](const uint4 (&src)[2], int buf) {
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            bf16x8* d = reinterpret_cast<bf16x8*>(&ws[buf][i ? wdst1 : wdst0]);
            if constexpr (FP4) {
                d[0] = fp4x8_to_bf16<F>(src[i].x, src[i].z);
                d[1] = fp4x8_to_bf16<F>(src[i].y, src[i].z);
            } else {
                d[0] = fp8x8_to_bf16(src[i].x, src[i].y);
                d[1] = fp8x8_to_bf16(src[i].z, src[i].w);
            }
        }
    };
    auto load_a = [&](uint4 (&dst)[2][4], int s) {
        const int so = min(s, last) * 4096;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                dst[mb][i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ars, avo[mb] + 1024 * i, so, 0));
    };
    auto read_b = [&](bf16x8 (&dst)[4], int buf, int nb) {
        const bf16x8* bp = reinterpret_cast<const bf16x8*>(&ws[buf][(32 * nb + l32) * kCkWStride + 64 * hf]);
#pragma unroll
        for (int j = 0; j < 4; ++j) dst[j] = bp[j];
    };
    auto mfma8 = [&](const uint4 (&a)[2][4], const bf16x8 (&b)[4], auto NBI) {
        constexpr int nb = decltype(NBI)::value;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
                acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a[mb][j]), b[j], acc[mb][nb], 0, 0, 0);
    };

    // Three LDS buffers: step s reads buffer s mod 3 and stages W(s + 2) into buffer (s + 2) mod 3
    // (last read in step s - 1, before the barrier that opens step s), so the first fragment of
    // step s + 1 (buffer (s + 1) mod 3, staged in step s - 1) is read before step s ends. Within a
    // step, fragment nb + 1 is read while fragment nb's eight MFMAs run.
#pragma unroll
    for (int i = 0; i < WD; ++i) load_w(wr[i], i);
    load_a(ar[0], 0);
    load_a(ar[1], 1);
    store_w(wr[0], 0);
    store_w(wr[1], 1);
    load_w(wr[0], WD);
    load_w(wr[1], WD + 1);
    __syncthreads();
    read_b(bb[0], 0, 0);
    auto body4 = [&](auto P, int s) {
        constexpr int c = decltype(P)::value;  // s mod 6
        constexpr int cb = c % 3, nbuf = (c + 1) % 3;
        const uint4(&a)[2][4] = ar[c % 3];
        // Fences fix the issue order: each fragment's LDS reads go out during the previous
        // fragment's eight MFMAs, one or two other instructions after each MFMA (a single wave
        // per SIMD issues them while the MFMA runs); the A prefetch rides with fragment 0, the
        // weight staging (16 widenings, 4 LDS writes, 2 loads) with fragment 1.
        constexpr int kDsR = 0x100, kDsW = 0x200, kVmR = 0x020, kValu = 0x002, kMfma = 0x008;
        constexpr int kWLoads = FP4 ? 4 : 2;                    // weight (and scale) loads per step
        constexpr int kWValu = F == FfnFormat::NVFP4 ? 8 : 2;   // widening instructions per MFMA slot
        read_b(bb[1], cb, 1);
        load_a(ar[(c + 2) % 3], s + 2);
        mfma8(a, bb[0], Par<0>{});
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
            __builtin_amdgcn_sched_group_barrier(kDsR, 1, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
            __builtin_amdgcn_sched_group_barrier(kVmR, 2, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        read_b(bb[0], cb, 2);
        store_w(wr[(c + 2) % WD], (c + 2) % 3);
        load_w(wr[(c + 2) % WD], s + 2 + WD);
        mfma8(a, bb[1], Par<1>{});
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_sched_group_barrier(kMfma, 1, 1);
            __builtin_amdgcn_sched_group_barrier(kDsR, 1, 1);
            __builtin_amdgcn_sched_group_barrier(kValu, kWValu, 1);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_sched_group_barrier(kMfma, 1, 1);
            __builtin_amdgcn_sched_group_barrier(kValu, kWValu, 1);
            __builtin_amdgcn_sched_group_barrier(kDsW, 1, 1);
        }
        __builtin_amdgcn_sched_group_barrier(kVmR, kWLoads, 1);
        __builtin_amdgcn_sched_barrier(0);
        read_b(bb[1], cb, 3);
        mfma8(a, bb[0], Par<2>{});
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_sched_group_barrier(kMfma, 1, 2);
            __builtin_amdgcn_sched_group_barrier(kDsR, 1, 2);
        }
        __builtin_amdgcn_sched_group_barrier(kMfma, 4, 2);
        __builtin_amdgcn_sched_barrier(0);
        read_b(bb[0], nbuf, 0);
        mfma8(a, bb[1], Par<3>{});
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_sched_group_barrier(kMfma, 1, 3);
            __builtin_amdgcn_sched_group_barrier(kDsR, 1, 3);
        }
        __builtin_amdgcn_sched_group_barrier(kMfma, 4, 3);
        // Step barrier. Every read of the buffer the next step overwrites fed an MFMA of this step
        // (so it is complete); the next step's buffer needs this wave's LDS writes complete, and
        // only the four reads just issued may still be in flight: lgkmcnt(4), not 0.
        __builtin_amdgcn_sched_barrier(0);
        __asm__ volatile("s_waitcnt lgkmcnt(4)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    };
    // BN = 64: two fragments per step. Fragment 0 carries the staging (widenings and LDS writes of
    // W(s + 2)) beside fragment 1's LDS reads; fragment 1 the A and weight prefetches and, last of
    // the step's LDS operations, the next step's first fragment -- so lgkmcnt(4) at the barrier
    // still leaves every LDS write of this wave complete.
    auto body2 = [&](auto P, int s) {
        constexpr int c = decltype(P)::value;  // s mod 6
        constexpr int cb = c % 3, nbuf = (c + 1) % 3;
        const uint4(&a)[2][4] = ar[c % 3];
        constexpr int kDsR = 0x100, kDsW = 0x200, kVmR = 0x020, kValu = 0x002, kMfma = 0x008;
        constexpr int kWLoads = FP4 ? 2 : 1;
        constexpr int kWValu = F == FfnFormat::NVFP4 ? 4 : 1;
        read_b(bb[1], cb, 1);
        store_w(wr[(c + 2) % WD], (c + 2) % 3);
        mfma8(a, bb[0], Par<0>{});
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
            __builtin_amdgcn_sched_group_barrier(kDsR, 1, 0);
            __builtin_amdgcn_sched_group_barrier(kValu, kWValu, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
            __builtin_amdgcn_sched_group_barrier(kValu, kWValu, 0);
            __builtin_amdgcn_sched_group_barrier(kDsW, 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        load_a(ar[(c + 2) % 3], s + 2);
        load_w(wr[(c + 2) % WD], s + 2 + WD);
        read_b(bb[0], nbuf, 0);
        mfma8(a, bb[1], Par<1>{});
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_sched_group_barrier(kMfma, 1, 1);
            __builtin_amdgcn_sched_group_barrier(kVmR, 2, 1);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_sched_group_barrier(kMfma, 1, 1);
            __builtin_amdgcn_sched_group_barrier(kDsR, 1, 1);
        }
        __builtin_amdgcn_sched_group_barrier(kVmR, kWLoads, 1);
        __builtin_amdgcn_sched_barrier(0);
        __asm__ volatile("s_waitcnt lgkmcnt(4)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    };
    auto body = [&](auto P, int s) {
        if constexpr (NB == 4) body4(P, s);
        else body2(P, s);
    };
    int s = 0;
    for (; s + 5 < nsteps; s += 6) {
        body(Par<0>{}, s);
        body(Par<1>{}, s + 1);
        body(Par<2>{}, s + 2);
        body(Par<3>{}, s + 3);
        body(Par<4>{}, s + 4);
        body(Par<5>{}, s + 5);
    }
    if (s < nsteps) body(Par<0>{}, s++);
    if (s < nsteps) body(Par<1>{}, s++);
    if (s < nsteps) body(Par<2>{}, s++);
    if (s < nsteps) body(Par<3>{}, s++);
    if (s < nsteps) body(Par<4>{}, s++);

    if constexpr (E == Epi::GeGLU) __syncthreads();  // the loop's LDS reads are done: the transpose may reuse it
    if (m_wave >= g.M) return;
    // Accumulator element r of lane l: row 8 (r / 4) + 4 (l / 32) + r % 4 of the 32-row block,
    // column l % 32 of the 32-column block. A wave whose 64 rows all lie below M stores without
    // per-element tests (a test per element would serialise the 64-128 element computations).
    const bool full = m_wave + 64 <= g.M;
    if constexpr (E == Epi::F32Partial) {
        float* yz = g.yf + (size_t)blockIdx.z * g.M * g.N + blockIdx.x * BN + l32;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m_wave + 32 * mb + 8 * (r >> 2) + 4 * hf + (r & 3);
                    if (full || m < g.M) yz[(size_t)m * g.N + nb * 32] = acc[mb][nb][r];
                }
    } else {
        // p = bf16(gelu(gate) * up) for the wave's 64 rows x 64 columns, transposed through the
        // wave's own 9 KB of LDS (row stride 72 elements) so that each lane then stores whole
        // 16-byte units of the A tiles (row, 8 consecutive columns).
        uint16_t* tp = reinterpret_cast<uint16_t*>(smem) + wave * (64 * kTpStride);
        // the format's commit of each projection: FP8 bf16(sum * s[n]); NVFP4 bf16(bf16(sum) * 1/g);
        // MXFP4 bf16(sum) (generate_references.py:265-274, 358-372)
        const float gu = F == FfnFormat::NVFP4 ? *g.g0 : 1.0f, gg = F == FfnFormat::NVFP4 ? *g.g2 : 1.0f;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            const int n = blockIdx.x * 64 + nb * 32 + l32;
            const float su = FP4 ? 1.0f : chunk_scale<SK>(g.s0, n), sg = FP4 ? 1.0f : chunk_scale<SK>(g.s2, n);
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int ml = 32 * mb + 8 * (r >> 2) + 4 * hf + (r & 3);
                    float up, gate;
                    if constexpr (F == FfnFormat::FP8) {
                        up = rbf(acc[mb][nb][r] * su);
                        gate = rbf(acc[mb][nb + 2][r] * sg);
                    } else if constexpr (F == FfnFormat::NVFP4) {
                        up = rbf(rbf(acc[mb][nb][r]) * gu);
                        gate = rbf(rbf(acc[mb][nb + 2][r]) * gg);
                    } else {
                        up = rbf(acc[mb][nb][r]);
                        gate = rbf(acc[mb][nb + 2][r]);
                    }
                    tp[ml * kTpStride + nb * 32 + l32] = (uint16_t)f2bf(rbf(gelu_tanh(gate)) * up);  // gemma4.py:197
                }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes are done
        __builtin_amdgcn_wave_barrier();
        // 64 rows x 8 units of 16 bytes = 512 units; lane takes units lane + 64 i
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int u = lane + 64 * i, ml = u >> 3, cu = u & 7;
            const int m = m_wave + ml;
            const uint4 v = *reinterpret_cast<const uint4*>(&tp[ml * kTpStride + cu * 8]);
            if (full || m < g.M) *reinterpret_cast<uint4*>(g.y + atile_off(m, blockIdx.x * 64 + cu * 8, g.N)) = v;
        }
    }
}

// Rows of the A-tile producers. A 128-byte line of a tile holds one 16-byte unit of each of 8
// consecutive rows, so with one workgroup per row each line is written by 8 workgroups; they are
// dealt to the 8 XCDs round-robin (XCD = b % 8), and rows 8g .. 8g + 7 go to workgroups on XCD
// g % 8, where one L2 assembles the whole line. Rows past the last multiple of 64 keep b.
__device__ __forceinline__ int tile_row(int b, int M) {
    if (b >= (M & ~63)) return b;
    const int x = b & 7, j = b >> 3;
    return ((x + 8 * (j >> 3)) << 3) | (j & 7);
}


// out[m] = bf16(x[m] * rsqrt(mean(x[m]^2) + eps) * w) (gemma4.py:83-89), written as A tiles
// (Tiles) or row-major [M][kH]. One workgroup per row (for tiles, row tile_row(b)); thread t < 240
// owns elements 16t .. 16t+15.
// Row m's norm from thread t's 16 elements xv (16t .. 16t+15, t < 240) and weights wv, stored.
template <bool Tiles>
__device__ __forceinline__ void rms_row_store(const float (&xv)[16], const float (&wv)[16], int m, float* red,
                                              uint16_t* __restrict__ out) {
    const int t = threadIdx.x;
    const int c = min(t, kH / 16 - 1);
    uint32_t h[8];
    rms_row_values(xv, wv, red, h);
    if (t >= kH / 16) return;
    const size_t o0 = Tiles ? atile_off(m, c * 16, kH) : (size_t)m * kH + c * 16;
    const size_t o1 = Tiles ? atile_off(m, c * 16 + 8, kH) : (size_t)m * kH + c * 16 + 8;
    *reinterpret_cast<uint4*>(out + o0) = make_uint4(h[0], h[1], h[2], h[3]);
    *reinterpret_cast<uint4*>(out + o1) = make_uint4(h[4], h[5], h[6], h[7]);
}

template <bool Tiles = true>
__global__ __launch_bounds__(kCkBlock) void chunk_rmsnorm_rows_kernel(const uint16_t* __restrict__ x,
                                                                      const uint16_t* __restrict__ w,
                                                                      uint16_t* __restrict__ out) {
    __shared__ float red[4];
    const int t = threadIdx.x, m = Tiles ? tile_row(blockIdx.x, gridDim.x) : blockIdx.x;
    const int c = min(t, kH / 16 - 1);
    const uint16_t* xr = x + (size_t)m * kH + c * 16;
    float xv[16], wv[16];
    bf16x8_to_f32(ld16(xr), xv);
    bf16x8_to_f32(ld16(xr + 8), xv + 8);
    bf16x8_to_f32(ld16(w + c * 16), wv);
    bf16x8_to_f32(ld16(w + c * 16 + 8), wv + 8);
    rms_row_store<Tiles>(xv, wv, m, red, out);
}

// Row-major bf16 [M][K] -> A tiles (the O-projection's input arrives row-major). One workgroup
// per row (tile_row); thread t moves 16-byte units t, t + 256, ...
__global__ __launch_bounds__(kCkBlock) void chunk_tile_rows_kernel(const uint16_t* __restrict__ x, int K,
                                                                   uint16_t* __restrict__ out) {
    const int m = tile_row(blockIdx.x, gridDim.x);
    for (int u = threadIdx.x; u < K / 8; u += kCkBlock)
        *reinterpret_cast<uint4*>(out + atile_off(m, u * 8, K)) = ld16(x + (size_t)m * K + u * 8);
}

// Per (head, row): raw = bf16((sum of the split-K partials) * s), RMSNorm over the head's 256 raw
// values (q, k weighted; v plain), RoPE on q and k, and the q_out / ring-cache stores
// (generate_references.py:265-274; sliding/rmsnorm.rs:22-153, rope.rs:9-211, ops.rs:72-75).
// Thread t owns head element t; RoPE partners (t, t ^ 128) meet in LDS. A row whose offsets are bad
// writes nothing, and its head-0 workgroup reports them.
template <ScaleKind SK, int ZS = kCkSplitMax>
__global__ __launch_bounds__(kCkBlock) void chunk_qkv_heads_kernel(QkvParams p, int m0, int M,
                                                                   const float* __restrict__ part, int splits,
                                                                   uint32_t* err) {
    __shared__ float red[4];
    __shared__ float xch[kDs];
    const int head = blockIdx.x, m = blockIdx.y, t = threadIdx.x;
    const int32_t rope_off = *p.rope_off, kv_off = *p.kv_off;
    const int mm = m0 + m;
    const bool rope_ok = rope_off >= 0 && (rope_off % (kDs * 2)) == 0 && rope_off / (kDs * 2) + mm < kE;
    const bool kv_ok = kv_off >= 0 && (kv_off % (kNs * kDs * 2)) == 0 && kv_off / (kNs * kDs * 2) < kTs;
    if (!rope_ok || !kv_ok) {
        if (head == 0 && t == 0) atomicOr(err, (rope_ok ? 0u : kErrRopeOffset) | (kv_ok ? 0u : kErrKvOffset));
        return;
    }
    const int slot = (kv_off / (kNs * kDs * 2) + mm) % kTs;
    const int trow = rope_off / (kDs * 2) + mm;
    const int col = head * kDs + t;
    float pz[ZS];  // all partial loads in flight at once (index clamped), summed in split order
#pragma unroll
    for (int z = 0; z < ZS; ++z) pz[z] = part[((size_t)min(z, splits - 1) * M + m) * kQkvRowsTotal + col];
    float acc = pz[0];
#pragma unroll
    for (int z = 1; z < ZS; ++z) acc = z < splits ? acc + pz[z] : acc;
    const float sc = head < 16 ? chunk_scale<SK>(p.qs, col)
                               : (head < 24 ? chunk_scale<SK>(p.ks, col - kQs) : chunk_scale<SK>(p.vs, col - kQs - kPs));
    const float v = rbf(acc * sc);
    const uint16_t* wn = head < 16 ? p.q_rms : (head < 24 ? p.k_rms : nullptr);
    const float wv = wn ? bf2f(wn[t]) : 1.0f;
    const float cv = bf2f(p.cos[(size_t)trow * kDs + t]);
    const float sv = bf2f(p.sin[(size_t)trow * kDs + t]);
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

// The same per (head, row) work for the MFMA path, four heads of one row per workgroup: wave w
// takes head 4 x + w of row y (x = blockIdx.x < 8, so the four are all Q, all K or all V), lane l
// its elements l, l + 64, l + 128 and l + 192. Both RoPE pairs (t, t ^ 128) are then within the
// lane, and the head's sum of squares is four wave sums added in the order of ck_block_sum (wave k
// there holds elements 64 k ..), so every output has chunk_qkv_heads_kernel's bits; no LDS and no
// barrier. 8 x M workgroups instead of 32 x M.
template <ScaleKind SK, int ZS>
__global__ __launch_bounds__(kCkBlock) void chunk_qkv_heads4_kernel(QkvParams p, int m0, int M,
                                                                    const float* __restrict__ part, int splits,
                                                                    uint32_t* err) {
    const int lane = threadIdx.x & 63, head = 4 * blockIdx.x + (threadIdx.x >> 6), m = blockIdx.y;
    const int32_t rope_off = *p.rope_off, kv_off = *p.kv_off;
    const int mm = m0 + m;
    const bool rope_ok = rope_off >= 0 && (rope_off % (kDs * 2)) == 0 && rope_off / (kDs * 2) + mm < kE;
    const bool kv_ok = kv_off >= 0 && (kv_off % (kNs * kDs * 2)) == 0 && kv_off / (kNs * kDs * 2) < kTs;
    if (!rope_ok || !kv_ok) {
        if (blockIdx.x == 0 && threadIdx.x == 0) atomicOr(err, (rope_ok ? 0u : kErrRopeOffset) | (kv_ok ? 0u : kErrKvOffset));
        return;
    }
    const int slot = (kv_off / (kNs * kDs * 2) + mm) % kTs;
    const int trow = rope_off / (kDs * 2) + mm;
    const float* prow = part + (size_t)m * kQkvRowsTotal + head * kDs + lane;
    float pz[4][ZS];  // all partial loads in flight at once (split index clamped)
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int z = 0; z < ZS; ++z) pz[k][z] = prow[(size_t)min(z, splits - 1) * M * kQkvRowsTotal + 64 * k];
    const uint16_t* wn = head < 16 ? p.q_rms : (head < 24 ? p.k_rms : nullptr);
    float v[4], ss[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int col = head * kDs + 64 * k + lane;
        float acc = pz[k][0];
#pragma unroll
        for (int z = 1; z < ZS; ++z) acc = z < splits ? acc + pz[k][z] : acc;
        const float sc = head < 16 ? chunk_scale<SK>(p.qs, col)
                                   : (head < 24 ? chunk_scale<SK>(p.ks, col - kQs) : chunk_scale<SK>(p.vs, col - kQs - kPs));
        v[k] = rbf(acc * sc);
        ss[k] = wave_sum(v[k] * v[k]);
    }
    const float inv = rms_inverse(((ss[0] + ss[1]) + ss[2]) + ss[3], kDs);
    float n[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float x = v[k] * inv;
        if (wn) x = x * bf2f(wn[64 * k + lane]);
        n[k] = rbf(x);
    }
    if (head >= 24) {
        uint16_t* vd = p.v_cache + (size_t)slot * (kNs * kDs) + (head - 24) * kDs + lane;
#pragma unroll
        for (int k = 0; k < 4; ++k) vd[64 * k] = (uint16_t)f2bf(n[k]);
        return;
    }
    // the table's sin has its low half negated (generate_references.py:200-210): plain half swap
    uint16_t* dst = (head < 16 ? p.q_out + (size_t)mm * kQs + head * kDs
                               : p.k_cache + (size_t)slot * (kNs * kDs) + (head - 16) * kDs) + lane;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int t = 64 * k + lane;
        const float cv = bf2f(p.cos[(size_t)trow * kDs + t]);
        const float sv = bf2f(p.sin[(size_t)trow * kDs + t]);
        dst[64 * k] = (uint16_t)f2bf(rbf(n[k] * cv) + rbf(n[k ^ 2] * sv));
    }
}

template <ScaleKind SK, FfnFormat F = FfnFormat::FP8, int ZS = kCkSplitMax>
__global__ __launch_bounds__(kCkBlock) void chunk_post_rows_kernel(const float* __restrict__ part, int splits, int M,
                                                                   const void* scale, const float* __restrict__ gscale,
                                                                   const uint16_t* __restrict__ w_post,
                                                                   uint16_t* __restrict__ res, const uint16_t* __restrict__ ls) {
    __shared__ float red[4];
    uint4 out[2];
    post_row<SK, F, ZS>(part, splits, M, scale, gscale, w_post, res, ls, blockIdx.x, red, out);
}

// O's post rows with the FFN's pre-norm behind them (sliding_attention_output then
// decoder_feedforward on one residual, FO/src/host/runtime.rs:440-459 then 543-571): a row gets
// O's post-norm and residual as chunk_post_rows_kernel computes them, then the FFN's pre-norm of
// the new residual, written into hout exactly as chunk_rmsnorm_rows_kernel<Tiles> writes it (the
// row through LDS, so that thread t < 240 sums elements 16t .. 16t+15 in the same order): A tiles
// for the MFMA GEMMs (row tile_row(b)), row-major for the rows path (row b). The FFN then starts
// at its first projection.
template <ScaleKind SK, int ZS, bool Tiles = true>
__global__ __launch_bounds__(kCkBlock) void chunk_post_pre_rows_kernel(const float* __restrict__ part, int splits, int M,
                                                                       const void* scale,
                                                                       const uint16_t* __restrict__ w_post,
                                                                       uint16_t* __restrict__ res,
                                                                       const uint16_t* __restrict__ w_pre,
                                                                       uint16_t* __restrict__ hout) {
    __shared__ float red[4];
    __shared__ __attribute__((aligned(16))) uint16_t row[kH];
    const int t = threadIdx.x, m = Tiles ? tile_row(blockIdx.x, gridDim.x) : blockIdx.x;
    const int c = min(t, kH / 16 - 1);
    float wv[16];
    bf16x8_to_f32(ld16(w_pre + c * 16), wv);
    bf16x8_to_f32(ld16(w_pre + c * 16 + 8), wv + 8);
    uint4 out[2];
    post_row<SK, FfnFormat::FP8, ZS>(part, splits, M, scale, nullptr, w_post, res, nullptr, m, red, out);
#pragma unroll
    for (int i = 0; i < 2; ++i)
        if (t + 256 * i < kH / 8) *reinterpret_cast<uint4*>(row + (t + 256 * i) * 8) = out[i];
    __syncthreads();
    float xv[16];
    bf16x8_to_f32(*reinterpret_cast<const uint4*>(row + c * 16), xv);
    bf16x8_to_f32(*reinterpret_cast<const uint4*>(row + c * 16 + 8), xv + 8);
    rms_row_store<Tiles>(xv, wv, m, red, hout);
}

template <typename K, typename... A>
hipError_t ck_launch(K kernel, dim3 grid, hipStream_t s, A... args) {
    hipLaunchKernelGGL(kernel, grid, dim3(kCkBlock), 0, s, args...);
    return hipGetLastError();
}

// Split-K factor: the largest of 1, 2, 4, 8 that divides the 64-k steps, keeps the grid near one
// workgroup per CU and fits the partial-sum buffer.
int pick_splits(int tiles, int ksteps, size_t rows_x_cols) {
    int sp = 1;
    for (int c = 2; c <= kCkSplitMax; c *= 2)
        if (ksteps % c == 0 && tiles * c <= kCkTilesTarget && (size_t)c * rows_x_cols <= kChunkPartFloats) sp = c;
    return sp;
}

// Weight rows per workgroup of a split-K projection. The O projection (K = 4096) takes 64: twice
// the tiles of 128-row tiles, so half the k splits fill the device and half the f32 partial sums
// are written and read back (measured at M = 256: GEMM 17.3 -> 16.5 us, post rows 9.1 -> 6.9 us).
// QKV takes 64 up to 256 rows (launch_qkv_chunk). Down keeps 128, whose main loop does twice the
// MFMA work per A load and per barrier (with 64, down measured 39.1 -> 44.6 us against 9.5 ->
// 7.1 us saved in its post rows).
constexpr int kCkOBN = 64;

template <FfnFormat F = FfnFormat::FP8, int BN = kCkBN>
hipError_t gemm_partial(const GemmArgs& g, int splits, ScaleKind sk, hipStream_t s) {
    if (g.N % BN || g.K % (kCkBK * splits) || (size_t)splits * g.M * g.N > kChunkPartFloats) return hipErrorInvalidValue;
    const dim3 grid(g.N / BN, (g.M + kCkBM - 1) / kCkBM, splits);
    if constexpr (F != FfnFormat::FP8) return ck_launch(chunk_gemm_kernel<Epi::F32Partial, ScaleKind::F32, F, BN>, grid, s, g);
    return sk == ScaleKind::F32 ? ck_launch(chunk_gemm_kernel<Epi::F32Partial, ScaleKind::F32, F, BN>, grid, s, g)
                                : ck_launch(chunk_gemm_kernel<Epi::F32Partial, ScaleKind::BF16, F, BN>, grid, s, g);
}

template <FfnFormat F = FfnFormat::FP8>
hipError_t gemm_geglu(const GemmArgs& g, ScaleKind sk, hipStream_t s) {
    if (g.N % 64 || g.K % kCkBK) return hipErrorInvalidValue;
    const dim3 grid(g.N / 64, (g.M + kCkBM - 1) / kCkBM, 1);
    if constexpr (F != FfnFormat::FP8) return ck_launch(chunk_gemm_kernel<Epi::GeGLU, ScaleKind::F32, F>, grid, s, g);
    return sk == ScaleKind::F32 ? ck_launch(chunk_gemm_kernel<Epi::GeGLU, ScaleKind::F32>, grid, s, g)
                                : ck_launch(chunk_gemm_kernel<Epi::GeGLU, ScaleKind::BF16>, grid, s, g);
}

int m_tiles(int M) { return (M + kCkBM - 1) / kCkBM; }

template <ScaleKind SK>
hipError_t post_rows(const float* part, int splits, int M, const void* scale, const uint16_t* w_post, uint16_t* res,
                     const uint16_t* ls, hipStream_t s) {
    if (splits <= 4)
        return ck_launch(chunk_post_rows_kernel<SK, FfnFormat::FP8, 4>, dim3(M), s, part, splits, M, scale,
                         (const float*)nullptr, w_post, res, ls);
    return ck_launch(chunk_post_rows_kernel<SK>, dim3(M), s, part, splits, M, scale, (const float*)nullptr, w_post, res, ls);
}

}  // namespace

hipError_t launch_qkv_chunk(const QkvParams& p, int m0, int M, hipStream_t s, DevCtx* ctx) {
    hipError_t e = ck_launch(chunk_rmsnorm_rows_kernel<true>, dim3(M), s, p.x + (size_t)m0 * kH, p.in_rms, ctx->hbuf);
    if (e != hipSuccess) return e;
    GemmArgs g{};
    g.x = ctx->hbuf; g.M = M; g.N = kQkvRowsTotal; g.K = kH;
    g.w[0] = p.qw; g.w[1] = p.kw; g.w[2] = p.vw;
    g.nseg[0] = 0; g.nseg[1] = kQs; g.nseg[2] = kQs + kPs; g.nseg[3] = kQkvRowsTotal; g.nsegs = 3;
    g.yf = ctx->fbuf;
    // Up to 256 rows, 64-row weight tiles (128 tiles x 2 k splits instead of 64 x 4: half the
    // partial sums; M = 256: 39.3 -> 37.4 us). Beyond, they would not split, and the 512 tiles
    // of M = 1024 measured 112 us against 102 with 128-row tiles.
    const bool narrow = m_tiles(M) == 1;
    const int sp = pick_splits(kQkvRowsTotal / (narrow ? kCkOBN : kCkBN) * m_tiles(M), kH / kCkBK,
                               (size_t)M * kQkvRowsTotal);
    e = narrow ? gemm_partial<FfnFormat::FP8, kCkOBN>(g, sp, p.scale_kind, s) : gemm_partial(g, sp, p.scale_kind, s);
    if (e != hipSuccess) return e;
    const float* part = ctx->fbuf;
    if (sp > 4) return hipErrorInvalidValue;  // 60 k steps: pick_splits never gives 8
    // Up to 256 rows, one workgroup per (head, row): more workgroups hide the loads better (four
    // heads per workgroup measured 28.5 -> 30.6 us for the call at M = 100, even at 256); beyond,
    // four heads per workgroup (M = 1024: 101.5 -> 94.1 us).
    if (narrow) return launch_qkv_heads(p, m0, M, part, sp, s, ctx);
    if (sp <= 2)  // as many partial loads in flight as there are splits
        return p.scale_kind == ScaleKind::F32
            ? ck_launch(chunk_qkv_heads4_kernel<ScaleKind::F32, 2>, dim3(8, M), s, p, m0, M, part, sp, ctx->err)
            : ck_launch(chunk_qkv_heads4_kernel<ScaleKind::BF16, 2>, dim3(8, M), s, p, m0, M, part, sp, ctx->err);
    return p.scale_kind == ScaleKind::F32
        ? ck_launch(chunk_qkv_heads4_kernel<ScaleKind::F32, 4>, dim3(8, M), s, p, m0, M, part, sp, ctx->err)
        : ck_launch(chunk_qkv_heads4_kernel<ScaleKind::BF16, 4>, dim3(8, M), s, p, m0, M, part, sp, ctx->err);
}

// O's A tiles and its split-K GEMM into ctx->fbuf; *sp: the splits
static hipError_t o_chunk_gemm(const OParams& p, int m0, int M, hipStream_t s, DevCtx* ctx, int* sp) {
    hipError_t e = ck_launch(chunk_tile_rows_kernel, dim3(M), s, p.x + (size_t)m0 * kQs, kQs, ctx->pbuf);
    if (e != hipSuccess) return e;
    GemmArgs g{};
    g.x = ctx->pbuf; g.M = M; g.N = kH; g.K = kQs;
    g.w[0] = p.ow; g.nseg[0] = 0; g.nseg[1] = kH; g.nsegs = 1;
    g.yf = ctx->fbuf;
    *sp = pick_splits(kH / kCkOBN * m_tiles(M), kQs / kCkBK, (size_t)M * kH);
    return gemm_partial<FfnFormat::FP8, kCkOBN>(g, *sp, p.scale_kind, s);
}

hipError_t launch_o_chunk(const OParams& p, int m0, int M, hipStream_t s, DevCtx* ctx) {
    int sp = 1;
    const hipError_t e = o_chunk_gemm(p, m0, M, s, ctx, &sp);
    if (e != hipSuccess) return e;
    uint16_t* res = p.residual + (size_t)m0 * kH;
    return p.scale_kind == ScaleKind::F32
        ? post_rows<ScaleKind::F32>(ctx->fbuf, sp, M, p.os, p.post_rms, res, nullptr, s)
        : post_rows<ScaleKind::BF16>(ctx->fbuf, sp, M, p.os, p.post_rms, res, nullptr, s);
}

// normed: the pre-norm's A tiles are already in ctx->hbuf (o_ffn_chunk)
template <FfnFormat F>
hipError_t ffn_chunk(const FfnParams& p, int m0, int M, hipStream_t s, DevCtx* ctx, bool normed = false) {
    uint16_t* res = p.residual + (size_t)m0 * kH;
    hipError_t e = normed ? hipSuccess
                          : ck_launch(chunk_rmsnorm_rows_kernel<true>, dim3(M), s, (const uint16_t*)res, p.pre_rms, ctx->hbuf);
    if (e != hipSuccess) return e;
    GemmArgs g{};
    g.x = ctx->hbuf; g.M = M; g.N = kL; g.K = kH;
    g.w[0] = p.up; g.w2 = p.gate; g.s0 = p.up_s; g.s2 = p.gate_s;
    g.wsc[0] = (const uint8_t*)p.up_s; g.wsc2 = (const uint8_t*)p.gate_s; g.g0 = p.up_g; g.g2 = p.gate_g;
    g.y = ctx->pbuf;
    e = gemm_geglu<F>(g, p.scale_kind, s);
    if (e != hipSuccess) return e;
    GemmArgs d{};
    d.x = ctx->pbuf; d.M = M; d.N = kH; d.K = kL;
    d.w[0] = p.down; d.nseg[0] = 0; d.nseg[1] = kH; d.nsegs = 1;
    d.wsc[0] = (const uint8_t*)p.down_s;
    d.yf = ctx->fbuf;
    const int sp = pick_splits(kH / kCkBN * m_tiles(M), kL / kCkBK, (size_t)M * kH);
    e = gemm_partial<F>(d, sp, p.scale_kind, s);
    if (e != hipSuccess) return e;
    return launch_ffn_post_rows(p, ctx->fbuf, sp, M, res, s);
}

hipError_t launch_ffn_chunk(const FfnParams& p, int m0, int M, hipStream_t s, DevCtx* ctx) {
    switch (p.fmt) {
        case FfnFormat::FP8: return ffn_chunk<FfnFormat::FP8>(p, m0, M, s, ctx);
        case FfnFormat::NVFP4: return ffn_chunk<FfnFormat::NVFP4>(p, m0, M, s, ctx);
        case FfnFormat::MXFP4: return ffn_chunk<FfnFormat::MXFP4>(p, m0, M, s, ctx);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_o_ffn_chunk(const OParams& o, const FfnParams& p, int m0, int M, hipStream_t s, DevCtx* ctx) {
    if (o.residual != p.residual) return hipErrorInvalidValue;
    int sp = 1;
    hipError_t e = o_chunk_gemm(o, m0, M, s, ctx, &sp);
    if (e != hipSuccess) return e;
    uint16_t* res = o.residual + (size_t)m0 * kH;
    const float* part = ctx->fbuf;
    if (o.scale_kind == ScaleKind::F32)
        e = sp <= 4 ? ck_launch(chunk_post_pre_rows_kernel<ScaleKind::F32, 4>, dim3(M), s, part, sp, M, o.os, o.post_rms,
                                res, p.pre_rms, ctx->hbuf)
                    : ck_launch(chunk_post_pre_rows_kernel<ScaleKind::F32, kCkSplitMax>, dim3(M), s, part, sp, M, o.os,
                                o.post_rms, res, p.pre_rms, ctx->hbuf);
    else
        e = sp <= 4 ? ck_launch(chunk_post_pre_rows_kernel<ScaleKind::BF16, 4>, dim3(M), s, part, sp, M, o.os, o.post_rms,
                                res, p.pre_rms, ctx->hbuf)
                    : ck_launch(chunk_post_pre_rows_kernel<ScaleKind::BF16, kCkSplitMax>, dim3(M), s, part, sp, M, o.os,
                                o.post_rms, res, p.pre_rms, ctx->hbuf);
    if (e != hipSuccess) return e;
    switch (p.fmt) {
        case FfnFormat::FP8: return ffn_chunk<FfnFormat::FP8>(p, m0, M, s, ctx, true);
        case FfnFormat::NVFP4: return ffn_chunk<FfnFormat::NVFP4>(p, m0, M, s, ctx, true);
        case FfnFormat::MXFP4: return ffn_chunk<FfnFormat::MXFP4>(p, m0, M, s, ctx, true);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_qkv_heads(const QkvParams& p, int m0, int M, const float* part, int splits, hipStream_t s, DevCtx* ctx) {
    if (splits > 2) return hipErrorInvalidValue;
    return p.scale_kind == ScaleKind::F32
        ? ck_launch(chunk_qkv_heads_kernel<ScaleKind::F32, 2>, dim3(32, M), s, p, m0, M, part, splits, ctx->err)
        : ck_launch(chunk_qkv_heads_kernel<ScaleKind::BF16, 2>, dim3(32, M), s, p, m0, M, part, splits, ctx->err);
}

hipError_t launch_post_rows(const float* part, int splits, int M, const void* scale, ScaleKind sk, const uint16_t* w_post,
                            uint16_t* res, const uint16_t* ls, hipStream_t s) {
    return sk == ScaleKind::F32 ? post_rows<ScaleKind::F32>(part, splits, M, scale, w_post, res, ls, s)
                                : post_rows<ScaleKind::BF16>(part, splits, M, scale, w_post, res, ls, s);
}

hipError_t launch_post_pre_rows(const float* part, int splits, int M, const void* scale, ScaleKind sk,
                                const uint16_t* w_post, uint16_t* res, const uint16_t* w_pre, uint16_t* hout, hipStream_t s) {
    if (splits > 4) return hipErrorInvalidValue;
    return sk == ScaleKind::F32
        ? ck_launch(chunk_post_pre_rows_kernel<ScaleKind::F32, 4, false>, dim3(M), s, part, splits, M, scale, w_post, res,
                    w_pre, hout)
        : ck_launch(chunk_post_pre_rows_kernel<ScaleKind::BF16, 4, false>, dim3(M), s, part, splits, M, scale, w_post, res,
                    w_pre, hout);
}

hipError_t launch_rmsnorm_rows(const uint16_t* x, const uint16_t* w, uint16_t* out, int M, hipStream_t s) {
    return ck_launch(chunk_rmsnorm_rows_kernel<false>, dim3(M), s, x, w, out);
}

hipError_t launch_ffn_post_rows(const FfnParams& p, const float* part, int splits, int M, uint16_t* res, hipStream_t s) {
    switch (p.fmt) {
        case FfnFormat::FP8:
            return p.scale_kind == ScaleKind::F32 ? post_rows<ScaleKind::F32>(part, splits, M, p.down_s, p.post_rms, res, p.layer_scalar, s)
                                                  : post_rows<ScaleKind::BF16>(part, splits, M, p.down_s, p.post_rms, res, p.layer_scalar, s);
        case FfnFormat::NVFP4:
            if (splits > kCkSplitMax) return hipErrorInvalidValue;
            return splits <= 4
                ? ck_launch(chunk_post_rows_kernel<ScaleKind::F32, FfnFormat::NVFP4, 4>, dim3(M), s, part, splits, M,
                            (const void*)nullptr, p.down_g, p.post_rms, res, p.layer_scalar)
                : ck_launch(chunk_post_rows_kernel<ScaleKind::F32, FfnFormat::NVFP4>, dim3(M), s, part, splits, M,
                            (const void*)nullptr, p.down_g, p.post_rms, res, p.layer_scalar);
        case FfnFormat::MXFP4:
            if (splits > kCkSplitMax) return hipErrorInvalidValue;
            return splits <= 4
                ? ck_launch(chunk_post_rows_kernel<ScaleKind::F32, FfnFormat::MXFP4, 4>, dim3(M), s, part, splits, M,
                            (const void*)nullptr, (const float*)nullptr, p.post_rms, res, p.layer_scalar)
                : ck_launch(chunk_post_rows_kernel<ScaleKind::F32, FfnFormat::MXFP4>, dim3(M), s, part, splits, M,
                            (const void*)nullptr, (const float*)nullptr, p.post_rms, res, p.layer_scalar);
    }
    return hipErrorInvalidValue;
}

}  // namespace moa
