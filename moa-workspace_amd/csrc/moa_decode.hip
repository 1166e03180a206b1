// moa_decode.hip -- decode (small-M, weight-streaming GEMV) kernels for gfx950.
//
// At M = 1 the three operators are HBM-bound streams of 1-byte FP8 or packed E2M1 weights.
// Every kernel here:
//   * gives each wavefront a few whole weight rows and issues all of their 16-byte loads
//     first, so a launch keeps ~16-32 KB per wave in flight while the activations are
//     being prepared;
//   * stages the (normalised) activation row in LDS as f32 once per workgroup -- barriers
//     on gfx950 wait only on LDS, so the weight loads stay in flight across them;
//   * dequantises in registers (v_cvt_pk_f32_fp8 / v_cvt_scalef32_pk_f32_fp4) and
//     accumulates exact bf16 x fp8/fp4 products in f32 with fmaf;
//   * reduces each row across the wave with a butterfly (bit-identical in every lane);
//   * resolves the grid-wide dependency (head RMSNorm + RoPE, post-norm + residual) in the
//     last-arriving wave, found with a device-scope ticket -- no second launch.
// blockIdx.y indexes the token row (M <= kMaxDecodeM); rows re-read the same weights, which
// for small M mostly hit L2/MALL.
#include <mutex>
#include <utility>

#include "moa_device.h"
#include "moa_internal.h"
#include "moa_sync.h"

namespace moa {
namespace {

constexpr int kBlock = 256;  // four waves

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

template <ScaleKind SK>
__device__ __forceinline__ float load_scale(const void* p, int i) {
    if constexpr (SK == ScaleKind::F32) return static_cast<const float*>(p)[i];
    else return bf2f(static_cast<const uint16_t*>(p)[i]);
}

// Whole block: true in every thread of the block that arrives last of `expected` on `ctr`.
__device__ __forceinline__ bool block_arrive(uint32_t* ctr, uint32_t expected) {
    __shared__ uint32_t s_last;
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's publishes are done
    __syncthreads();
    if (threadIdx.x == 0) {
        const bool last = counter_add(ctr) + 1u == expected;
        if (last) counter_reset(ctr);
        s_last = last;
    }
    __syncthreads();
    return s_last;
}

// Whole block: two-level arrival of all `nblocks` blocks of the grid row -- block b counts on
// leaf b % kTreeLeaves; the last block of each leaf counts on the root. `tree` holds
// kTreeCounters counters kTicketStride apart.
__device__ __forceinline__ bool block_arrive_tree(uint32_t* tree, uint32_t nblocks) {
    __shared__ uint32_t s_last;
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t leaf = blockIdx.x % kTreeLeaves;
        const uint32_t n_leaf = (nblocks - leaf + kTreeLeaves - 1) / kTreeLeaves;
        const uint32_t n_root = nblocks < (uint32_t)kTreeLeaves ? nblocks : (uint32_t)kTreeLeaves;
        bool last = false;
        uint32_t* lc = tree + leaf * kTicketStride;
        if (counter_add(lc) + 1u == n_leaf) {
            counter_reset(lc);
            uint32_t* rc = tree + kTreeLeaves * kTicketStride;
            last = counter_add(rc) + 1u == n_root;
            if (last) counter_reset(rc);
        }
        s_last = last;
    }
    __syncthreads();
    return s_last;
}

// Post-norm hand-off of the single-launch O and FFN kernels (240 workgroups of 16 output rows):
// per workgroup one partial sum of squares (f32 bits) and eight words of two bf16 outputs; the FFN
// also keeps per workgroup the tag of the last launch whose up/gate rows of that block have been
// claimed (claim words are exchanged, never polled).
struct PostSlots {
    uint64_t part[kFfnPartSlots];
    uint64_t d[kFfnPartSlots][8];
    uint64_t claim[kFfnPartSlots];
};
static_assert(sizeof(PostSlots) == sizeof(uint64_t) * kFfnSlotWords, "slot area size");
constexpr int kPostGrid = 240;     // workgroups of a post-norm hand-off
constexpr int kPostWgRows = 16;    // output rows per workgroup
constexpr int kPostLeaders = 8;    // leader workgroups
constexpr int kPostGroup = kPostGrid / kPostLeaders;  // 30 workgroups per leader
static_assert(kPostGrid * kPostWgRows == kH && 2 * kPostGroup <= 64, "a leader lane owns 8 outputs");

// Test only (Stall::hold; the kernels' Hold instantiations, launched only while a test holds
// workgroups): the held workgroups of a launch wait at entry, bounded by the wall clock.
__device__ __forceinline__ void stall_hold(const Stall& st) {
    if (st.hold_ticks == 0) return;
    const int b = blockIdx.x;
    if (b != st.hold[0] && b != st.hold[1] && b != st.hold[2] && b != st.hold[3]) return;
    const uint64_t t0 = wall_clock64();
    while (wall_clock64() - t0 < st.hold_ticks) __builtin_amdgcn_s_sleep(64);
}

// One wave: publish workgroup b's 16 outputs (bf16 bits dl[0..16)) and their partial sum of
// squares (in row order); post_publish for the calling workgroup.
__device__ __forceinline__ void post_publish_at(PostSlots* slots, uint32_t tag, int b, const uint32_t* dl, int lane) {
    if (lane < kPostWgRows / 2) publish64(&slots->d[b][lane], tagged(tag, dl[2 * lane] | (dl[2 * lane + 1] << 16)));
    if (lane == 0) {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < kPostWgRows; ++i) ss = fmaf(bf2f(dl[i]), bf2f(dl[i]), ss);
        publish64(&slots->part[b], tagged(tag, __float_as_uint(ss)));
    }
}

__device__ __forceinline__ void post_publish(PostSlots* slots, uint32_t tag, const uint32_t* dl, int lane) {
    post_publish_at(slots, tag, blockIdx.x, dl, lane);
}

// post_publish for workgroup b from registers (lane i < 16 holds output i): the same words and the
// same partial sum, for a wave that computed another workgroup's outputs.
__device__ __forceinline__ void post_publish_vals(PostSlots* slots, uint32_t tag, int b, uint32_t v, int lane) {
    const uint32_t lo = __shfl(v, (2 * lane) & 15, kWave), hi = __shfl(v, (2 * lane + 1) & 15, kWave);
    if (lane < kPostWgRows / 2) publish64(&slots->d[b][lane], tagged(tag, lo | (hi << 16)));
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < kPostWgRows; ++i) {
        const float f = bf2f(__shfl(v, i, kWave));
        ss = fmaf(f, f, ss);
    }
    if (lane == 0) publish64(&slots->part[b], tagged(tag, __float_as_uint(ss)));
}

// Rows owned by lane l of leader g: 8 outputs of workgroup g + 8 (l / 2), from row (l % 2) * 8.
__device__ __forceinline__ int post_leader_row(int lane) {
    return (blockIdx.x + kPostLeaders * min(lane / 2, kPostGroup - 1)) * kPostWgRows + (lane % 2) * 8;
}

// One wave of leader workgroup g < kPostLeaders: poll until all 240 partial sums and the outputs of
// workgroups g, g + 8, ... carry `tag`; sum the partials in a fixed order (the same bits in every
// leader) and write those workgroups' residual rows in place (nothing when the poll expired, so
// rows are never computed from stale words). After steal_ticks of waiting the wave computes and
// publishes the lowest missing workgroup's outputs itself (steal(b): the same bits as workgroup b's
// own), then polls again at once. Through: the residual rows go out as agent-scope stores, written
// through to memory rather than left dirty in the L2 (O 0.07-0.15 us faster on two boxes; the FFN
// measured 0.2 us slower that way and keeps plain stores; QKV's output stores gained nothing):
//   out = bf16(bf16(r + bf16(bf16(d * inv) * w)) * ls)    (ls skipped when has_ls is false)
// FO/src/device/shared/rmsnorm.rs:204-296 + residual.rs:189-241. r8 / w8: the lane's residual and
// norm-weight values (prefetched by the caller at post_leader_row).
template <bool Through, typename Steal>
__device__ __forceinline__ void post_leader(PostSlots* slots, uint32_t tag, uint16_t* res, const uint4& r8,
                                            const uint4& w8, bool has_ls, float lsv, int lane, uint32_t* err,
                                            uint32_t steal_ticks, Steal steal) {
    constexpr int NP = (kPostGrid + 63) / 64;
    float part[NP];
    uint32_t dq[4];
    const bool mine_rows = lane < 2 * kPostGroup;
    const int lwg = blockIdx.x + kPostLeaders * min(lane / 2, kPostGroup - 1);
    const uint64_t t0 = wall_clock64();
    bool expired = false;
    for (;;) {
        bool ok = true;
        int victim = kPostGrid;  // the lowest workgroup with a stale word (uniform)
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const bool real = lane + 64 * i < kPostGrid;
            const uint64_t v = collect64(&slots->part[min(lane + 64 * i, kPostGrid - 1)]);
            part[i] = real ? __uint_as_float((uint32_t)v) : 0.0f;
            const bool stale = real && (uint32_t)(v >> 32) != tag;
            ok = ok && !stale;
            const uint64_t m = __ballot(stale);
            if (m && victim == kPostGrid) victim = 64 * i + __builtin_ctzll(m);
        }
        bool dstale = false;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint64_t v = collect64(&slots->d[lwg][(lane % 2) * 4 + k]);
            dq[k] = (uint32_t)v;
            dstale = dstale || (mine_rows && (uint32_t)(v >> 32) != tag);
        }
        ok = ok && !dstale;
        if (__all(ok)) break;
        const uint64_t dt = wall_clock64() - t0;
        if (dt > kSpinTicks) {
            if (lane == 0) atomicOr(err, kErrSpinTimeout);
            expired = true;
            break;
        }
        if (__builtin_expect(dt > steal_ticks, 0)) {
            const uint64_t md = __ballot(dstale);
            if (victim == kPostGrid && md) victim = blockIdx.x + kPostLeaders * (__builtin_ctzll(md) / 2);
            if (victim < kPostGrid) {
                if (lane == 0) atomicAdd(err + kErrTakeOvers, 1u);
                steal(victim);
                continue;
            }
        }
        __builtin_amdgcn_s_sleep(1);
    }
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < NP; ++i) tot += part[i];
    const float inv = rms_inverse(wave_sum(tot), kH);
    if (mine_rows && !expired) {
        const uint32_t rw[4] = {r8.x, r8.y, r8.z, r8.w}, ww[4] = {w8.x, w8.y, w8.z, w8.w};
        uint32_t o[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            uint32_t pair = 0;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float d = bf2f((dq[k] >> (16 * h)) & 0xffffu);
                const float n = rbf((d * inv) * bf2f((ww[k] >> (16 * h)) & 0xffffu));
                float sres = rbf(bf2f((rw[k] >> (16 * h)) & 0xffffu) + n);
                if (has_ls) sres = rbf(sres * lsv);
                pair |= f2bf(sres) << (16 * h);
            }
            o[k] = pair;
        }
        if constexpr (Through) {
            uint64_t* rp = reinterpret_cast<uint64_t*>(res + post_leader_row(lane));
            __hip_atomic_store(rp, ((uint64_t)o[1] << 32) | o[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(rp + 1, ((uint64_t)o[3] << 32) | o[2], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            *reinterpret_cast<uint4*>(res + post_leader_row(lane)) = make_uint4(o[0], o[1], o[2], o[3]);
        }
    }
}

// Deterministic block sum (wave butterflies, then the four wave totals in order).
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    __syncthreads();
    if (lane_id() == 0) red[wave_id()] = v;
    __syncthreads();
    return ((red[0] + red[1]) + red[2]) + red[3];
}

// Activation staging in two phases: *_issue() loads the row into registers and must come
// before the weight loads -- loads retire in order (vmcnt), so staging loads issued after a
// wave's weight loads would make the LDS write wait for the whole weight stream -- and
// *_finish() writes LDS once they arrive.

// h = RMSNorm(x, w) (gemma4.py:83-89) over kH elements; w may be null. Thread t owns elements
// [16t, 16t+16) for t < 240.
struct RmsStage {
    uint4 x0, x1, w0, w1;
};

__device__ __forceinline__ void rms_issue(RmsStage& s, const uint16_t* __restrict__ x,
                                          const uint16_t* __restrict__ w) {
    const int t = min((int)threadIdx.x, kH / 16 - 1);  // threads past the row reload its last chunk
    s.x0 = ld16(x + t * 16);
    s.x1 = ld16(x + t * 16 + 8);
    if (w) {
        s.w0 = ld16(w + t * 16);
        s.w1 = ld16(w + t * 16 + 8);
    }
}

// Whole block: finishes h into LDS as f32.
__device__ __forceinline__ void rms_finish(const RmsStage& s, bool weighted, float* __restrict__ lds, float* __restrict__ red) {
    const int t = threadIdx.x;
    const bool act = t < kH / 16;
    float xv[16];
    float ss = 0.0f;
    if (act) {
        bf16x8_to_f32(s.x0, xv);
        bf16x8_to_f32(s.x1, xv + 8);
#pragma unroll
        for (int i = 0; i < 16; ++i) ss = fmaf(xv[i], xv[i], ss);  // x*x is exact in f32
    }
    ss = wave_sum(ss);
    if (lane_id() == 0) red[wave_id()] = ss;
    __syncthreads();
    const float inv = rms_inverse(((red[0] + red[1]) + red[2]) + red[3], kH);
    if (act) {
        float wv[16];
        if (weighted) {
            bf16x8_to_f32(s.w0, wv);
            bf16x8_to_f32(s.w1, wv + 8);
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float y = xv[i] * inv;
            if (weighted) y = y * wv[i];
            lds[t * 16 + i] = rbf(y);
        }
    }
    __syncthreads();
}

// Whole block of NW waves: h = RMSNorm(x, w) from an RmsStage into LDS as bf16.
template <int NW>
__device__ __forceinline__ void rms_finish_bf16(const RmsStage& s, uint16_t* __restrict__ lds, float* __restrict__ red) {
    const int t = threadIdx.x;
    const bool act = t < kH / 16;
    float xv[16];
    float ss = 0.0f;
    bf16x8_to_f32(s.x0, xv);
    bf16x8_to_f32(s.x1, xv + 8);
    if (act) {
#pragma unroll
        for (int i = 0; i < 16; ++i) ss = fmaf(xv[i], xv[i], ss);  // x*x is exact in f32
    }
    ss = wave_sum(ss);
    if (lane_id() == 0) red[wave_id()] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) tot += red[w];
    const float inv = rms_inverse(tot, kH);
    if (act) {
        float wv[16];
        bf16x8_to_f32(s.w0, wv);
        bf16x8_to_f32(s.w1, wv + 8);
        uint32_t h[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            h[i] = pk_bf16((xv[2 * i] * inv) * wv[2 * i], (xv[2 * i + 1] * inv) * wv[2 * i + 1]);
        *reinterpret_cast<uint4*>(lds + t * 16) = make_uint4(h[0], h[1], h[2], h[3]);
        *reinterpret_cast<uint4*>(lds + t * 16 + 8) = make_uint4(h[4], h[5], h[6], h[7]);
    }
    __syncthreads();
}

// One wave: h = RMSNorm(x, w) over kH elements into LDS as bf16 -- 480 chunks of 8, lane l owning
// chunks l + 64 i (i < 8; lanes 32-63 own 7). No workgroup barrier: the wave alone reduces, so the
// other waves stay free to issue their weight loads. *_issue() loads the row (before any weight
// load of the workgroup), *_finish() writes LDS once it has arrived.
struct WaveRms {
    static constexpr int N = (kH / 8 + 63) / 64;  // 8
    uint4 x[N], w[N];
};
__device__ __forceinline__ void wave_rms_issue(WaveRms& s, const uint16_t* __restrict__ x,
                                               const uint16_t* __restrict__ w, int lane) {
#pragma unroll
    for (int i = 0; i < WaveRms::N; ++i) {
        const int c = min(lane + 64 * i, kH / 8 - 1);  // clamped: lanes past the row reload its last chunk
        s.x[i] = ld16(x + c * 8);
        s.w[i] = ld16(w + c * 8);
    }
}
__device__ __forceinline__ void wave_rms_finish(const WaveRms& s, uint16_t* __restrict__ lds, int lane) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < WaveRms::N; ++i) {
        if (lane + 64 * i < kH / 8) {
            float v[8];
            bf16x8_to_f32(s.x[i], v);
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = fmaf(v[e], v[e], ss);  // x*x is exact in f32
        }
    }
    const float inv = rms_inverse(wave_sum(ss), kH);
#pragma unroll
    for (int i = 0; i < WaveRms::N; ++i) {
        const int c = lane + 64 * i;
        if (c < kH / 8) {
            float v[8], wv[8];
            bf16x8_to_f32(s.x[i], v);
            bf16x8_to_f32(s.w[i], wv);
            uint32_t h[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                h[e] = pk_bf16((v[2 * e] * inv) * wv[2 * e], (v[2 * e + 1] * inv) * wv[2 * e + 1]);
            *reinterpret_cast<uint4*>(lds + c * 8) = make_uint4(h[0], h[1], h[2], h[3]);
        }
    }
}

// A bf16 row of NC 8-element chunks, thread t owning chunks t + 256 i.
template <int NC>
struct RowStage {
    static constexpr int N = (NC + kBlock - 1) / kBlock;
    uint4 v[N];
};

template <int NC>
__device__ __forceinline__ void row_issue(RowStage<NC>& s, const uint16_t* __restrict__ x) {
#pragma unroll
    for (int i = 0; i < RowStage<NC>::N; ++i) {
        const int c = min((int)threadIdx.x + i * kBlock, NC - 1);  // clamped: no branch around the load
        s.v[i] = ld16(x + c * 8);
    }
}

// Whole block: the row into LDS as f32.
template <int NC>
__device__ __forceinline__ void row_finish(const RowStage<NC>& s, float* __restrict__ lds) {
#pragma unroll
    for (int i = 0; i < RowStage<NC>::N; ++i) {
        const int c = threadIdx.x + i * kBlock;
        if (c < NC) {
            float v[8];
            bf16x8_to_f32(s.v[i], v);
            *reinterpret_cast<f32x4*>(lds + c * 8) = f32x4{v[0], v[1], v[2], v[3]};
            *reinterpret_cast<f32x4*>(lds + c * 8 + 4) = f32x4{v[4], v[5], v[6], v[7]};
        }
    }
    __syncthreads();
}

template <int N>
__device__ __forceinline__ void lds_read(const float* lds, int at, float* out) {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
        f32x4 v = *reinterpret_cast<const f32x4*>(lds + at + i);
        out[i] = v[0]; out[i + 1] = v[1]; out[i + 2] = v[2]; out[i + 3] = v[3];
    }
}

// N bf16 activations at element `at` of an LDS row (16-byte aligned), as N/2 pairs.
template <int N>
__device__ __forceinline__ void lds_pairs(const uint16_t* lds, int at, uint32_t* out) {
#pragma unroll
    for (int i = 0; i < N / 8; ++i) {
        const uint4 v = *reinterpret_cast<const uint4*>(lds + at + 8 * i);
        out[4 * i] = v.x; out[4 * i + 1] = v.y; out[4 * i + 2] = v.z; out[4 * i + 3] = v.w;
    }
}

// ------------------------------------------------------------ weight chunks
// A chunk is the 16 weight bytes one lane loads per row per iteration: 16 FP8 codes or 32
// E2M1 codes, plus (FP4) the block-scale codes that cover them. Iteration j, lane l covers
// row bytes [1024 j + 16 l, +16).
template <FfnFormat F>
struct Chunk {
    uint4 q;
    uint32_t s;
};

template <FfnFormat F>
constexpr int elems_per_chunk() { return F == FfnFormat::FP8 ? 16 : 32; }

template <FfnFormat F>
__device__ __forceinline__ void load_chunk(Chunk<F>& c, const uint8_t* row, const uint8_t* srow,
                                           int j, int lane, bool valid) {
    // Invalid (past-the-row) lanes load the row's first chunk -- always in bounds, so the load
    // needs no branch -- and zero it.
    const int l = valid ? lane : 0;
    const int jj = valid ? j : 0;
    uint4 q = ld_stream(row + jj * 1024 + l * 16);
    uint32_t sc = 0;
    if constexpr (F == FfnFormat::NVFP4)  // block 16: two E4M3 scale codes per chunk
        sc = *reinterpret_cast<const uint16_t*>(srow + (jj * 64 + l) * 2);
    else if constexpr (F == FfnFormat::MXFP4)  // block 32: one E8M0 scale code per chunk
        sc = srow[jj * 64 + l];
    c.q = valid ? q : make_uint4(0, 0, 0, 0);
    c.s = valid ? sc : 0u;
}

__device__ __forceinline__ float dot_fp8_16(const float* x, const uint4& q, float acc) {
    float w[16];
    fp8x4_to_f32(q.x, w); fp8x4_to_f32(q.y, w + 4); fp8x4_to_f32(q.z, w + 8); fp8x4_to_f32(q.w, w + 12);
#pragma unroll
    for (int t = 0; t < 16; ++t) acc = fmaf(x[t], w[t], acc);
    return acc;
}

// Eight E2M1 values (decoded at scale 1, exact) times x, accumulated onto acc.
__device__ __forceinline__ float dot_fp4_8(const float* x, uint32_t q, float acc) {
    float w[8];
    fp4x8_to_f32(q, 1.0f, w);
#pragma unroll
    for (int t = 0; t < 8; ++t) acc = fmaf(x[t], w[t], acc);
    return acc;
}

// v_cvt_scalef32_pk_f32_fp4 applies only the exponent of its f32 scale (MX, E8M0 semantics),
// so E2M1 codes are decoded at scale 1 and the block scale multiplies the block's partial sum:
// exact for MXFP4's power-of-two scales; for NVFP4's E4M3 scales it adds one f32 rounding per
// 16 elements to the reference's per-element fold (generate_references.py:398,407).
template <FfnFormat F>
__device__ __forceinline__ float chunk_dot(const float* x, const Chunk<F>& c, float acc) {
    if constexpr (F == FfnFormat::FP8) {
        return dot_fp8_16(x, c.q, acc);
    } else if constexpr (F == FfnFormat::NVFP4) {
        f32x2 s = __builtin_amdgcn_cvt_pk_f32_fp8(c.s, false);  // two E4M3 block scales
        float b0 = dot_fp4_8(x + 8, c.q.y, dot_fp4_8(x, c.q.x, 0.0f));
        float b1 = dot_fp4_8(x + 24, c.q.w, dot_fp4_8(x + 16, c.q.z, 0.0f));
        return fmaf(b1, s[1], fmaf(b0, s[0], acc));
    } else {
        const float s = e8m0_to_f32(c.s);
        float b = dot_fp4_8(x, c.q.x, 0.0f);
        b = dot_fp4_8(x + 8, c.q.y, b);
        b = dot_fp4_8(x + 16, c.q.z, b);
        b = dot_fp4_8(x + 24, c.q.w, b);
        return fmaf(b, s, acc);
    }
}

// Projection commit with the format's rounding rule:
//   FP8:   bf16(dot * s_row)                 generate_references.py:265-274
//   NVFP4: bf16(bf16(dot) * inv_global)      generate_references.py:358-372
//   MXFP4: bf16(dot)
template <FfnFormat F>
__device__ __forceinline__ float proj_commit(float dot, float scale) {
    if constexpr (F == FfnFormat::FP8) return rbf(dot * scale);
    else if constexpr (F == FfnFormat::NVFP4) return rbf(rbf(dot) * scale);
    else return rbf(dot);
}

// out[0:3840] = bf16(bf16(r + N(d)) * ls), N = RMSNorm with w_post or identity when null,
// ls = layer scalar (skipped when null). Whole block: 480 chunks of 8, thread t owns chunks t
// and t + 256. d holds values published by other workgroups (read with collect16).
// FO/src/device/shared/rmsnorm.rs:204-296 + residual.rs:189-241; oracle generate_references.py:411-413.
__device__ __forceinline__ void block_post_residual(const uint16_t* __restrict__ d, const uint16_t* __restrict__ w_post,
                                    uint16_t* __restrict__ r, const uint16_t* __restrict__ ls) {
    __shared__ float red[4];
    constexpr int NC = kH / 8;  // 480
    const int t = threadIdx.x;
    // Residual, post-norm weight and layer scalar first: their loads overlap the collect.
    // Clamped chunk indices keep every load unconditional, so all of them are in flight at once.
    uint4 rq[2], wq[2], dq[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = min(t + i * kBlock, NC - 1);
        rq[i] = ld16(r + c * 8);
        if (w_post) wq[i] = ld16(w_post + c * 8);
    }
    const float lsv = ls ? bf2f(ls[0]) : 1.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) dq[i] = collect16(d + min(t + i * kBlock, NC - 1) * 8);
    float dv[2][8];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        bf16x8_to_f32(dq[i], dv[i]);
        if (t + i * kBlock < NC) {
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = fmaf(dv[i][e], dv[i][e], ss);
        }
    }
    const float inv = rms_inverse(block_sum(ss, red), kH);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = t + i * kBlock;
        if (c >= NC) continue;
        float wv[8], rv[8];
        if (w_post) bf16x8_to_f32(wq[i], wv);
        bf16x8_to_f32(rq[i], rv);
        uint32_t packed[4];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float n = dv[i][e];
            if (w_post) n = rbf((n * inv) * wv[e]);
            float sres = rbf(rv[e] + n);
            if (ls) sres = rbf(sres * lsv);
            const uint32_t bits = f2bf(sres);
            if (e & 1) packed[e >> 1] |= bits << 16; else packed[e >> 1] = bits;
        }
        *reinterpret_cast<uint4*>(r + c * 8) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    }
}

// =================================================================== QKV
// ops::sliding_project_qkv (FO/src/ops.rs:37-76). 8192 projection rows (Q 4096 | K 2048 |
// V 2048), K = 3840. Four rows per wave, 16 per workgroup, 512 workgroups per token row.
constexpr int kQkvR = 4;
constexpr int kQkvRows = kQs + 2 * kPs;

// Per-head epilogue by the head's last workgroup: RMSNorm over 256 (sliding/rmsnorm.rs:22-153),
// RoPE on q/k (sliding/rope.rs:9-211), and the q_out / ring-cache stores (ops.rs:72-75).
// Thread t owns head element t; RoPE partners (t, t ^ 128) meet through LDS.
__device__ __forceinline__ void qkv_head_epilogue(const QkvParams& p, const uint16_t* __restrict__ raw, int head,
                                  int m, uint32_t* err) {
    __shared__ float red[4];
    __shared__ float xch[kDs];
    const int t = threadIdx.x;
    const int32_t rope_off = *p.rope_off;
    const int32_t kv_off = *p.kv_off;
    const bool rope_ok = rope_off >= 0 && (rope_off % (kDs * 2)) == 0 && rope_off / (kDs * 2) + m < kE;
    const bool kv_ok = kv_off >= 0 && (kv_off % (kNs * kDs * 2)) == 0 && kv_off / (kNs * kDs * 2) < kTs;
    if (!rope_ok || !kv_ok) {  // this token row writes nothing (no q_out, K or V) on a bad offset
        if (t == 0) atomicOr(err, (rope_ok ? 0u : kErrRopeOffset) | (kv_ok ? 0u : kErrKvOffset));
        return;
    }
    const int slot = (kv_off / (kNs * kDs * 2) + m) % kTs;
    const int trow = rope_off / (kDs * 2) + m;
    const uint16_t* wn = head < 16 ? p.q_rms : (head < 24 ? p.k_rms : nullptr);
    // norm weight and RoPE row first: their loads overlap the collect
    const float wv = wn ? bf2f(wn[t]) : 1.0f;
    const float cv = bf2f(p.cos[(size_t)trow * kDs + t]);
    const float sv = bf2f(p.sin[(size_t)trow * kDs + t]);
    const float v = bf2f(collect(&raw[head * kDs + t]));
    const float inv = rms_inverse(block_sum(v * v, red), kDs);  // v*v is exact in f32
    float n = v * inv;
    if (wn) n = n * wv;
    n = rbf(n);
    if (head >= 24) {
        p.v_cache[(size_t)slot * (kNs * kDs) + (head - 24) * kDs + t] = (uint16_t)f2bf(n);
        return;
    }
    // y = bf16(bf16(x*cos) + bf16(x_swap*sin_dev)); the table's sin has its low half negated
    // (generate_references.py:200-210), so x_swap is a plain half swap.
    xch[t] = n;
    __syncthreads();
    const float partner = xch[t ^ (kDs / 2)];
    const float a = rbf(n * cv);
    const float b = rbf(partner * sv);
    uint16_t* dst = head < 16 ? p.q_out + (size_t)m * kQs + head * kDs
                              : p.k_cache + (size_t)slot * (kNs * kDs) + (head - 16) * kDs;
    dst[t] = (uint16_t)f2bf(a + b);
}

// ------------------------------------------------------------ QKV of a full-attention layer
// ops::full_project_qkv (FO/src/ops.rs:78-116): 8704 projection rows (Q 8192 | K 512), K = 3840.
// The one KV head's raw projection gives K (weighted RMSNorm over 512, RoPE) and V (unweighted
// RMSNorm) -- the CPU reference's attention_k_eq_v path (gemma4.py:152-166; full/rmsnorm.rs).
// The slot is kv_offset / 1024 + m of the caller's page: a row whose slot falls past the page's
// 512 slots writes nothing and raises the kv-offset error bit.
constexpr int kFqkvRows = kQf + kPf;

// Per-head epilogue by the head's last workgroup: thread t owns head elements t and t + 256,
// which are each other's RoPE partners.
__device__ __forceinline__ void fqkv_head_epilogue(const QkvParams& p, const uint16_t* __restrict__ raw, int head,
                                                   int m, uint32_t* err) {
    __shared__ float red[4];
    const int t = threadIdx.x;
    constexpr int Hf = kDf / 2;
    const int32_t rope_off = *p.rope_off;
    const int32_t kv_off = *p.kv_off;
    const bool rope_ok = rope_off >= 0 && (rope_off % (kDf * 2)) == 0 && rope_off / (kDf * 2) + m < kE;
    const bool kv_ok = kv_off >= 0 && (kv_off % (kDf * 2)) == 0 && kv_off / (kDf * 2) + m < kTf;
    if (!rope_ok || !kv_ok) {  // the row writes nothing (no q_out, K or V)
        if (t == 0) atomicOr(err, (rope_ok ? 0u : kErrRopeOffset) | (kv_ok ? 0u : kErrKvOffset));
        return;
    }
    const int slot = kv_off / (kDf * 2) + m;
    const int trow = rope_off / (kDf * 2) + m;
    const uint16_t* wn = head < kGf ? p.q_rms : p.k_rms;
    const float w0 = bf2f(wn[t]), w1 = bf2f(wn[t + Hf]);
    const float c0 = bf2f(p.cos[(size_t)trow * kDf + t]), c1 = bf2f(p.cos[(size_t)trow * kDf + t + Hf]);
    const float s0 = bf2f(p.sin[(size_t)trow * kDf + t]), s1 = bf2f(p.sin[(size_t)trow * kDf + t + Hf]);
    const float v0 = bf2f(collect(&raw[head * kDf + t])), v1 = bf2f(collect(&raw[head * kDf + t + Hf]));
    const float inv = rms_inverse(block_sum(v0 * v0 + v1 * v1, red), kDf);  // squares of bf16 are exact
    const float u0 = v0 * inv, u1 = v1 * inv;
    if (head == kGf) {  // V: the unweighted norm (full/rmsnorm.rs normalize_value)
        p.v_cache[(size_t)slot * kDf + t] = (uint16_t)f2bf(u0);
        p.v_cache[(size_t)slot * kDf + t + Hf] = (uint16_t)f2bf(u1);
    }
    const float n0 = rbf(u0 * w0), n1 = rbf(u1 * w1);
    // y = bf16(bf16(x*cos) + bf16(x_swap*sin_dev)); the table's sin has its low half negated
    uint16_t* dst = head < kGf ? p.q_out + (size_t)m * kQf + head * kDf : p.k_cache + (size_t)slot * kDf;
    dst[t] = (uint16_t)f2bf(rbf(n0 * c0) + rbf(n1 * s0));
    dst[t + Hf] = (uint16_t)f2bf(rbf(n1 * c1) + rbf(n0 * s1));
}

// Full: false -- sliding_project_qkv (32 heads of 256); true -- full_project_qkv (17 heads of 512;
// raw_all rows are kFqkvRows wide).
template <ScaleKind SK, bool Full>
__global__ __launch_bounds__(kBlock) void qkv_decode_kernel(QkvParams p, int m0, uint16_t* raw_all,
                                                            uint32_t* tickets, uint32_t* err) {
    __shared__ float hs[kH];
    __shared__ float red[4];
    constexpr int R = kQkvR, KI = 4;  // 3840 = 3.75 x 1024: lanes >= 48 idle in the last chunk
    const int m = blockIdx.y;
    const int lane = lane_id(), wave = wave_id();
    const int row0 = blockIdx.x * (4 * R) + wave * R;
    const uint8_t* W;
    const void* S;
    int lr;
    if constexpr (Full) {
        if (row0 < kQf) { W = p.qw; S = p.qs; lr = row0; }
        else { W = p.kw; S = p.ks; lr = row0 - kQf; }
    } else {
        if (row0 < kQs) { W = p.qw; S = p.qs; lr = row0; }
        else if (row0 < kQs + kPs) { W = p.kw; S = p.ks; lr = row0 - kQs; }
        else { W = p.vw; S = p.vs; lr = row0 - kQs - kPs; }
    }

    const float my_scale = load_scale<SK>(S, lr + min(lane, R - 1));  // lane r: row r's scale
    RmsStage st;
    rms_issue(st, p.x + (size_t)(m0 + m) * kH, p.in_rms);
    uint4 wq[R][KI];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int j = 0; j < KI; ++j) {
            const int col = j * 1024 + lane * 16;
            const uint4 q = ld_stream(W + (size_t)(lr + r) * kH + (col < kH ? col : 0));
            wq[r][j] = (col < kH) ? q : make_uint4(0, 0, 0, 0);
        }

    rms_finish(st, true, hs, red);

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < KI; ++j) {
        const int col = j * 1024 + lane * 16;
        if (col < kH) {
            float h[16];
            lds_read<16>(hs, col, h);
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] = dot_fp8_16(h, wq[r][j], acc[r]);
        }
    }
    float mine = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float d = wave_sum(acc[r]);
        if (lane == r) mine = d;
    }
    constexpr int D = Full ? kDf : kDs;
    uint16_t* raw = raw_all + (size_t)m * (Full ? kFqkvRows : kQkvRows);
    if (lane < R) publish(&raw[row0 + lane], f2bf(mine * my_scale));

    // sliding: 0..15 q, 16..23 k, 24..31 v; full: 0..15 q, 16 k (uniform over the block)
    const int head = row0 / D;
    if (!block_arrive(&tickets[(kTicketQkv + m * 32 + head) * kTicketStride], D / (4 * R))) return;
    if constexpr (Full) fqkv_head_epilogue(p, raw, head, m0 + m, err);
    else qkv_head_epilogue(p, raw, head, m0 + m, err);
}

// ------------------------------------------------------------ QKV: single launch (one token row)
// 256 workgroups of nine waves: eight compute four rows each and the ninth (the control wave)
// normalises the activation row and finishes the head. Workgroup b computes 32 rows of head
// h = b % 32 -- rows 16q .. 16q+15 and 128+16q .. 128+16q+15 of the head for q = b / 32, so every
// row's RoPE partner (t ^ 128) is in the same workgroup. The dispatcher deals workgroups to the
// 8 XCDs round-robin (XCD = b % 8), so a head's 8 workgroups share one XCD and its exchange
// never crosses to the other I/O die: an agent-scope round trip between two workgroups measured
// about 635 ns on one XCD and 1015 ns across the dies, and the kernel 9.0 against 9.3 us with
// h = b / 8. Only latency depends on this placement, not the result.
// The head's RMSNorm needs the sum of squares of all 256 rows: each workgroup publishes its
// partial sum tagged with the launch's epoch (the head's epoch counter gets one add per workgroup
// at entry; epoch_tag) and polls the head's 8 tagged words. Then the control wave normalises,
// rotates and stores the workgroup's 32 values.
// Every output depends only on the inputs (nothing is read that the launch writes), so a control
// wave that has waited stall.steal_ticks for a sibling's partial sum computes that sibling's 32 rows
// itself, publishes their partial sum and stores their outputs too; a sibling that was only late
// writes the same bits again.
constexpr int kQkvWaves = 8;                                // row waves; wave 8 is the control wave
constexpr int kQkvBlock = 64 * (kQkvWaves + 1);
constexpr int kQkvRowsW = 4;                                // rows per row wave
constexpr int kQkvWgRows = kQkvWaves * kQkvRowsW;           // 32
constexpr int kQkvGrid = kQkvRows / kQkvWgRows;             // 256
constexpr int kQkvPerHead = kDs / kQkvWgRows;               // 8 workgroups per head
static_assert(kQkvPerHead * kQkvWgRows == kDs && kQkvGrid == 32 * kQkvPerHead, "QKV grid");
static_assert(kQkvPerHead == kQkvEpochPer && kQkvEpochCounters == 32, "one epoch counter per head");
static_assert(32 * kQkvPerHead == kQkvSlotWords, "one tagged word per workgroup");

// Head-local row of slot s = 4 w + r (w < 4: first half of the head, w >= 4: second half).
__device__ __forceinline__ int qkv_local_row(int q, int s) { return s < 16 ? 16 * q + s : 128 + 16 * q + (s - 16); }

template <ScaleKind SK, bool Hold = false>
__global__ __launch_bounds__(kQkvBlock) void qkv_fused_kernel(QkvParams p, int m0, uint64_t* slots, uint32_t* tickets,
                                                              uint32_t* err, Stall stall) {
    __shared__ uint16_t hs[kH];
    __shared__ float raw[kQkvWgRows];
    __shared__ float sraw[kQkvPerHead][kQkvWgRows];  // rows of siblings taken over
    __shared__ uint32_t s_hs;                         // hs complete (written by the control wave)
    if constexpr (Hold) stall_hold(stall);
    const int lane = lane_id(), wave = wave_id();
    const bool ctl = wave == kQkvWaves;
    const int head = blockIdx.x % 32, q = blockIdx.x / 32;

    // the wave's four consecutive rows (the control wave's are never loaded)
    const int t0 = qkv_local_row(q, min(wave, kQkvWaves - 1) * kQkvRowsW);
    const uint8_t* W;
    const void* S;
    if (head < 16) { W = p.qw; S = p.qs; }
    else if (head < 24) { W = p.kw; S = p.ks; }
    else { W = p.vw; S = p.vs; }
    const int hrow0 = (head < 16 ? head : (head < 24 ? head - 16 : head - 24)) * kDs;  // the head's first row in its matrix
    const int mrow0 = hrow0 + t0;
    const float scale = load_scale<SK>(S, mrow0 + min(lane, kQkvRowsW - 1));

    // Control wave: offsets and norm weight at entry (ahead of every weight load, so waiting for
    // them later costs nothing); lane i < 32 serves head-local row qkv_local_row(q, i).
    uint32_t tag = 0;
    float wv = 1.0f, cv = 0.0f, sv = 0.0f;
    int32_t rope_off = 0, kv_off = 0;
    const int te = qkv_local_row(q, min(lane, kQkvWgRows - 1));
    if (ctl) {
        rope_off = *p.rope_off;
        kv_off = *p.kv_off;
        const uint16_t* wn = head < 16 ? p.q_rms : (head < 24 ? p.k_rms : nullptr);
        if (wn) wv = bf2f(wn[te]);
    }

    // The control wave loads the activation row and normalises it alone; a barrier keeps every
    // row wave's weight loads behind that row (a CU serves its loads in order).
    WaveRms st;
    if (ctl) {
        if (lane == 0) s_hs = 0u;
        wave_rms_issue(st, p.x + (size_t)m0 * kH, p.in_rms, lane);
    }
    __syncthreads();
    constexpr int KI = 4;  // 3840 = 3.75 x 1024: lanes >= 48 idle in the last chunk
    uint4 wq[kQkvRowsW][KI];
    auto issue_row = [&](int r) {
#pragma unroll
        for (int j = 0; j < KI; ++j) {
            const int col = j * 1024 + lane * 16;
            const uint4 v = ld_stream(W + (size_t)(mrow0 + r) * kH + (col < kH ? col : 0));
            wq[r][j] = col < kH ? v : make_uint4(0, 0, 0, 0);
        }
    };
    // Every row wave issues all four rows at once and then waits for the normalised row on a flag
    // the control wave raises, not on a barrier: a wave's issue stalls while its CU's load queue
    // is full, and behind a barrier such a wave would hold up the control wave (the activation
    // row comes back late, queued behind every CU's weights). Measured 9.08 -> 8.91 us against
    // three rows before a barrier and the fourth behind the first dots. The wait is bounded.
    if (!ctl) {
#pragma unroll
        for (int r = 0; r < kQkvRowsW; ++r) issue_row(r);
        const uint64_t tw = wall_clock64();
        while (__hip_atomic_load(&s_hs, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) == 0u) {
            if (wall_clock64() - tw > kSpinTicks) {
                if (lane == 0) atomicOr(err, kErrSpinTimeout);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    } else {
        wave_rms_finish(st, hs, lane);
        if (lane == 0) __hip_atomic_store(&s_hs, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    }

    // The epoch and the RoPE row behind the weights: they are needed only after the head's
    // exchange, and loads retire in order -- issued first, the epoch add's return would hold up
    // every later wait of the wave.
    if (ctl) {
        if (lane == 0) tag = epoch_tag<kQkvEpochPer>(epoch_add(tickets + (kTicketQkvEpoch + head) * kTicketStride));
        const int trow = rope_off / (kDs * 2) + m0;
        if (head < 24 && rope_off >= 0 && (rope_off % (kDs * 2)) == 0 && trow < kE) {
            cv = bf2f(p.cos[(size_t)trow * kDs + te]);
            sv = bf2f(p.sin[(size_t)trow * kDs + te]);
        }
    }

    if (!ctl) {
        uint32_t x[KI][8];
#pragma unroll
        for (int j = 0; j < KI; ++j) {
            const int col = j * 1024 + lane * 16;
            if (col < kH) lds_pairs<16>(hs, col, x[j]);
            else {
#pragma unroll
                for (int i = 0; i < 8; ++i) x[j][i] = 0u;
            }
        }
        float mine = 0.0f;
#pragma unroll
        for (int r = 0; r < kQkvRowsW; ++r) {
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < KI; ++j) acc = dot_fp8x16_bf16(x[j], wq[r][j], acc);
            acc = wave_sum(acc);
            if (lane == r) mine = acc;
        }
        if (lane < kQkvRowsW) raw[wave * kQkvRowsW + lane] = rbf(mine * scale);  // generate_references.py:265-274
    }
    __syncthreads();
    if (!ctl) return;

    // RMSNorm over the head (sliding/rmsnorm.rs:22-153): partial sum of this workgroup's 32 rows,
    // then the head's 8 partials in workgroup order.
    tag = __shfl(tag, 0, kWave);
    uint64_t* hslots = slots + head * kQkvPerHead;
    if (lane == 0) {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < kQkvWgRows; ++i) ss = fmaf(raw[i], raw[i], ss);  // exact squares of bf16
        publish64(hslots + q, tagged(tag, __float_as_uint(ss)));
    }
    // sibling qv's 32 raw rows by this wave, each row as qv's row waves compute it, into sraw[qv];
    // then their partial sum, published as qv would, and returned
    auto take_over = [&](int qv) -> float {
        float rv = 0.0f;  // lane s < 32: slot s
#pragma unroll 1
        for (int w = 0; w < kQkvWaves; ++w) {
            const int row = hrow0 + qkv_local_row(qv, w * kQkvRowsW);
            uint4 sq[kQkvRowsW][KI];
#pragma unroll
            for (int r = 0; r < kQkvRowsW; ++r)
#pragma unroll
                for (int j = 0; j < KI; ++j) {
                    const int col = j * 1024 + lane * 16;
                    const uint4 v = ld_stream(W + (size_t)(row + r) * kH + (col < kH ? col : 0));
                    sq[r][j] = col < kH ? v : make_uint4(0, 0, 0, 0);
                }
#pragma unroll
            for (int r = 0; r < kQkvRowsW; ++r) {
                float acc = 0.0f;
#pragma unroll
                for (int j = 0; j < KI; ++j) {
                    const int col = j * 1024 + lane * 16;
                    uint32_t x[8];
                    if (col < kH) lds_pairs<16>(hs, col, x);
                    else {
#pragma unroll
                        for (int i = 0; i < 8; ++i) x[i] = 0u;
                    }
                    acc = dot_fp8x16_bf16(x, sq[r][j], acc);
                }
                acc = wave_sum(acc);
                if (lane == w * kQkvRowsW + r) rv = rbf(acc * load_scale<SK>(S, row + r));
            }
        }
        if (lane < kQkvWgRows) sraw[qv][lane] = rv;
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < kQkvWgRows; ++i) {
            const float f = __shfl(rv, i, kWave);
            ss = fmaf(f, f, ss);
        }
        if (lane == 0) publish64(hslots + qv, tagged(tag, __float_as_uint(ss)));
        return ss;
    };
    float part = 0.0f, tpart = 0.0f;  // tpart: lane qv's partial sum when qv was taken over
    uint32_t taken = 0;               // siblings taken over
    const uint64_t tp = wall_clock64();
    for (;;) {
        const uint64_t v = collect64(hslots + min(lane, kQkvPerHead - 1));
        const bool took = lane < kQkvPerHead && ((taken >> lane) & 1u);
        part = took ? tpart : __uint_as_float((uint32_t)v);
        const uint64_t ms = __ballot(lane < kQkvPerHead && !took && (uint32_t)(v >> 32) != tag);
        if (ms == 0) break;
        const uint64_t dt = wall_clock64() - tp;
        if (dt > kSpinTicks) {  // expired: store nothing rather than stale values
            if (lane == 0) atomicOr(err, kErrSpinTimeout);
            return;
        }
        if (__builtin_expect(dt > stall.steal_ticks, 0)) {
            const int qv = __builtin_ctzll(ms);
            if (lane == 0) atomicAdd(err + kErrTakeOvers, 1u);
            const float ss = take_over(qv);
            if (lane == qv) tpart = ss;
            taken |= 1u << qv;
            continue;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < kQkvPerHead; ++i) tot += __shfl(part, i, kWave);
    const float inv = rms_inverse(tot, kDs);

    const bool rope_ok = rope_off >= 0 && (rope_off % (kDs * 2)) == 0 && rope_off / (kDs * 2) + m0 < kE;
    const bool kv_ok = kv_off >= 0 && (kv_off % (kNs * kDs * 2)) == 0 && kv_off / (kNs * kDs * 2) < kTs;
    if (!rope_ok || !kv_ok) {  // this token row writes nothing (no q_out, K or V) on a bad offset
        if (blockIdx.x == 0 && lane == 0) atomicOr(err, (rope_ok ? 0u : kErrRopeOffset) | (kv_ok ? 0u : kErrKvOffset));
        return;
    }
    const int slot = (kv_off / (kNs * kDs * 2) + m0) % kTs;
    // lane s < 32: slot s (head-local row t) from its raw value, norm weight and RoPE factors
    auto emit = [&](float rawv, float wvv, float cvv, float svv, int t) {
        float n = rawv * inv;
        if (head < 24) n = n * wvv;
        n = rbf(n);
        // y = bf16(bf16(x*cos) + bf16(x_swap*sin_dev)); the table's sin has its low half negated
        // (generate_references.py:200-210), so x_swap is a plain half swap: slot i ^ 16 holds row t ^ 128.
        const float partner = __shfl_xor(n, 16, kWave);
        if (lane >= kQkvWgRows) return;
        if (head >= 24) {
            p.v_cache[(size_t)slot * (kNs * kDs) + (head - 24) * kDs + t] = (uint16_t)f2bf(n);
            return;
        }
        const float a = rbf(n * cvv);
        const float b = rbf(partner * svv);
        uint16_t* dst = head < 16 ? p.q_out + (size_t)m0 * kQs + head * kDs
                                  : p.k_cache + (size_t)slot * (kNs * kDs) + (head - 16) * kDs;
        dst[t] = (uint16_t)f2bf(a + b);
    };
    emit(raw[min(lane, kQkvWgRows - 1)], wv, cv, sv, te);
    while (taken) {
        const int qv = __builtin_ctz(taken);
        taken &= taken - 1;
        const int tv = qkv_local_row(qv, min(lane, kQkvWgRows - 1));
        const uint16_t* wn = head < 16 ? p.q_rms : (head < 24 ? p.k_rms : nullptr);
        const int trow = rope_off / (kDs * 2) + m0;
        const float wvv = wn ? bf2f(wn[tv]) : 1.0f;
        const float cvv = head < 24 ? bf2f(p.cos[(size_t)trow * kDs + tv]) : 0.0f;
        const float svv = head < 24 ? bf2f(p.sin[(size_t)trow * kDs + tv]) : 0.0f;
        emit(sraw[qv][min(lane, kQkvWgRows - 1)], wvv, cvv, svv, tv);
    }
}

// ===================================================================== O
// ops::sliding_attention_output (FO/src/ops.rs:130-146). 3840 rows, K = 4096. Two rows per
// wave, 8 per workgroup, 480 workgroups per token row.
constexpr int kOR = 2;

// The attention row as the O projection reads it. Sliding layers: x itself. Full-attention layers
// (KX = kQf; div = the running softmax sums [16] of the row): x divided by its head's sum and
// rounded to bf16, as full_attention_output does before projecting (full/attention.rs
// divide_by_softmax_sum). A head with a zero sum (no valid slot) gives zeros.
__device__ __forceinline__ uint4 o_input_chunk(uint4 v, const float* div, int k) {
    const float d = div[k / kDf];
    float f[8];
    bf16x8_to_f32(v, f);
    uint32_t h[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        h[i] = pk_bf16(d > 0.0f ? f[2 * i] / d : 0.0f, d > 0.0f ? f[2 * i + 1] / d : 0.0f);
    return make_uint4(h[0], h[1], h[2], h[3]);
}

template <ScaleKind SK, int KX>
__global__ __launch_bounds__(kBlock) void o_decode_kernel(OParams p, int m0, uint16_t* pbuf_all,
                                                          uint32_t* tickets) {
    __shared__ float xs[KX];
    constexpr int R = kOR, KI = KX / 1024;
    const int m = blockIdx.y;
    const int lane = lane_id(), wave = wave_id();
    const int row0 = blockIdx.x * (4 * R) + wave * R;

    const float my_scale = load_scale<SK>(p.os, row0 + min(lane, R - 1));
    RowStage<KX / 8> st;
    row_issue(st, p.x + (size_t)(m0 + m) * KX);
    uint4 wq[R][KI];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int j = 0; j < KI; ++j) wq[r][j] = ld_stream(p.ow + (size_t)(row0 + r) * KX + j * 1024 + lane * 16);

    if constexpr (KX == kQf) {  // full-attention layer: divide by the softmax sums
        const float* dv = p.div + (size_t)(m0 + m) * kGf;
#pragma unroll
        for (int i = 0; i < RowStage<KX / 8>::N; ++i)
            st.v[i] = o_input_chunk(st.v[i], dv, min((int)threadIdx.x + i * kBlock, KX / 8 - 1) * 8);
    }
    row_finish(st, xs);

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < KI; ++j) {
        float h[16];
        lds_read<16>(xs, j * 1024 + lane * 16, h);
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = dot_fp8_16(h, wq[r][j], acc[r]);
    }
    float mine = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float d = wave_sum(acc[r]);
        if (lane == r) mine = d;
    }
    uint16_t* pbuf = pbuf_all + (size_t)m * kH;
    if (lane < R) publish(&pbuf[row0 + lane], f2bf(mine * my_scale));

    if (!block_arrive_tree(&tickets[(kTicketO + m * kTreeCounters) * kTicketStride], gridDim.x)) return;
    block_post_residual(pbuf, p.post_rms, p.residual + (size_t)(m0 + m) * kH, nullptr);
}

// ------------------------------------------------------------ O: single launch (one token row)
// kPostGrid workgroups of eight waves, two rows per wave (16 per workgroup). The attention row
// (4096 bf16) is loaded first -- one 16-byte chunk per thread -- and a barrier keeps every wave's
// weight loads behind it (a CU serves its loads in order); the wave's two rows (8 KB) then go out
// at once. Outputs and partial sums of squares leave through the tagged post-norm hand-off; the
// kPostLeaders leaders apply post-norm and residual. The tag is the launch's epoch: the control
// wave of workgroup b adds one to epoch counter b % 15 (16 workgroups per counter; epoch_tag).
// A workgroup's outputs depend only on the attention row and the weights, so a leader that has
// waited stall.steal_ticks computes a missing workgroup's outputs itself (a workgroup that was only
// late publishes the same bits again); only leader g writes the residual rows of its group, so a
// late leader still reads them unchanged.
constexpr int kOWaves = 8;
constexpr int kOBlock = 64 * kOWaves;
constexpr int kORowsW = 2;  // rows per wave
static_assert(kPostGrid * kPostWgRows == kH && kOWaves * kORowsW == kPostWgRows, "O grid");
static_assert(kPostGrid == kOEpochCounters * kOEpochPer, "equal workgroups per epoch counter");

template <ScaleKind SK, int KX, bool Hold = false>
__global__ __launch_bounds__(kOBlock) void o_fused_kernel(OParams p, int m0, PostSlots* slots, uint32_t* tickets,
                                                          uint32_t* err, Stall stall) {
    __shared__ uint16_t xs[KX];
    __shared__ uint32_t dl[kPostWgRows];
    if constexpr (Hold) stall_hold(stall);
    const int lane = lane_id(), wave = wave_id();
    const bool ctl = wave == kOWaves - 1;
    const bool leader = blockIdx.x < kPostLeaders;
    uint16_t* res = p.residual + (size_t)m0 * kH;

    uint32_t tag = 0;
    uint4 r8 = make_uint4(0, 0, 0, 0), w8 = make_uint4(0, 0, 0, 0);
    if (ctl) {
        if (leader) {
            r8 = ld16(res + post_leader_row(lane));
            w8 = ld16(p.post_rms + post_leader_row(lane));
        }
    }
    const int row0 = blockIdx.x * kPostWgRows + wave * kORowsW;
    const float scale = load_scale<SK>(p.os, row0 + min(lane, kORowsW - 1));
    constexpr int XC = KX / 8 / kOBlock;  // 16-byte chunks of the row per thread
    static_assert(XC * 8 * kOBlock == KX, "O row staging");
    uint4 xq[XC];
#pragma unroll
    for (int i = 0; i < XC; ++i) xq[i] = ld16(p.x + (size_t)m0 * KX + (threadIdx.x + i * kOBlock) * 8);
    __syncthreads();
    constexpr int KI = KX / 1024;
    uint4 wq[kORowsW][KI];
#pragma unroll
    for (int r = 0; r < kORowsW; ++r)
#pragma unroll
        for (int j = 0; j < KI; ++j) wq[r][j] = ld_stream(p.ow + (size_t)(row0 + r) * KX + j * 1024 + lane * 16);
    // the epoch add behind the weights (loads retire in order: issued first, its return would
    // hold up every later wait of the wave)
    if (ctl && lane == 0)
        tag = epoch_tag<kOEpochPer>(epoch_add(tickets + (kTicketOEpoch + blockIdx.x % kOEpochCounters) * kTicketStride));
#pragma unroll
    for (int i = 0; i < XC; ++i) {
        const int k = (threadIdx.x + i * kOBlock) * 8;
        *reinterpret_cast<uint4*>(xs + k) = KX == kQf ? o_input_chunk(xq[i], p.div + (size_t)m0 * kGf, k) : xq[i];
    }
    __syncthreads();

    float acc[kORowsW];
#pragma unroll
    for (int r = 0; r < kORowsW; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < KI; ++j) {
        uint32_t x[8];
        lds_pairs<16>(xs, j * 1024 + lane * 16, x);
#pragma unroll
        for (int r = 0; r < kORowsW; ++r) acc[r] = dot_fp8x16_bf16(x, wq[r][j], acc[r]);
    }
    float mine = 0.0f;
#pragma unroll
    for (int r = 0; r < kORowsW; ++r) {
        const float d = wave_sum(acc[r]);
        if (lane == r) mine = d;
    }
    if (lane < kORowsW) dl[wave * kORowsW + lane] = f2bf(mine * scale);  // generate_references.py:265-274
    __syncthreads();
    if (!ctl) return;
    tag = __shfl(tag, 0, kWave);
    post_publish(slots, tag, dl, lane);
    if (!leader) return;
    // workgroup b's 16 outputs by this wave: two rows at a time, each row as b's waves compute it
    auto steal = [&](int b) {
        uint32_t v = 0;
#pragma unroll 1
        for (int r0 = 0; r0 < kPostWgRows; r0 += kORowsW) {
            const int row = b * kPostWgRows + r0;
            uint4 sq[kORowsW][KI];
#pragma unroll
            for (int r = 0; r < kORowsW; ++r)
#pragma unroll
                for (int j = 0; j < KI; ++j) sq[r][j] = ld_stream(p.ow + (size_t)(row + r) * KX + j * 1024 + lane * 16);
            float sa[kORowsW];
#pragma unroll
            for (int r = 0; r < kORowsW; ++r) sa[r] = 0.0f;
#pragma unroll
            for (int j = 0; j < KI; ++j) {
                uint32_t x[8];
                lds_pairs<16>(xs, j * 1024 + lane * 16, x);
#pragma unroll
                for (int r = 0; r < kORowsW; ++r) sa[r] = dot_fp8x16_bf16(x, sq[r][j], sa[r]);
            }
#pragma unroll
            for (int r = 0; r < kORowsW; ++r) {
                const float d = wave_sum(sa[r]);
                if (lane == r0 + r) v = f2bf(d * load_scale<SK>(p.os, row + r));
            }
        }
        post_publish_vals(slots, tag, b, v, lane);
    };
    post_leader<true>(slots, tag, res, r8, w8, false, 1.0f, lane, err, stall.steal_ticks, steal);
}

// =================================================================== FFN
// ops::decoder_feedforward (FO/src/ops.rs:201-239). Two halves:
//   up_gate: pre-RMSNorm, up and gate rows, GeGLU -> p[15360] (bf16)
//   down:    p . W_down rows -> d[3840], then post-norm, residual and the layer scalar in place.
// One token row runs both halves in a single launch (ffn_fused_kernel) when its grid fits on the
// device at once; otherwise, and for 2..16 rows, the matrix-core rows path (moa_rows.hip) runs them.
// Activations (normalised x, p) are bf16 in LDS and enter the dot products as bf16 pairs.
constexpr int kUgRL = 8;     // L rows (an up row and a gate row each) per wave
constexpr int kUgDepth = 2;  // up/gate pipeline ring depth (FP8 rows)
constexpr int kUgDepthFp4 = 2;  // the same for FP4 rows, half as long (measured: depths 3 and 4 are slower)
constexpr int kUgPre = 1;    // ring stages issued before the pre-norm completes (<= kUgDepth - 1)

template <FfnFormat F>
constexpr int row_bytes(int k) { return F == FfnFormat::FP8 ? k : k / 2; }
template <FfnFormat F>
constexpr int scale_row_bytes(int k) { return F == FfnFormat::NVFP4 ? k / 16 : (F == FfnFormat::MXFP4 ? k / 32 : 0); }
template <FfnFormat F>
constexpr int down_chunks() { return (row_bytes<F>(kL) + 1023) / 1024; }

template <FfnFormat F, ScaleKind SK>
__device__ __forceinline__ float row_scale(const void* s, const float* g, int row) {
    if constexpr (F == FfnFormat::FP8) return load_scale<SK>(s, row);
    else if constexpr (F == FfnFormat::NVFP4) return *g;
    else return 1.0f;
}

// A chunk's dot with its EPC activations x[0 .. EPC/2) (bf16 pairs). FP4 block scales multiply
// the block partial sums (see chunk_dot).
template <FfnFormat F>
__device__ __forceinline__ float chunk_dot2(const uint32_t* x, const Chunk<F>& c, float acc) {
    if constexpr (F == FfnFormat::FP8) {
        return dot_fp8x16_bf16(x, c.q, acc);
    } else if constexpr (F == FfnFormat::NVFP4) {
        f32x2 s = __builtin_amdgcn_cvt_pk_f32_fp8(c.s, false);  // two E4M3 block scales
        float b0 = dot_fp4x8_bf16(x + 4, c.q.y, dot_fp4x8_bf16(x, c.q.x, 0.0f));
        float b1 = dot_fp4x8_bf16(x + 12, c.q.w, dot_fp4x8_bf16(x + 8, c.q.z, 0.0f));
        return fmaf(b1, s[1], fmaf(b0, s[0], acc));
    } else {
        float b = dot_fp4x8_bf16(x, c.q.x, 0.0f);
        b = dot_fp4x8_bf16(x + 4, c.q.y, b);
        b = dot_fp4x8_bf16(x + 8, c.q.z, b);
        b = dot_fp4x8_bf16(x + 12, c.q.w, b);
        return fmaf(b, e8m0_to_f32(c.s), acc);
    }
}


struct NoHook {
    __device__ void operator()() const {}
};

// Pre-RMSNorm of the residual row x into hs (whole block of NW waves), then the wave's kUgRL
// up/gate row pairs -- L-rows lbase + g*lstride, g < kUgRL -- through a D-deep ring of loads:
// D - 1 row pairs stay in flight while one is reduced. Returns, in lane g < kUgRL, GeGLU of
// L-row lbase + g*lstride (before its bf16 rounding). after_norm() runs once hs is complete.
template <FfnFormat F, ScaleKind SK, int NW, typename H = NoHook>
__device__ __forceinline__ float up_gate_rows(const FfnParams& p, const uint16_t* __restrict__ x, int lbase,
                                              int lstride, uint16_t* __restrict__ hs, float* __restrict__ red,
                                              H after_norm = H{}) {
    constexpr int EPC = elems_per_chunk<F>();
    constexpr int RB = row_bytes<F>(kH);
    constexpr int SB = scale_row_bytes<F>(kH);
    constexpr int KI = (RB + 1023) / 1024;
    constexpr int RL = kUgRL;
    constexpr int D = F == FfnFormat::FP8 ? kUgDepth : kUgDepthFp4;
    const int lane = lane_id();

    Chunk<F> ring[D][2][KI];
    auto issue = [&](int g, Chunk<F> (&dst)[2][KI]) {
        const int l = lbase + g * lstride;
#pragma unroll
        for (int j = 0; j < KI; ++j) {
            const bool valid = j * 1024 + lane * 16 < RB;
            load_chunk<F>(dst[0][j], p.up + (size_t)l * RB, (const uint8_t*)p.up_s + (size_t)l * SB, j, lane, valid);
            load_chunk<F>(dst[1][j], p.gate + (size_t)l * RB, (const uint8_t*)p.gate_s + (size_t)l * SB, j, lane, valid);
        }
    };
    // lane g holds L-row lbase+g*lstride's up and gate scales (FP8) or the global scales (NVFP4)
    const int lrow = lbase + min(lane, RL - 1) * lstride;
    const float su = row_scale<F, SK>(p.up_s, p.up_g, lrow);
    const float sg = row_scale<F, SK>(p.gate_s, p.gate_g, lrow);
    // The activation row (threads 0-239) goes first, and a barrier keeps every wave's weight
    // loads behind it: a CU serves its waves' loads in order, so an activation load queued after
    // another wave's weight ring would wait for that ring.
    // Only kUgPre stages go out before the pre-norm completes: a wave's issue stalls once its
    // CU's load queue is full, and the norm's barriers wait for every wave.
    RmsStage st{};
    if (wave_id() < 4) rms_issue(st, x, p.pre_rms);
    __syncthreads();
#pragma unroll
    for (int g = 0; g < kUgPre; ++g) issue(g, ring[g]);

    rms_finish_bf16<NW>(st, hs, red);
    after_norm();
#pragma unroll
    for (int g = kUgPre; g < D - 1; ++g) issue(g, ring[g]);
    uint32_t xv[KI][EPC / 2];
#pragma unroll
    for (int j = 0; j < KI; ++j) {
        const int e0 = j * 64 * EPC + lane * EPC;
        if (e0 < kH) lds_pairs<EPC>(hs, e0, xv[j]);
        else {
#pragma unroll
            for (int t = 0; t < EPC / 2; ++t) xv[j][t] = 0u;
        }
    }

    float pv = 0.0f;
#pragma unroll
    for (int g = 0; g < RL; ++g) {
        if (g + D - 1 < RL) issue(g + D - 1, ring[(g + D - 1) % D]);
        const Chunk<F> (&src)[2][KI] = ring[g % D];
        float du = 0.0f, dg = 0.0f;
#pragma unroll
        for (int j = 0; j < KI; ++j) {
            du = chunk_dot2<F>(xv[j], src[0][j], du);
            dg = chunk_dot2<F>(xv[j], src[1][j], dg);
        }
        du = wave_sum(du);
        dg = wave_sum(dg);
        const float up = proj_commit<F>(du, __shfl(su, g, kWave));
        const float gate = proj_commit<F>(dg, __shfl(sg, g, kWave));
        // gemma4.py:197: bf16(bf16(gelu_tanh(gate)) * up)
        if (lane == g) pv = rbf(gelu_tanh(gate)) * up;
    }
    return pv;
}

// The same values as up_gate_rows for a row already normalised in hs, with one row pair in flight
// and the activations read from LDS chunk by chunk: the take-over of another workgroup's rows,
// where the caller's down prefetch and p words hold most registers. Same loads, same dot order.
template <FfnFormat F, ScaleKind SK>
__device__ __forceinline__ float up_gate_rows_lean(const FfnParams& p, int lbase, int lstride, const uint16_t* hs) {
    constexpr int EPC = elems_per_chunk<F>();
    constexpr int RB = row_bytes<F>(kH);
    constexpr int SB = scale_row_bytes<F>(kH);
    constexpr int KI = (RB + 1023) / 1024;
    const int lane = lane_id();
    float pv = 0.0f;
#pragma unroll 1
    for (int g = 0; g < kUgRL; ++g) {
        const int l = lbase + g * lstride;
        Chunk<F> c[2][KI];
#pragma unroll
        for (int j = 0; j < KI; ++j) {
            const bool valid = j * 1024 + lane * 16 < RB;
            load_chunk<F>(c[0][j], p.up + (size_t)l * RB, (const uint8_t*)p.up_s + (size_t)l * SB, j, lane, valid);
            load_chunk<F>(c[1][j], p.gate + (size_t)l * RB, (const uint8_t*)p.gate_s + (size_t)l * SB, j, lane, valid);
        }
        float du = 0.0f, dg = 0.0f;
#pragma unroll
        for (int j = 0; j < KI; ++j) {
            uint32_t x[EPC / 2];
            const int e0 = j * 64 * EPC + lane * EPC;
            if (e0 < kH) lds_pairs<EPC>(hs, e0, x);
            else {
#pragma unroll
                for (int t = 0; t < EPC / 2; ++t) x[t] = 0u;
            }
            du = chunk_dot2<F>(x, c[0][j], du);
            dg = chunk_dot2<F>(x, c[1][j], dg);
        }
        du = wave_sum(du);
        dg = wave_sum(dg);
        const float up = proj_commit<F>(du, row_scale<F, SK>(p.up_s, p.up_g, l));
        const float gate = proj_commit<F>(dg, row_scale<F, SK>(p.gate_s, p.gate_g, l));
        if (lane == g) pv = rbf(gelu_tanh(gate)) * up;  // gemma4.py:197
    }
    return pv;
}

// Chunk j of each of the wave's first n (<= R, uniform over the wave) down rows row0 ...
template <FfnFormat F, int R>
__device__ __forceinline__ void down_chunk_issue(Chunk<F> (&dst)[R], const FfnParams& p, int row0, int n, int j,
                                                 int lane) {
    constexpr int RB = row_bytes<F>(kL);
    constexpr int SB = scale_row_bytes<F>(kL);
#pragma unroll
    for (int r = 0; r < R; ++r)
        if (r < n)
            load_chunk<F>(dst[r], p.down + (size_t)(row0 + r) * RB,
                          p.down_s ? (const uint8_t*)p.down_s + (size_t)(row0 + r) * SB : nullptr, j, lane,
                          j * 1024 + lane * 16 < RB);
}

// ------------------------------------------------------------ single launch (one token row)
// Both halves in one grid of kFfnGrid workgroups of eight waves -- one workgroup per CU, so the
// waves sharing a CU's memory path are symmetric -- that must all be resident at once (the host
// checks the occupancy before choosing this kernel). Each workgroup computes 64 GeGLU values
// (8 per wave; stage g of the ring reads eight consecutive L-rows, one per wave), then 16 down
// rows (2 per wave).
//
// Two grid-wide dependencies: every down row needs all 15360 GeGLU values (p), and the post-norm
// of every output needs the sum of squares of all 3840 down outputs.
//
// p: tagged words instead of a barrier. Every workgroup's control wave publishes the workgroup's
// 64 GeGLU values as 32 64-bit words (two bf16 values and the launch's tag). It issues them before
// any other load of the workgroup: a CU serves its loads in order, so the words are not queued
// behind the workgroup's weight loads. Then every wave issues its first kFfnDownPre down chunks,
// and behind them every thread its first read of p (15 words; workgroups start at different words
// so that they do not all request one line). Words that do not yet carry the tag are read again
// until they do. No atomic arrival or poll sits between the last workgroup's up/gate rows and
// everyone's p. (FP4 weights used an arrival-tree barrier here before; the tagged words measured
// 0.2-0.35 us faster.)
// The launch's tag: 15 epoch counters, each advanced by 16 workgroups per launch of any format
// (epoch_tag). Consecutive launches never share a tag, so a word left by an earlier launch does
// not carry the current one.
//
// Post-norm: every workgroup publishes its 16 down outputs and its partial sum of squares, each
// 64-bit word carrying the launch's tag (a word holding the tag is complete, so no counters), and
// is done. The kPostLeaders leader workgroups poll the tags. Leader g sums all 240 partials in a
// fixed order (deterministic, the same bits in every leader) and writes the outputs of the
// workgroups b = g (mod kPostLeaders). Few pollers keep the tagged lines free of contention.
//
// Every poll is bounded by the wall clock (kSpinTicks): on expiry it sets kErrSpinTimeout in the
// device error word and carries on, so every wave exits even if the grid were not resident.
//
// Waits that last stall.steal_ticks take the missing work over, so the launch completes correctly
// with any part of its grid resident:
//   * p: a waiting workgroup computes a missing block's 64 GeGLU values from its own normalised
//     row and publishes them. Each block's values are published by exactly one workgroup, the
//     first to exchange the launch's tag into the block's claim word (the owner does so as soon as
//     its norm is done, long before any wait could expire). An owner that loses the exchange
//     started late and may have read residual rows the leaders had already rewritten; it
//     publishes nothing.
//   * post-norm: a leader computes a missing workgroup's down outputs from p and publishes them
//     (the same bits as the owner's, which depend only on p and the weights).
//   * Leader g alone writes the residual rows of its group, so a late leader finds them unchanged.
constexpr int kFfnWaves = 8;
constexpr int kFfnBlock = 64 * kFfnWaves;
constexpr int kFfnGrid = kL / (kFfnWaves * kUgRL);  // 240 workgroups
constexpr int kFfnWgRows = kH / kFfnGrid;           // 16 down rows per workgroup
constexpr int kFfnCtl = kFfnWaves - 1;              // the control wave
constexpr int kFfnDownR = kFfnWgRows / kFfnWaves;   // 2 down rows per wave
constexpr int kFfnDownPre = 8;                      // down chunks per row loaded before p is staged (FP8; 6-10 measured alike, 12 spills)
// FP8 down chunks per row loaded right behind the reads of p (ffn_fused_kernel; graph-replayed
// 30.60 -> 30.29 us with 3, 30.46 with 2, 30.51 with 4). FP4 rows load none there (1 or 2 measured
// alike or slower), nor does o_ffn_fused_kernel (3: no change).
constexpr int kFfnDownPost = 3;
constexpr int kFfnDownPreFp4 = 4;                   // the same for FP4 rows (8 chunks; measured: 2 equal, 6 and 8 slower)
static_assert(kFfnGrid == kFfnEpochCounters * kFfnEpochPer, "equal workgroups per epoch counter");
static_assert(kFfnDownR * kFfnWaves == kFfnWgRows, "two down rows per wave");
static_assert(kFfnGrid == kPostGrid && kFfnWgRows == kPostWgRows, "post-norm hand-off shape");

// Tagged words w[i] whose high half is not `tag` are read again from addr(i).
template <int N, typename A, int... I>
__device__ __forceinline__ void reload_stale(uint64_t (&w)[N], uint32_t tag, A addr, std::integer_sequence<int, I...>) {
    ((w[I] = (uint32_t)(w[I] >> 32) != tag ? collect64(addr(I)) : w[I]), ...);
}

// word w of thread t in read i of the p words: workgroups start at different words (rotation by
// 32 b), so that 240 readers of the same 61 KB do not request the same lines at the same time
__device__ __forceinline__ int ffn_pword(int i) { return (threadIdx.x + kFfnBlock * i + blockIdx.x * 32) % (kL / 2); }

// Shared memory of the FFN half of the single-launch kernels (the kernel declares each array).
struct FfnShared {
    uint16_t* sh;  // [kL] normalised x (first kH), then the GeGLU row p
    uint16_t* sx;  // [kH] normalised x, kept for a take-over of another block's rows
    float* red;    // [kFfnWaves]
    float* pl;     // [kFfnWaves * kUgRL]
    uint32_t* dl;  // [kFfnWgRows] the workgroup's down outputs (bf16 bits)
    uint32_t *s_tag, *s_expired, *s_stall;
    int* s_victim;
};

// The FFN from the GeGLU values on, in a grid of kFfnGrid workgroups (ffn_fused_kernel and
// o_ffn_fused_kernel): p through the tagged words, the down rows, then the post-norm hand-off or
// (without a post-norm) each workgroup's own rows. pv: lane g < kUgRL of wave w holds GeGLU row
// 8 g + w of the block (before its bf16 rounding); claim_old: what the block's claim exchange
// returned (control wave, lane 0); dscale: down scale of row drow0 + lane (lanes < kFfnDownR);
// control wave: r8 / w8 a leader's residual and post-norm weight values at post_leader_row (with
// the post-norm), r1 the residual value of row 16 b + lane (without it), ls_bits the layer scalar.
// LS: down chunks per row issued right behind the first reads of p.
template <FfnFormat F, ScaleKind SK, int LS = 0>
__device__ __forceinline__ void ffn_down_post(const FfnParams& p, const FfnShared& s, float pv, uint32_t ep_tag,
                                              uint32_t claim_old, uint16_t* res, int drow0, float dscale,
                                              const uint4& r8, const uint4& w8, uint32_t r1, uint32_t ls_bits,
                                              uint64_t* ptag, PostSlots* slots, uint32_t* err, const Stall& stall) {
    constexpr int KD = down_chunks<F>();
    constexpr int EPC = elems_per_chunk<F>();
    const int lane = lane_id(), wave = wave_id();
    const bool ctl = wave == kFfnCtl;
    const bool leader = blockIdx.x < kPostLeaders;
    const bool post = p.post_rms != nullptr;
    uint16_t* const sh = s.sh;
    const uint16_t* const sx = s.sx;
    float* const pl = s.pl;
    uint32_t* const dl = s.dl;
    uint32_t& s_tag = *s.s_tag;
    uint32_t& s_expired = *s.s_expired;
    uint32_t& s_stall = *s.s_stall;
    int& s_victim = *s.s_victim;
    if (lane < kUgRL) pl[lane * kFfnWaves + wave] = pv;
    if (ctl && lane == 0) {
        s_tag = ep_tag;
        s_expired = 0u;
        s_stall = 0u;
    }
    __syncthreads();  // pl complete; every wave has read its x out of sh
    const uint32_t tag = s_tag;

    // Down loads only once the whole workgroup is through its up/gate rows (issued earlier they
    // would queue ahead of the slower waves' up/gate loads, which the barrier waits for).
    constexpr int PDW = F == FfnFormat::FP8 ? kFfnDownPre : kFfnDownPreFp4;
    constexpr int PD = PDW < KD ? PDW : KD;
    // Chunks [0, PD) of the wave's rows are loaded ahead of the reads of p, chunks [PD, PR) right
    // behind them (so that the memory keeps streaming while p comes back), the rest through the
    // ring while the dots run.
    constexpr int PA = PD + LS <= KD ? LS : KD - PD;
    constexpr int PR = PD + PA;
    constexpr int RS = PR < KD ? PR + 1 : PR;  // ring slots
    Chunk<F> ring[RS][kFfnDownR];
    {
        // p by tagged words instead of a barrier. The control wave's 32 words (two GeGLU values and
        // the launch's tag each) are issued before any other load of the workgroup: a CU serves
        // its loads in order, so they are not queued behind this workgroup's weight loads. Every
        // wave (the control wave too) then issues its first PD down chunks and every thread its
        // first read of p; words not yet current are read again until they are.
        if (ctl) {
            const bool won = __shfl(claim_old, 0, kWave) != tag;
            if (won && lane < kFfnWaves * kUgRL / 2)
                publish64(ptag + blockIdx.x * (kFfnWaves * kUgRL / 2) + lane,
                          tagged(tag, pk_bf16(pl[2 * lane], pl[2 * lane + 1])));
        }
        __syncthreads();  // the publish is issued ahead of every load below
        constexpr int PW = kL / 2 / kFfnBlock;  // 15 words per thread
        static_assert(PW * kFfnBlock == kL / 2, "p words per thread");
        auto pword = [](int i) { return ffn_pword(i); };
        // The down prefetch goes out first and the reads of p behind it: a CU returns its loads in
        // order, so a read of p issued ahead of the prefetch would come back early, find the words
        // of the slowest workgroups not yet published, and its re-read would then queue behind the
        // whole prefetch. Behind it, the first read lands when nearly every word is current.
#pragma unroll
        for (int j = 0; j < PD; ++j) down_chunk_issue<F, kFfnDownR>(ring[j], p, drow0, kFfnDownR, j, lane);
        uint64_t pw[PW];
#pragma unroll
        for (int i = 0; i < PW; ++i) pw[i] = collect64(ptag + pword(i));
        if constexpr (PA > 0) {
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = PD; j < PR; ++j) down_chunk_issue<F, kFfnDownR>(ring[j], p, drow0, kFfnDownR, j, lane);
            __builtin_amdgcn_sched_barrier(0);
        }
        const uint64_t t0 = wall_clock64();
        bool stalled = false;
        auto current = [&]() {
            bool ok = true;
#pragma unroll
            for (int i = 0; i < PW; ++i) ok = ok && (uint32_t)(pw[i] >> 32) == tag;
            return __all(ok) != 0;
        };
        // One round of the wait: false while the words are still stale and time is left.
        auto poll = [&]() {
            const uint64_t dt = wall_clock64() - t0;
            if (dt > kSpinTicks) {
                if (lane == 0) {
                    atomicOr(err, kErrSpinTimeout);
                    s_expired = 1u;
                }
                return true;
            }
            if (__builtin_expect(dt > stall.steal_ticks, 0)) {
                stalled = true;
                if (lane == 0) s_stall = 1u;
                return true;
            }
            __builtin_amdgcn_s_sleep(1);
            // reload the words still carrying an older tag (unrolled at compile time)
            reload_stale(pw, tag, [&](int i) { return ptag + pword(i); }, std::make_integer_sequence<int, PW>{});
            return current();
        };
        if constexpr (PA > 0) {
            // The first check in straight-line code: the compiler then waits for the reads of p
            // alone, not for the chunks behind them (at a loop head it waits for every load).
            if (!current()) {
                while (!poll()) {
                }
                // every load of this path complete, so that the compiler's count stays exact below
                __builtin_amdgcn_s_waitcnt(0);
            }
        } else {
            while (!current() && !poll()) {
            }
        }
        if (!stalled) {
#pragma unroll
            for (int i = 0; i < PW; ++i) *reinterpret_cast<uint32_t*>(sh + 2 * pword(i)) = (uint32_t)pw[i];
        }
        __syncthreads();  // p staged, unless a wave stalled
        if (__builtin_expect(s_stall && !s_expired, 0)) {
            // Every wave of the workgroup together: the control wave finds the blocks whose first
            // word is stale (a block whose first word is current has an owner that is publishing
            // it), claims one, and the workgroup computes its values from the copy of the
            // normalised row and publishes them; until every word carries the tag.
            for (;;) {
                reload_stale(pw, tag, [&](int i) { return ptag + pword(i); }, std::make_integer_sequence<int, PW>{});
                bool ok = true;
#pragma unroll
                for (int i = 0; i < PW; ++i) ok = ok && (uint32_t)(pw[i] >> 32) == tag;
                if (__syncthreads_and(ok)) break;
                if (ctl) {
                    constexpr int NB = (kFfnGrid + kWave - 1) / kWave;
                    uint64_t cand[NB];
#pragma unroll
                    for (int i = 0; i < NB; ++i) {
                        const int b = lane + kWave * i;
                        const uint64_t w0 = collect64(ptag + min(b, kFfnGrid - 1) * 32);
                        cand[i] = __ballot(b < kFfnGrid && (uint32_t)(w0 >> 32) != tag);
                    }
                    int victim = -1;
                    if (wall_clock64() - t0 > kSpinTicks) {
                        if (lane == 0) atomicOr(err, kErrSpinTimeout);
                        victim = -2;
                    } else if (lane == 0) {
                        for (int i = 0; i < NB && victim < 0; ++i)
                            for (uint64_t m = cand[i]; m && victim < 0; m &= m - 1) {
                                const int b = kWave * i + __builtin_ctzll(m);
                                if (__hip_atomic_exchange(reinterpret_cast<uint32_t*>(&slots->claim[b]), tag,
                                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != tag)
                                    victim = b;
                            }
                    }
                    if (lane == 0) {
                        if (victim == -2) s_expired = 1u;
                        if (victim >= 0) atomicAdd(err + kErrTakeOvers, 1u);
                        s_victim = victim;
                    }
                }
                __syncthreads();
                const int victim = s_victim;
                if (victim == -2) break;
                if (victim < 0) {
                    __builtin_amdgcn_s_sleep(8);
                    continue;
                }
                const float vv = up_gate_rows_lean<F, SK>(p, victim * (kFfnWaves * kUgRL) + wave, kFfnWaves, sx);
                if (lane < kUgRL) pl[lane * kFfnWaves + wave] = vv;
                __syncthreads();
                // the next round reads the words back (the block's claim keeps it from being taken
                // again while they become visible)
                if (ctl && lane < kFfnWaves * kUgRL / 2)
                    publish64(ptag + victim * (kFfnWaves * kUgRL / 2) + lane,
                              tagged(tag, pk_bf16(pl[2 * lane], pl[2 * lane + 1])));
                __syncthreads();  // pl is free again
            }
#pragma unroll
            for (int i = 0; i < PW; ++i) *reinterpret_cast<uint32_t*>(sh + 2 * pword(i)) = (uint32_t)pw[i];
            // The down prefetch again: the take-over used its registers (and with them, its
            // values are not kept live through the take-over).
#pragma unroll
            for (int j = 0; j < PR; ++j) down_chunk_issue<F, kFfnDownR>(ring[j], p, drow0, kFfnDownR, j, lane);
            __syncthreads();  // p staged
        }
    }

    // ---- down: the ring streams the rest of the rows while the dots run
    {
        float acc[kFfnDownR];
#pragma unroll
        for (int r = 0; r < kFfnDownR; ++r) acc[r] = 0.0f;
#pragma unroll
        for (int j = 0; j < KD; ++j) {
            if (j + PR < KD) down_chunk_issue<F, kFfnDownR>(ring[(j + PR) % RS], p, drow0, kFfnDownR, j + PR, lane);
            const int e0 = j * 64 * EPC + lane * EPC;
            if (e0 < kL) {
                uint32_t x[EPC / 2];
                lds_pairs<EPC>(sh, e0, x);
#pragma unroll
                for (int r = 0; r < kFfnDownR; ++r) acc[r] = chunk_dot2<F>(x, ring[j % RS][r], acc[r]);
            }
        }
        float mine = 0.0f;
#pragma unroll
        for (int r = 0; r < kFfnDownR; ++r) {
            const float dsum = wave_sum(acc[r]);
            if (lane == r) mine = dsum;
        }
        if (lane < kFfnDownR) dl[wave * kFfnDownR + lane] = f2bf(proj_commit<F>(mine, dscale));
    }
    __syncthreads();  // dl complete
    // A workgroup whose wait for p expired has computed from stale words: it stores and publishes
    // nothing, so its residual rows keep their input values (and the leaders' polls expire too).
    if (!ctl || s_expired) return;

    // FO/src/device/shared/rmsnorm.rs:204-296 + residual.rs:189-241: out = bf16(bf16(r + n) * ls),
    // n = bf16(bf16(d * inv) * w) with the post-norm, n = d without it.
    const float lsv = p.layer_scalar ? bf2f(ls_bits) : 1.0f;
    if (!post) {
        // Nothing to wait for: the barrier already ordered every workgroup's read of the residual
        // row before these writes.
        if (lane < kFfnWgRows) {
            float sres = rbf(bf2f(r1) + bf2f(dl[lane]));
            if (p.layer_scalar) sres = rbf(sres * lsv);
            res[blockIdx.x * kFfnWgRows + lane] = (uint16_t)f2bf(sres);
        }
        return;
    }
    post_publish(slots, tag, dl, lane);
    if (!leader) return;
    // workgroup b's 16 down outputs by this wave: two rows at a time, each row as b's waves compute
    // it (the chunks in order, kSB loads of each row in flight)
    auto steal = [&](int b) {
        constexpr int kSB = 4;
        uint32_t v = 0;
#pragma unroll 1
        for (int r0 = 0; r0 < kFfnWgRows; r0 += kFfnDownR) {
            const int drow = b * kFfnWgRows + r0;
            float acc[kFfnDownR];
#pragma unroll
            for (int r = 0; r < kFfnDownR; ++r) acc[r] = 0.0f;
#pragma unroll 1
            for (int j0 = 0; j0 < KD; j0 += kSB) {
                Chunk<F> c[kSB][kFfnDownR];
#pragma unroll
                for (int jj = 0; jj < kSB; ++jj)
                    if (j0 + jj < KD) down_chunk_issue<F, kFfnDownR>(c[jj], p, drow, kFfnDownR, j0 + jj, lane);
#pragma unroll
                for (int jj = 0; jj < kSB; ++jj) {
                    const int e0 = (j0 + jj) * 64 * EPC + lane * EPC;
                    if (j0 + jj < KD && e0 < kL) {
                        uint32_t x[EPC / 2];
                        lds_pairs<EPC>(sh, e0, x);
#pragma unroll
                        for (int r = 0; r < kFfnDownR; ++r) acc[r] = chunk_dot2<F>(x, c[jj][r], acc[r]);
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < kFfnDownR; ++r) {
                const float dsum = wave_sum(acc[r]);
                if (lane == r0 + r) v = f2bf(proj_commit<F>(dsum, row_scale<F, SK>(p.down_s, p.down_g, drow + r)));
            }
        }
        post_publish_vals(slots, tag, b, v, lane);
    };
    post_leader<false>(slots, tag, res, r8, w8, p.layer_scalar != nullptr, lsv, lane, err, stall.steal_ticks, steal);
}

template <FfnFormat F, ScaleKind SK, bool Hold = false>
__global__ __launch_bounds__(kFfnBlock) __attribute__((amdgpu_waves_per_eu(2, 2)))
void ffn_fused_kernel(FfnParams p, int m0, uint64_t* ptag, PostSlots* slots, uint32_t* tickets, uint32_t* err,
                      Stall stall) {
    __shared__ uint16_t sh[kL];
    __shared__ uint16_t sx[kH];
    __shared__ float red[kFfnWaves];
    __shared__ float pl[kFfnWaves * kUgRL];
    __shared__ uint32_t dl[kFfnWgRows];
    constexpr int kLs = F == FfnFormat::FP8 ? kFfnDownPost : 0;
    __shared__ uint32_t s_tag, s_expired, s_stall;
    __shared__ int s_victim;
    const FfnShared s{sh, sx, red, pl, dl, &s_tag, &s_expired, &s_stall, &s_victim};
    if constexpr (Hold) stall_hold(stall);
    const int lane = lane_id(), wave = wave_id();
    const bool ctl = wave == kFfnCtl;
    const bool leader = blockIdx.x < kPostLeaders;
    // The launch's tag: 15 counters of 16 workgroups each advance by one block per launch (every
    // format shares them, so post-norm slot tags never repeat across formats). Needed only after
    // up/gate.
    uint32_t ep_tag = 0;
    if (ctl && lane == 0)
        ep_tag = epoch_tag<kFfnEpochPer>(epoch_add(tickets + (kTicketFfnEpoch + blockIdx.x % kFfnEpochCounters) * kTicketStride));
    uint16_t* res = p.residual + (size_t)m0 * kH;
    const bool post = p.post_rms != nullptr;

    const int drow0 = blockIdx.x * kFfnWgRows + wave * kFfnDownR;
    const float dscale = row_scale<F, SK>(p.down_s, p.down_g, drow0 + min(lane, kFfnDownR - 1));

    // Epilogue operands of the control wave, fetched now (off the critical path). With a post-norm
    // a leader's lane l < 2 * kPostGroup owns 8 outputs of workgroup g + 8 (l / 2), rows
    // (l % 2) * 8 ..; without one, every workgroup writes its own 16 outputs (lanes 0-15).
    uint4 r8 = make_uint4(0, 0, 0, 0), w8 = make_uint4(0, 0, 0, 0);
    uint32_t r1 = 0, ls_bits = 0;
    if (ctl) {
        if (p.layer_scalar) ls_bits = p.layer_scalar[0];
        if (post && leader) {
            r8 = ld16(res + post_leader_row(lane));
            w8 = ld16(p.post_rms + post_leader_row(lane));
        } else if (!post) {
            r1 = res[blockIdx.x * kFfnWgRows + min(lane, kFfnWgRows - 1)];
        }
    }

    // ---- up/gate: stage g reads L-rows base + 8g + wave; lane g's value is GeGLU row 8g + wave.
    // Once the norm is done the block's claim goes out (its return arrives behind the first stage)
    // and the normalised row is copied aside.
    uint32_t claim_old = 0;
    auto claim = [&] {
        if (ctl && lane == 0)
            claim_old = __hip_atomic_exchange(reinterpret_cast<uint32_t*>(&slots->claim[blockIdx.x]), ep_tag,
                                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (threadIdx.x < kH / 8)
            reinterpret_cast<uint4*>(sx)[threadIdx.x] = reinterpret_cast<const uint4*>(sh)[threadIdx.x];
    };
    const int lbase = blockIdx.x * (kFfnWaves * kUgRL) + wave;
    const float pv = up_gate_rows<F, SK, kFfnWaves>(p, res, lbase, kFfnWaves, sh, red, claim);
    ffn_down_post<F, SK, kLs>(p, s, pv, ep_tag, claim_old, res, drow0, dscale, r8, w8, r1, ls_bits, ptag, slots, err,
                         stall);
}

// ============================================================= O -> FFN (one launch)
// The tail of the reference's sliding-layer decode step (FO/src/host/runtime.rs:440-459, then
// the mlp call at 543-571): ops::sliding_attention_output and then ops::decoder_feedforward on
// the same residual row, in one grid of kFfnGrid workgroups of eight waves. The result has the
// same bits as the two operators called one after the other.
//
// O phase: workgroup b computes O rows 16 b .. 16 b + 15 (two per wave, as o_fused_kernel) and
// publishes them with their partial sum of squares through tagged post-norm words. Every
// workgroup -- not only leaders -- then reads all 240 workgroups' words and applies O's post-norm
// and residual add itself, summing the partial sums in the leaders' order (post_leader), so
// every workgroup holds the same bits. The residual row after O (r1) never goes to memory: it is
// the FFN's input row, and stays in LDS for the FFN's own residual add.
//
// The FFN's first two up/gate ring stages go out during the O phase: the first behind O's weight
// loads, the second behind the reads of O's words. A CU returns its loads in order, so those
// reads land once the first stage has (about 2 us after O's weights), when normally every
// workgroup has published; the second stage is in flight behind them, so the weight stream does
// not pause for O's grid-wide dependency.
//
// Tags: the FFN's epoch counters give the launch one tag for its three hand-offs; O's words live
// in a slot area only this kernel writes (the FFN's p and post-norm words are shared with
// ffn_fused_kernel, whose tags come from the same counters).
//
// Take-over: a workgroup that has waited stall.steal_ticks for O's words computes the lowest
// missing workgroup's O rows itself (they depend only on the attention row and W_o) and
// publishes them; several workgroups may do so for one, with the same bits. From the GeGLU
// values on, the FFN's take-overs apply (ffn_down_post). A workgroup that started so late that
// the leaders had already written residual rows computes a wrong r1, but its up/gate block has
// then been claimed by another workgroup, so it publishes no GeGLU value; its O and down rows
// depend only on the attention row, p and the weights, and a leader's own residual rows are
// written by it alone.
// O's post-norm words of the single-launch O -> FFN kernel, in kOfnReplicas copies: every
// workgroup reads all 240 workgroups' words, and 240 coherent reads of each line serialise where
// the line lives; workgroup b reads copy b % kOfnReplicas.
constexpr int kOfnReplicas = kOfnCopies;

// One wave: publish workgroup b's outputs (dl) and partial sum in every copy -- lane l writes word
// l % 9 of copy l / 9 (seven copies per store instruction).
__device__ __forceinline__ void ofn_publish(PostSlots* copies, uint32_t tag, int b, const uint32_t* dl, int lane) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < kPostWgRows; ++i) ss = fmaf(bf2f(dl[i]), bf2f(dl[i]), ss);  // post_publish's order
    const int w = lane % 9;
    const uint64_t v = w < 8 ? tagged(tag, dl[2 * w] | (dl[2 * w + 1] << 16)) : tagged(tag, __float_as_uint(ss));
#pragma unroll
    for (int c0 = 0; c0 < kOfnReplicas; c0 += 7) {
        const int c = c0 + lane / 9;
        if (lane < 63 && c < kOfnReplicas) publish64(w < 8 ? &copies[c].d[b][w] : &copies[c].part[b], v);
    }
}

template <FfnFormat F, ScaleKind SKO, ScaleKind SK, bool Hold = false>
__global__ __launch_bounds__(kFfnBlock) __attribute__((amdgpu_waves_per_eu(2, 2)))
void o_ffn_fused_kernel(OParams o, FfnParams p, int m0, PostSlots* oslots, uint64_t* ptag, PostSlots* slots,
                        uint32_t* tickets, uint32_t* err, Stall stall) {
    constexpr int EPC = elems_per_chunk<F>();
    constexpr int RB = row_bytes<F>(kH);
    constexpr int SB = scale_row_bytes<F>(kH);
    constexpr int KI = (RB + 1023) / 1024;
    constexpr int KO = kQs / 1024;  // O weight chunks per row and lane
    constexpr int RL = kUgRL;
    static_assert(kFfnWaves * kORowsW == kPostWgRows && kFfnGrid == kPostGrid, "O rows per workgroup");
    static_assert(kQs == 8 * kFfnBlock, "one 16-byte chunk of the attention row per thread");
    static_assert(kH == 16 * kPostGrid, "thread t < 240 owns O workgroup t's 16 outputs");
    __shared__ uint16_t sh[kL];
    __shared__ uint16_t sx[kH];
    __shared__ float red[kFfnWaves];
    __shared__ float pl[kFfnWaves * kUgRL];
    __shared__ uint32_t dl[kFfnWgRows];
    __shared__ uint32_t s_tag, s_expired, s_stall;
    __shared__ int s_victim;
    __shared__ uint16_t xs[kQs];        // the attention row
    __shared__ uint16_t r1s[kH];        // the residual row after O
    __shared__ uint32_t odl[kPostWgRows];  // this workgroup's O outputs (bf16 bits)
    __shared__ uint32_t vdl[kPostWgRows];  // a taken-over workgroup's
    __shared__ int s_ovictim;
    const FfnShared s{sh, sx, red, pl, dl, &s_tag, &s_expired, &s_stall, &s_victim};
    if constexpr (Hold) stall_hold(stall);
    const int lane = lane_id(), wave = wave_id(), t = threadIdx.x;
    const bool ctl = wave == kFfnCtl;
    const bool leader = blockIdx.x < kPostLeaders;
    const bool post = p.post_rms != nullptr;
    const bool own = t < kPostGrid;  // owns O workgroup t's outputs: rows 16 t .. 16 t + 15
    uint16_t* res = p.residual + (size_t)m0 * kH;
    // The launch's tag, before any load (as ffn_fused_kernel): the control wave waits for the
    // exchange's return where the result is first held, and issued behind the O weights that wait
    // would cover them too, delaying its share of up/gate stage 0.
    uint32_t ep_tag = 0;
    if (ctl && lane == 0)
        ep_tag = epoch_tag<kFfnEpochPer>(epoch_add(tickets + (kTicketFfnEpoch + blockIdx.x % kFfnEpochCounters) * kTicketStride));

    // Operands first in every wave's load order: the attention row (a 16-byte chunk per thread);
    // thread t < 240 its 16 residual values and both norm weights there; the scales; the control
    // wave its epilogue operands.
    const uint4 xq = ld16(o.x + (size_t)m0 * kQs + t * 8);
    uint4 rv0 = make_uint4(0, 0, 0, 0), rv1 = rv0, wo0 = rv0, wo1 = rv0;
    RmsStage st{};
    if (own) {
        rv0 = ld16(res + t * 16);
        rv1 = ld16(res + t * 16 + 8);
        wo0 = ld16(o.post_rms + t * 16);
        wo1 = ld16(o.post_rms + t * 16 + 8);
        st.w0 = ld16(p.pre_rms + t * 16);
        st.w1 = ld16(p.pre_rms + t * 16 + 8);
    }
    const int orow0 = blockIdx.x * kPostWgRows + wave * kORowsW;
    const float oscale = load_scale<SKO>(o.os, orow0 + min(lane, kORowsW - 1));
    const int lbase = blockIdx.x * (kFfnWaves * RL) + wave;
    const int lrow = lbase + min(lane, RL - 1) * kFfnWaves;
    const float su = row_scale<F, SK>(p.up_s, p.up_g, lrow);
    const float sg = row_scale<F, SK>(p.gate_s, p.gate_g, lrow);
    const int drow0 = blockIdx.x * kFfnWgRows + wave * kFfnDownR;
    const float dscale = row_scale<F, SK>(p.down_s, p.down_g, drow0 + min(lane, kFfnDownR - 1));
    uint4 w8 = make_uint4(0, 0, 0, 0);
    uint32_t ls_bits = 0;
    if (ctl) {
        if (p.layer_scalar) ls_bits = p.layer_scalar[0];
        if (post && leader) w8 = ld16(p.post_rms + post_leader_row(lane));
    }
    __syncthreads();  // every wave's operand loads are issued ahead of the weight loads below

    // O's two rows per wave, then up/gate stage 0
    uint4 wq[kORowsW][KO];
#pragma unroll
    for (int r = 0; r < kORowsW; ++r)
#pragma unroll
        for (int j = 0; j < KO; ++j) wq[r][j] = ld_stream(o.ow + (size_t)(orow0 + r) * kQs + j * 1024 + lane * 16);
    __builtin_amdgcn_sched_barrier(0);
    // Three register stages of up/gate rows: stages 0 and 1 go out around the reads of O's words,
    // stage 2 once the words are complete (graph-replayed 36.97 -> 36.56 us; issued with stage 1,
    // 37.3, or once the pre-norm is done, 36.96; four stages, 37.4).
    constexpr int NR = 3;
    Chunk<F> ring[NR][2][KI];
    auto issue = [&](int g, Chunk<F> (&dst)[2][KI]) {
        const int l = lbase + g * kFfnWaves;
#pragma unroll
        for (int j = 0; j < KI; ++j) {
            const bool valid = j * 1024 + lane * 16 < RB;
            load_chunk<F>(dst[0][j], p.up + (size_t)l * RB, (const uint8_t*)p.up_s + (size_t)l * SB, j, lane, valid);
            load_chunk<F>(dst[1][j], p.gate + (size_t)l * RB, (const uint8_t*)p.gate_s + (size_t)l * SB, j, lane, valid);
        }
    };
    *reinterpret_cast<uint4*>(xs + t * 8) = xq;
    __syncthreads();

    // this wave's two rows of an O workgroup: bf16((x . W_o[row]) * scale) into dst
    // (generate_references.py:265-274)
    auto o_rows = [&](const uint4 (&w)[kORowsW][KO], float sc, uint32_t* dst) {
        float acc[kORowsW];
#pragma unroll
        for (int r = 0; r < kORowsW; ++r) acc[r] = 0.0f;
#pragma unroll
        for (int j = 0; j < KO; ++j) {
            uint32_t x[8];
            lds_pairs<16>(xs, j * 1024 + lane * 16, x);
#pragma unroll
            for (int r = 0; r < kORowsW; ++r) acc[r] = dot_fp8x16_bf16(x, w[r][j], acc[r]);
        }
        float mine = 0.0f;
#pragma unroll
        for (int r = 0; r < kORowsW; ++r) {
            const float d = wave_sum(acc[r]);
            if (lane == r) mine = d;
        }
        if (lane < kORowsW) dst[wave * kORowsW + lane] = f2bf(mine * sc);
    };
    o_rows(wq, oscale, odl);
    if (ctl && lane == 0) {
        s_tag = ep_tag;
        s_expired = 0u;
        s_stall = 0u;
    }
    __syncthreads();  // odl complete; the tag in LDS
    const uint32_t tag = s_tag;
    if (ctl) ofn_publish(oslots, tag, blockIdx.x, odl, lane);
    // The publish leaves the CU ahead of every later load of the workgroup: a store queued behind
    // stage 0 would reach memory only once stage 0 has landed, and the other workgroups' reads
    // would find it missing.
    __syncthreads();

    // O's words. A CU returns its loads in the order they were issued, but a load reads memory
    // when it is issued: a read queued behind a prefetch comes back late AND holds what memory
    // held at its issue. So the words are read twice at most, each read ahead of one up/gate
    // stage: the first right after this workgroup's publish (nothing but landed O weights ahead
    // of it: it comes back within a round trip, current for every workgroup that published by
    // then), stage 0 behind it; the second goes out once the first is back -- by then normally
    // every workgroup has published -- with stage 1 behind it, and lands with stage 0, which the
    // up/gate loop needs next anyway. The 2160 words are read flat and coalesced (word j =
    // t + 512 k: d[0][0] .. d[239][7], then part[0 .. 239]) and regrouped through LDS. The
    // workgroup's own words count as current -- its reads could overtake its own stores -- and
    // are taken from odl. Reads and checks are branch-free straight-line code, so each check waits
    // for its own read alone (a branch around the reads, or a check at the head of a loop, makes
    // the compiler wait for every load in flight).
    constexpr int kOWords = 9 * kPostGrid;
    constexpr int kOR = (kOWords + kFfnBlock - 1) / kFfnBlock;  // reads per thread
    PostSlots* const mine = oslots + blockIdx.x % kOfnReplicas;
    auto jof = [&](int k) { return min(t + kFfnBlock * k, kOWords - 1); };
    auto wg_of = [&](int k) { const int j = jof(k); return j < 8 * kPostGrid ? j >> 3 : j - 8 * kPostGrid; };
    auto waddr = [&](int k) {
        const int j = jof(k);
        return j < 8 * kPostGrid ? &mine->d[0][0] + j : &mine->part[j - 8 * kPostGrid];
    };
    uint64_t ow[kOR];
    auto current = [&] {
        bool ok = true;
#pragma unroll
        for (int k = 0; k < kOR; ++k) ok = ok && ((uint32_t)(ow[k] >> 32) == tag || wg_of(k) == (int)blockIdx.x);
        return ok;
    };
#pragma unroll
    for (int k = 0; k < kOR; ++k) ow[k] = collect64(waddr(k));
    // every wave's read goes out before any wave's stage: a read queued behind another wave's
    // stage would come back with that stage
    __syncthreads();
    issue(0, ring[0]);
    __builtin_amdgcn_sched_barrier(0);
    {
        // the second read once the first is back (the tag compares come first: the barrier
        // waits for every wave's), the words the first read found current kept
        bool keep[kOR];
#pragma unroll
        for (int k = 0; k < kOR; ++k) keep[k] = (uint32_t)(ow[k] >> 32) == tag;
        __syncthreads();
        uint64_t again[kOR];
#pragma unroll
        for (int k = 0; k < kOR; ++k) again[k] = collect64(waddr(k));
        __syncthreads();
        issue(1, ring[1]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < kOR; ++k) ow[k] = keep[k] ? ow[k] : again[k];
    }
    if (!__syncthreads_and(current())) {
        // Rare (a workgroup started late): poll until every word is current, taking a missing
        // workgroup's O rows over after stall.steal_ticks.
        const uint64_t t0 = wall_clock64();
        uint64_t tsteal = t0;
        for (;;) {
            const uint64_t now = wall_clock64();
            if (__syncthreads_or(now - t0 > kSpinTicks)) {
                // nothing of this launch is stored or published by this workgroup; the others'
                // waits for its GeGLU values take them over
                if (t == 0) atomicOr(err, kErrSpinTimeout);
                return;
            }
            if (__builtin_expect(__syncthreads_or(now - tsteal > stall.steal_ticks), 0)) {
                // the lowest workgroup with a stale word: its rows, two per wave, as its own waves
                // compute them
                if (t == 0) s_ovictim = kPostGrid;
                __syncthreads();
#pragma unroll
                for (int k = 0; k < kOR; ++k)
                    if ((uint32_t)(ow[k] >> 32) != tag && wg_of(k) != (int)blockIdx.x) atomicMin(&s_ovictim, wg_of(k));
                __syncthreads();
                const int v = s_ovictim;
                const int vrow0 = v * kPostWgRows + wave * kORowsW;
                uint4 vq[kORowsW][KO];
#pragma unroll
                for (int r = 0; r < kORowsW; ++r)
#pragma unroll
                    for (int j = 0; j < KO; ++j)
                        vq[r][j] = ld_stream(o.ow + (size_t)(vrow0 + r) * kQs + j * 1024 + lane * 16);
                o_rows(vq, load_scale<SKO>(o.os, vrow0 + min(lane, kORowsW - 1)), vdl);
                __syncthreads();
                if (ctl) ofn_publish(oslots, tag, v, vdl, lane);
                if (t == 0) atomicAdd(err + kErrTakeOvers, 1u);
                tsteal = wall_clock64();
            } else {
                __builtin_amdgcn_s_sleep(1);
            }
            reload_stale(ow, tag, waddr, std::make_integer_sequence<int, kOR>{});
            if (__syncthreads_and(current())) break;
        }
        // Every load of this path complete: after the loop the compiler cannot count the loads in
        // flight, and without this wait it would make the common path below wait for all of them
        // (stage 1 included) wherever it first uses a register loaded before the loop.
        __builtin_amdgcn_s_waitcnt(0);
    }
    // stage 2 behind every read of the words: a read queued behind it would come back with it
    issue(2, ring[2]);
    __builtin_amdgcn_sched_barrier(0);

    // The words into LDS (the FFN's p row area: free until the pre-norm writes it), this
    // workgroup's own from odl; then O's post-norm and residual (FO/src/device/shared/
    // rmsnorm.rs:204-296, projection.rs:577-605): r1 = bf16(r + bf16(bf16(d * inv) * w_post)),
    // inv from the 240 partial sums in post_leader's order (lane l: parts l, l + 64, l + 128,
    // l + 192; then the wave butterfly), in every wave.
    uint64_t* const owl = reinterpret_cast<uint64_t*>(sh);
    static_assert(sizeof(uint64_t) * kOWords <= sizeof(uint16_t) * kL, "O's words fit the p row area");
    {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < kPostWgRows; ++i) ss = fmaf(bf2f(odl[i]), bf2f(odl[i]), ss);  // post_publish's order
#pragma unroll
        for (int k = 0; k < kOR; ++k) {
            const int j = t + kFfnBlock * k;
            const int i = j & 7;
            const uint64_t own_word = j < 8 * kPostGrid ? tagged(tag, odl[2 * i] | (odl[2 * i + 1] << 16))
                                                         : tagged(tag, __float_as_uint(ss));
            if (j < kOWords) owl[j] = wg_of(k) == (int)blockIdx.x ? own_word : ow[k];
        }
    }
    __syncthreads();
    {
        float tot = 0.0f;
#pragma unroll
        for (int i = 0; i < (kPostGrid + 63) / 64; ++i) {
            const int b = lane + 64 * i;
            tot += b < kPostGrid ? __uint_as_float((uint32_t)owl[8 * kPostGrid + b]) : 0.0f;
        }
        const float oinv = rms_inverse(wave_sum(tot), kH);
        if (own) {
            const uint32_t rw[8] = {rv0.x, rv0.y, rv0.z, rv0.w, rv1.x, rv1.y, rv1.z, rv1.w};
            const uint32_t ww[8] = {wo0.x, wo0.y, wo0.z, wo0.w, wo1.x, wo1.y, wo1.z, wo1.w};
            uint32_t o8[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t dq = (uint32_t)owl[8 * t + k];
                uint32_t pair = 0;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const float d = bf2f((dq >> (16 * h)) & 0xffffu);
                    const float n = rbf((d * oinv) * bf2f((ww[k] >> (16 * h)) & 0xffffu));
                    pair |= f2bf(bf2f((rw[k] >> (16 * h)) & 0xffffu) + n) << (16 * h);
                }
                o8[k] = pair;
            }
            st.x0 = make_uint4(o8[0], o8[1], o8[2], o8[3]);
            st.x1 = make_uint4(o8[4], o8[5], o8[6], o8[7]);
            *reinterpret_cast<uint4*>(r1s + t * 16) = st.x0;
            *reinterpret_cast<uint4*>(r1s + t * 16 + 8) = st.x1;
        }
    }
    // the FFN's pre-norm of r1 (as ffn_fused_kernel's of the residual row), the block's claim and
    // the copy of the normalised row kept for take-overs
    rms_finish_bf16<kFfnWaves>(st, sh, red);
    uint32_t claim_old = 0;
    if (ctl && lane == 0)
        claim_old = __hip_atomic_exchange(reinterpret_cast<uint32_t*>(&slots->claim[blockIdx.x]), tag,
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (t < kH / 8) reinterpret_cast<uint4*>(sx)[t] = reinterpret_cast<const uint4*>(sh)[t];

    // up/gate (as up_gate_rows): stage g reads L-rows lbase + 8 g; stage g + NR goes out once stage
    // g's registers are consumed
    uint32_t xv[KI][EPC / 2];
#pragma unroll
    for (int j = 0; j < KI; ++j) {
        const int e0 = j * 64 * EPC + lane * EPC;
        if (e0 < kH) lds_pairs<EPC>(sh, e0, xv[j]);
        else {
#pragma unroll
            for (int i = 0; i < EPC / 2; ++i) xv[j][i] = 0u;
        }
    }
    float pv = 0.0f;
#pragma unroll
    for (int g = 0; g < RL; ++g) {
        Chunk<F> (&src)[2][KI] = ring[g % NR];
        float du = 0.0f, dg = 0.0f;
#pragma unroll
        for (int j = 0; j < KI; ++j) {
            du = chunk_dot2<F>(xv[j], src[0][j], du);
            dg = chunk_dot2<F>(xv[j], src[1][j], dg);
        }
        if (g + NR < RL) issue(g + NR, ring[g % NR]);
        du = wave_sum(du);
        dg = wave_sum(dg);
        const float up = proj_commit<F>(du, __shfl(su, g, kWave));
        const float gate = proj_commit<F>(dg, __shfl(sg, g, kWave));
        if (lane == g) pv = rbf(gelu_tanh(gate)) * up;  // gemma4.py:197
    }

    // the FFN's residual values from r1: a leader's rows with the post-norm, the workgroup's own
    // rows without it
    uint4 r8 = make_uint4(0, 0, 0, 0);
    uint32_t r1 = 0;
    if (ctl) {
        if (post && leader) r8 = *reinterpret_cast<const uint4*>(r1s + post_leader_row(lane));
        else if (!post) r1 = r1s[blockIdx.x * kFfnWgRows + min(lane, kFfnWgRows - 1)];
    }
    ffn_down_post<F, SK>(p, s, pv, tag, claim_old, res, drow0, dscale, r8, w8, r1, ls_bits, ptag, slots, err, stall);
}

// ========================================================== raw projection
// out[m, n] = bf16((x[m] . W[n]) * s[n]) for arbitrary N and K % 16 == 0. One row per wave,
// activations straight from global memory. Used for the raw-projection known answers.
template <ScaleKind SK>
__global__ __launch_bounds__(kBlock) void proj_decode_kernel(ProjParams p) {
    const int m = blockIdx.y;
    const int lane = lane_id();
    const int n = blockIdx.x * 4 + wave_id();
    if (n >= p.N) return;
    const uint16_t* x = p.x + (size_t)m * p.K;
    const uint8_t* w = p.w + (size_t)n * p.K;
    float acc = 0.0f;
    for (int c = lane * 16; c < p.K; c += 1024) {
        float h[16];
        bf16x8_to_f32(ld16(x + c), h);
        bf16x8_to_f32(ld16(x + c + 8), h + 8);
        acc = dot_fp8_16(h, ld_stream(w + c), acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) p.out[(size_t)m * p.N + n] = (uint16_t)f2bf(acc * load_scale<SK>(p.s, n));
}

// ================================================================ self-test
// Decodes every FP8 code, every FP4 byte (two nibbles, scale 1), every E8M0 code, and GeLU of
// every bf16 value, with the same device helpers the kernels use.
//   out[0,256)        f32 bits of E4M3 code i
//   out[256,768)      f32 bits of the two E2M1 nibbles of byte i (low nibble first)
//   out[768,1024)     f32 bits of E8M0 code i
//   out[1024,66560)   bf16 bits of bf16(gelu_tanh(bf16 value i))
//   out[66560,66564)  f32 bits of the first E2M1 value of byte 0x77 (6.0) converted with the
//                     f32 scale 15, 2, 3, 0.75 -- records how the hardware applies the scale
//   out[66564,132100) bf16 bits of the final-logit softcap of bf16 value i
__global__ void format_selftest_kernel(uint32_t* out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < 4) {
        const float scales[4] = {15.0f, 2.0f, 3.0f, 0.75f};
        float w[8];
        fp4x8_to_f32(0x77u, scales[i], w);
        out[66560 + i] = __float_as_uint(w[0]);
    }
    if (i < 256) {
        float v[4];
        fp8x4_to_f32((uint32_t)i, v);
        out[i] = __float_as_uint(v[0]);
        float w[8];
        fp4x8_to_f32((uint32_t)i, 1.0f, w);
        out[256 + 2 * i] = __float_as_uint(w[0]);
        out[256 + 2 * i + 1] = __float_as_uint(w[1]);
        out[768 + i] = __float_as_uint(e8m0_to_f32((uint32_t)i));
    }
    if (i < 65536) {
        out[1024 + i] = f2bf(gelu_tanh(bf2f((uint32_t)i)));
        out[66564 + i] = softcap30_bf16(bf2f((uint32_t)i));
        // f32 -> bf16 rounding: every bf16 high half with eight low halves (zero, one, below, at and
        // above the tie, ...), then one packed pair per high half
        const uint32_t lows[8] = {0x0000u, 0x0001u, 0x7fffu, 0x8000u, 0x8001u, 0x4000u, 0xc000u, 0xffffu};
        const uint32_t hi = (uint32_t)i << 16;
#pragma unroll
        for (int j = 0; j < 8; ++j) out[132100 + 8 * i + j] = f2bf(__uint_as_float(hi | lows[j]));
        out[656388 + i] = pk_bf16(__uint_as_float(hi | 0x8000u), __uint_as_float(hi | 0x7fffu));
    }
}

template <typename K, typename... A>
hipError_t launch(K kernel, dim3 grid, hipStream_t s, A... args) {
    hipLaunchKernelGGL(kernel, grid, dim3(kBlock), 0, s, args...);
    return hipGetLastError();
}

}  // namespace

template <typename K>
static bool fits_resident(int8_t& known, K kernel, int block, int grid, const DevCtx* ctx);

// The waits' take-over threshold (and, in tests, held workgroups) passed to every single-launch
// kernel. A test may change it from any thread while another launches: the mutex makes each
// launch copy one whole Stall.
static Stall g_stall = {kStealTicks, 0, {-1, -1, -1, -1}};
static std::mutex g_stall_mutex;

void set_stall(const Stall& st) {
    std::lock_guard<std::mutex> lock(g_stall_mutex);
    g_stall = st;
}

static Stall current_stall() {
    std::lock_guard<std::mutex> lock(g_stall_mutex);
    return g_stall;
}

// A single-launch kernel, or its Hold instantiation while a test holds workgroups.
template <typename K, typename KH, typename... A>
static hipError_t launch_fused(K kernel, KH kernel_hold, dim3 grid, int block, hipStream_t s, A... args) {
    const Stall st = current_stall();
    if (st.hold_ticks) hipLaunchKernelGGL(kernel_hold, grid, dim3(block), 0, s, args..., st);
    else hipLaunchKernelGGL(kernel, grid, dim3(block), 0, s, args..., st);
    return hipGetLastError();
}

hipError_t launch_qkv_decode(const QkvParams& p, int M, hipStream_t s, DevCtx* ctx) {
    for (int m0 = 0; m0 < M; m0 += kMaxDecodeM) {
        const int mm = M - m0 < kMaxDecodeM ? M - m0 : kMaxDecodeM;
        if (mm == 1) {
            const bool f32 = p.scale_kind == ScaleKind::F32;
            if (f32 && fits_resident(ctx->qkv_fused[0], qkv_fused_kernel<ScaleKind::F32>, kQkvBlock, kQkvGrid, ctx)) {
                const hipError_t e = launch_fused(qkv_fused_kernel<ScaleKind::F32>, qkv_fused_kernel<ScaleKind::F32, true>,
                                                  dim3(kQkvGrid), kQkvBlock, s, p, m0, ctx->qkv_part, ctx->tickets, ctx->err);
                if (e != hipSuccess) return e;
                continue;
            }
            if (!f32 && fits_resident(ctx->qkv_fused[1], qkv_fused_kernel<ScaleKind::BF16>, kQkvBlock, kQkvGrid, ctx)) {
                const hipError_t e = launch_fused(qkv_fused_kernel<ScaleKind::BF16>, qkv_fused_kernel<ScaleKind::BF16, true>,
                                                  dim3(kQkvGrid), kQkvBlock, s, p, m0, ctx->qkv_part, ctx->tickets, ctx->err);
                if (e != hipSuccess) return e;
                continue;
            }
        }
        if (mm >= kRowsProjMinM) {  // the matrix-core rows path reads the weights once for all rows
            const hipError_t e = launch_qkv_rows(p, m0, mm, s, ctx);
            if (e != hipSuccess) return e;
            continue;
        }
        const dim3 grid(kQkvRows / (4 * kQkvR), mm);
        hipError_t e = p.scale_kind == ScaleKind::F32
            ? launch(qkv_decode_kernel<ScaleKind::F32, false>, grid, s, p, m0, ctx->raw_qkv, ctx->tickets, ctx->err)
            : launch(qkv_decode_kernel<ScaleKind::BF16, false>, grid, s, p, m0, ctx->raw_qkv, ctx->tickets, ctx->err);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_full_qkv(const QkvParams& p, int M, hipStream_t s, DevCtx* ctx) {
    static_assert(kFqkvRows <= kL, "raw full-layer projections fit a pbuf row");
    for (int m0 = 0; m0 < M; m0 += kMaxDecodeM) {
        const int mm = M - m0 < kMaxDecodeM ? M - m0 : kMaxDecodeM;
        if (mm >= kRowsProjMinM) {  // the matrix-core rows path
            const hipError_t e = launch_full_qkv_rows(p, m0, mm, s, ctx);
            if (e != hipSuccess) return e;
            continue;
        }
        const dim3 grid(kFqkvRows / (4 * kQkvR), mm);
        // raw projections in pbuf, rows kFqkvRows apart (pbuf holds kMaxChunkM x kL >= 16 x 8704)
        hipError_t e = p.scale_kind == ScaleKind::F32
            ? launch(qkv_decode_kernel<ScaleKind::F32, true>, grid, s, p, m0, ctx->pbuf, ctx->tickets, ctx->err)
            : launch(qkv_decode_kernel<ScaleKind::BF16, true>, grid, s, p, m0, ctx->pbuf, ctx->tickets, ctx->err);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Whether a single-launch kernel's grid of `grid` workgroups fits on the device at once.
template <typename K>
static bool fits_resident(int8_t& known, K kernel, int block, int grid, const DevCtx* ctx) {
    if (known < 0) {
        int per_cu = 0;
        const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, 0);
        known = (e == hipSuccess && per_cu * ctx->cus >= grid) ? 1 : 0;
    }
    return known == 1;
}

template <int KX>
static hipError_t o_decode_impl(const OParams& p, int M, hipStream_t s, DevCtx* ctx, int8_t* fused_known) {
    for (int m0 = 0; m0 < M; m0 += kMaxDecodeM) {
        const int mm = M - m0 < kMaxDecodeM ? M - m0 : kMaxDecodeM;
        if (mm == 1) {
            const bool f32 = p.scale_kind == ScaleKind::F32;
            PostSlots* slots = reinterpret_cast<PostSlots*>(ctx->o_part);
            if (f32 && fits_resident(fused_known[0], o_fused_kernel<ScaleKind::F32, KX>, kOBlock, kPostGrid, ctx)) {
                const hipError_t e = launch_fused(o_fused_kernel<ScaleKind::F32, KX>, o_fused_kernel<ScaleKind::F32, KX, true>,
                                                  dim3(kPostGrid), kOBlock, s, p, m0, slots, ctx->tickets, ctx->err);
                if (e != hipSuccess) return e;
                continue;
            }
            if (!f32 && fits_resident(fused_known[1], o_fused_kernel<ScaleKind::BF16, KX>, kOBlock, kPostGrid, ctx)) {
                const hipError_t e = launch_fused(o_fused_kernel<ScaleKind::BF16, KX>, o_fused_kernel<ScaleKind::BF16, KX, true>,
                                                  dim3(kPostGrid), kOBlock, s, p, m0, slots, ctx->tickets, ctx->err);
                if (e != hipSuccess) return e;
                continue;
            }
        }
        // the matrix-core rows path (full-attention O, K = 8192: from two rows on)
        if (mm >= (KX == kQf ? 2 : kRowsProjMinM)) {
            const hipError_t e = launch_o_rows(p, m0, mm, s, ctx);
            if (e != hipSuccess) return e;
            continue;
        }
        const dim3 grid(kH / (4 * kOR), mm);
        hipError_t e = p.scale_kind == ScaleKind::F32
            ? launch(o_decode_kernel<ScaleKind::F32, KX>, grid, s, p, m0, ctx->pbuf, ctx->tickets)
            : launch(o_decode_kernel<ScaleKind::BF16, KX>, grid, s, p, m0, ctx->pbuf, ctx->tickets);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_o_decode(const OParams& p, int M, hipStream_t s, DevCtx* ctx) {
    return o_decode_impl<kQs>(p, M, s, ctx, ctx->o_fused);
}

hipError_t launch_full_o(const OParams& p, int M, hipStream_t s, DevCtx* ctx) {
    return o_decode_impl<kQf>(p, M, s, ctx, ctx->full_o_fused);
}

// Whether the single-launch FFN's grid fits on the device at once (checked once per device).
template <FfnFormat F, ScaleKind SK>
static bool ffn_fused_fits(DevCtx* ctx) {
    int8_t& known = ctx->ffn_fused[(int)F * 2 + (int)SK];
    if (known < 0) {
        int per_cu = 0;
        const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, ffn_fused_kernel<F, SK>, kFfnBlock, 0);
        known = (e == hipSuccess && per_cu * ctx->cus >= kFfnGrid) ? 1 : 0;
    }
    return known == 1;
}

template <FfnFormat F, ScaleKind SK>
static hipError_t ffn_decode_impl(const FfnParams& p, int M, hipStream_t s, DevCtx* ctx) {
    for (int m0 = 0; m0 < M; m0 += kMaxDecodeM) {
        const int mm = M - m0 < kMaxDecodeM ? M - m0 : kMaxDecodeM;
        hipError_t e;
        if (mm == 1 && ffn_fused_fits<F, SK>(ctx)) {
            e = launch_fused(ffn_fused_kernel<F, SK>, ffn_fused_kernel<F, SK, true>, dim3(kFfnGrid), kFfnBlock, s, p, m0,
                             ctx->ffn_ptag, reinterpret_cast<PostSlots*>(ctx->ffn_part), ctx->tickets, ctx->err);
            if (e != hipSuccess) return e;
            continue;
        }
        // 2..16 rows (or one row whose single-launch grid does not fit): the matrix-core path,
        // which reads each weight once for all rows
        e = launch_ffn_rows(p, m0, mm, s, ctx);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_ffn_decode(const FfnParams& p, int M, hipStream_t s, DevCtx* ctx) {
    switch (p.fmt) {
        case FfnFormat::FP8:
            return p.scale_kind == ScaleKind::F32 ? ffn_decode_impl<FfnFormat::FP8, ScaleKind::F32>(p, M, s, ctx)
                                                  : ffn_decode_impl<FfnFormat::FP8, ScaleKind::BF16>(p, M, s, ctx);
        case FfnFormat::NVFP4: return ffn_decode_impl<FfnFormat::NVFP4, ScaleKind::F32>(p, M, s, ctx);
        case FfnFormat::MXFP4: return ffn_decode_impl<FfnFormat::MXFP4, ScaleKind::F32>(p, M, s, ctx);
    }
    return hipErrorInvalidValue;
}

template <FfnFormat F, ScaleKind SKO, ScaleKind SK>
static bool o_ffn_fused(const OParams& o, const FfnParams& p, hipStream_t s, DevCtx* ctx, hipError_t* e) {
    if (!fits_resident(ctx->o_ffn_fused[(int)F], o_ffn_fused_kernel<F, SKO, SK>, kFfnBlock, kFfnGrid, ctx)) return false;
    *e = launch_fused(o_ffn_fused_kernel<F, SKO, SK>, o_ffn_fused_kernel<F, SKO, SK, true>, dim3(kFfnGrid), kFfnBlock, s,
                      o, p, 0, reinterpret_cast<PostSlots*>(ctx->ofn_part), ctx->ffn_ptag,
                      reinterpret_cast<PostSlots*>(ctx->ffn_part), ctx->tickets, ctx->err);
    return true;
}

bool launch_o_ffn_fused(const OParams& o, const FfnParams& p, hipStream_t s, DevCtx* ctx, hipError_t* e) {
    const bool of32 = o.scale_kind == ScaleKind::F32;
    switch (p.fmt) {
        case FfnFormat::FP8:
            return of32 && p.scale_kind == ScaleKind::F32 &&
                   o_ffn_fused<FfnFormat::FP8, ScaleKind::F32, ScaleKind::F32>(o, p, s, ctx, e);
        case FfnFormat::NVFP4:
            return !of32 && o_ffn_fused<FfnFormat::NVFP4, ScaleKind::BF16, ScaleKind::F32>(o, p, s, ctx, e);
        case FfnFormat::MXFP4:
            return of32 && o_ffn_fused<FfnFormat::MXFP4, ScaleKind::F32, ScaleKind::F32>(o, p, s, ctx, e);
    }
    return false;
}

hipError_t launch_proj_decode(const ProjParams& p, int M, hipStream_t s) {
    const dim3 grid((p.N + 3) / 4, M);
    return p.scale_kind == ScaleKind::F32 ? launch(proj_decode_kernel<ScaleKind::F32>, grid, s, p)
                                          : launch(proj_decode_kernel<ScaleKind::BF16>, grid, s, p);
}

hipError_t launch_format_selftest(uint32_t* out, hipStream_t s) {
    return launch(format_selftest_kernel, dim3(65536 / kBlock), s, out);
}

}  // namespace moa
