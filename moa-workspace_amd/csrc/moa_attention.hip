// moa_attention.hip -- ops::sliding_attention (FO/src/ops.rs:118-128): decode attention of one token
// row over the sliding layer's ring cache.
//
// For KV head n and its query heads g = 0, 1 (FO/src/axes.rs: Ns = 8, Gs = 2, Ds = 256, Ts = 1024):
//   s_t = q_g . k_t (scale 1.0), over the slots t whose mask value is non-zero;
//   out_g = sum_t softmax(s)_t v_t, rounded once to bf16.
// This is the CPU reference (FO/scripts/reference/gemma4.py:163-186: scaled_dot_product_attention
// with scale=1.0 over the window's positions). The runtime builds the mask rows as 1.0 for slots
// <= pos and 0.0 beyond (FO/src/host/runtime.rs:160, 409). The RNGD kernel
// (FO/src/device/sliding/attention.rs) applies the mask as min(exp, mask) after a max taken over
// every slot, and adds 1e-6 to the sum. With 0/1 masks that is the same softmax up to rounding,
// unless masked slots hold scores far above the valid ones. Here the max is taken over the valid
// slots only. A row with no valid slot returns zeros.
//
// Split over slots ("flash decoding"): workgroup (n, c, m) takes the 32 slots 32 c .. 32 c + 31
// of head n for token row m. It computes its partial (max, sum of exp, sum of exp * v) for both
// query heads and publishes it with agent-scope stores. Then it adds one to the head's ticket
// counter; the workgroup that completes the head's 32 (the counter's old value is 31 mod 32)
// combines the partials. Nothing waits on another workgroup, so residency is not required.
// The head is the grid's x index: workgroups go to the 8 XCDs round-robin by linear index, so all
// 32 of head n run on XCD n and its ticket and partials never cross XCDs (7.10 -> 6.96 us per
// call against the chunk as x index; the results do not depend on the placement).
#include <hip/hip_runtime.h>

#include "moa_device.h"
#include "moa_internal.h"

namespace moa {
namespace {

constexpr int kAtBlock = 256;
constexpr int kAtSlots = 32;                     // slots per workgroup
constexpr int kAtChunks = kTs / kAtSlots;        // 32 workgroups per head
constexpr int kAtPartFloats = 4 + kDs;           // max, sum, 2 unused, o[256] (16-byte aligned)
static_assert(kAtChunks == 32, "ticket arithmetic assumes 32 chunks per head");

__device__ __forceinline__ float sc1_load(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void sc1_store(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// part: [M][kNs][kAtChunks][kGs][kAtPartFloats]; tickets: one counter per (row, head).
__global__ __launch_bounds__(kAtBlock) void attn_split_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
                                                              const uint16_t* __restrict__ vc, const float* __restrict__ mask,
                                                              uint16_t* __restrict__ out, float* part, uint32_t* tickets) {
    __shared__ float qs[kGs][kDs];
    __shared__ float sc[kGs][kAtSlots];       // scores, then exp weights
    __shared__ float stat[kGs][2];            // max, sum
    __shared__ float ored[8][kGs][kDs];       // per slot group partial o
    __shared__ uint32_t s_last;
    const int t = threadIdx.x;
    const int n = blockIdx.x, c = blockIdx.y, m = blockIdx.z;
    const int t0 = c * kAtSlots;
    const uint16_t* qrow = q + ((size_t)m * kNs + n) * kGs * kDs;
    // The chunk's K and V rows and its mask values are requested first (none depends on q); q
    // of both query heads (512 bf16 values, two per thread) goes to LDS meanwhile.
    const int sg = t / 32, dg = t % 32;  // PV layout: slots sg, sg + 8, ..; dims 8 dg .. 8 dg + 7
    const int s = t / 8, pt = t % 8;     // score layout: slot s, dims 32 pt .. 32 pt + 31
    const uint16_t* kr = kc + ((size_t)(t0 + s) * kNs + n) * kDs + 32 * pt;
    uint4 kq[4], vq[kAtSlots / 8];
#pragma unroll
    for (int i = 0; i < 4; ++i) kq[i] = ld16(kr + 8 * i);
#pragma unroll
    for (int i = 0; i < kAtSlots / 8; ++i) vq[i] = ld16(vc + ((size_t)(t0 + sg + 8 * i) * kNs + n) * kDs + 8 * dg);
    const bool valid = mask[(size_t)m * kTs + t0 + s] != 0.0f;
    const uint32_t q2 = reinterpret_cast<const uint32_t*>(qrow)[t];
    qs[t / 128][2 * (t % 128)] = bf2f(q2 & 0xffffu);
    qs[t / 128][2 * (t % 128) + 1] = bf2f(q2 >> 16);
    __syncthreads();

    // scores: thread (s, pt) dots 32 dims of slot t0 + s with both query heads
    {
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float kv[8];
            bf16x8_to_f32(kq[i], kv);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                a0 = fmaf(qs[0][32 * pt + 8 * i + e], kv[e], a0);
                a1 = fmaf(qs[1][32 * pt + 8 * i + e], kv[e], a1);
            }
        }
#pragma unroll
        for (int o = 4; o >= 1; o >>= 1) {
            a0 += __shfl_xor(a0, o);
            a1 += __shfl_xor(a1, o);
        }
        if (pt == 0) {
            sc[0][s] = valid ? a0 : -INFINITY;
            sc[1][s] = valid ? a1 : -INFINITY;
        }
    }
    __syncthreads();
    // softmax statistics of the chunk: wave 0 (lanes 0-31: head 0, 32-63: head 1)
    if (t < 64) {
        const int g = t / 32, s = t % 32;
        const float v = sc[g][s];
        float mx = v;
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        const float e = v == -INFINITY ? 0.0f : __expf(v - mx);
        float sum = e;
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) sum += __shfl_xor(sum, o);
        sc[g][s] = e;
        if (s == 0) {
            stat[g][0] = mx;
            stat[g][1] = sum;
        }
    }
    __syncthreads();
    // o = sum_s e_s v_s: thread (sg, dg) takes 8 dims of slots sg, sg + 8, ...
    {
        float o0[8], o1[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o0[e] = o1[e] = 0.0f;
#pragma unroll
        for (int i = 0; i < kAtSlots / 8; ++i) {
            const int s = sg + 8 * i;
            float vv[8];
            bf16x8_to_f32(vq[i], vv);
            const float w0 = sc[0][s], w1 = sc[1][s];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                o0[e] = fmaf(w0, vv[e], o0[e]);
                o1[e] = fmaf(w1, vv[e], o1[e]);
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            ored[sg][0][8 * dg + e] = o0[e];
            ored[sg][1][8 * dg + e] = o1[e];
        }
    }
    __syncthreads();
    float* mypart = part + (((size_t)m * kNs + n) * kAtChunks + c) * kGs * kAtPartFloats;
#pragma unroll
    for (int g = 0; g < kGs; ++g) {
        float o = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) o += ored[k][g][t];
        sc1_store(mypart + g * kAtPartFloats + 4 + t, o);
        if (t < 2) sc1_store(mypart + g * kAtPartFloats + t, stat[g][t]);
    }
    // publish, then count the head's chunks; the workgroup completing the 32 combines them
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (t == 0) {
        const uint32_t old = __hip_atomic_fetch_add(tickets + ((size_t)m * kNs + n) * kTicketStride, 1u,
                                                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (old % kAtChunks) == kAtChunks - 1;
    }
    __syncthreads();
    if (!s_last) return;

    // combine. Threads 0-63 read the 32 chunks' max and sum of both heads and turn them into the
    // factors exp(max_c - max) and the head's sum. Every thread reads dims 4 q .. 4 q + 3
    // (q = t % 64) of chunks 8 (t / 64) .. + 7 for both heads as 16-byte loads, all issued before
    // any is used; the four chunk groups then meet in LDS in a fixed order. Partials are read
    // coherently (agent scope: 16-byte buffer loads with sc1, and per-thread one-float atomic loads).
    __shared__ float sf[kGs][kAtChunks], sl[kGs];
    __shared__ float4 so[4][kGs][kDs / 4];
    const float* hp = part + ((size_t)m * kNs + n) * kAtChunks * kGs * kAtPartFloats;
    const int q4 = t & 63, cg = t >> 6;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(hp), 0, (uint32_t)(kAtChunks * kGs * kAtPartFloats * sizeof(float)), 0x00020000);
    float mcv = 0.0f, lcv = 0.0f;
    if (t < 64) {  // first: the factors are computed while the outputs' loads are in flight
        mcv = sc1_load(hp + ((t & 31) * kGs + (t >> 5)) * kAtPartFloats);
        lcv = sc1_load(hp + ((t & 31) * kGs + (t >> 5)) * kAtPartFloats + 1);
    }
    float4 oc[kGs][8];
#pragma unroll
    for (int g = 0; g < kGs; ++g)
#pragma unroll
        for (int i = 0; i < 8; ++i)
            oc[g][i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      rs, (((cg * 8 + i) * kGs + g) * kAtPartFloats + 4 + 4 * q4) * 4,
                                                      0, 16 /* sc1 */));
    if (t < 64) {
        const int g = t >> 5, cc = t & 31;
        float mx = mcv;
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        const float f = mcv == -INFINITY ? 0.0f : __expf(mcv - mx);
        float l = f * lcv;
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) l += __shfl_xor(l, o);
        sf[g][cc] = f;
        if (cc == 0) sl[g] = l;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < kGs; ++g) {
        float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float f = sf[g][cg * 8 + i];
            a.x = fmaf(f, oc[g][i].x, a.x);
            a.y = fmaf(f, oc[g][i].y, a.y);
            a.z = fmaf(f, oc[g][i].z, a.z);
            a.w = fmaf(f, oc[g][i].w, a.w);
        }
        so[cg][g][q4] = a;
    }
    __syncthreads();
    if (t < kGs * 64) {
        const int g = t >> 6, q = t & 63;
        const float l = sl[g];
        const float4 a = so[0][g][q], b = so[1][g][q], c2 = so[2][g][q], d = so[3][g][q];
        float v[4] = {((a.x + b.x) + c2.x) + d.x, ((a.y + b.y) + c2.y) + d.y, ((a.z + b.z) + c2.z) + d.z,
                      ((a.w + b.w) + c2.w) + d.w};
        uint32_t h[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = f2bf(l > 0.0f ? v[e] / l : 0.0f);
        *reinterpret_cast<uint2*>(out + (((size_t)m * kNs + n) * kGs + g) * kDs + 4 * q) =
            make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
    }
}

}  // namespace

hipError_t launch_sliding_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, const float* mask,
                                    uint16_t* out, int M, hipStream_t s, DevCtx* ctx) {
    for (int m0 = 0; m0 < M; m0 += kMaxDecodeM) {
        const int mm = M - m0 < kMaxDecodeM ? M - m0 : kMaxDecodeM;
        hipLaunchKernelGGL(attn_split_kernel, dim3(kNs, kAtChunks, mm), dim3(kAtBlock), 0, s,
                           q + (size_t)m0 * kQs, k_cache, v_cache, mask + (size_t)m0 * kTs, out + (size_t)m0 * kQs,
                           ctx->attn_part, ctx->tickets + kTicketAttn * kTicketStride);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace moa
