// moa_api.hip -- the C ABI (include/moa_ops.h): argument validation, per-device scratch,
// and dispatch to the decode (small M) or chunk (large M) kernels.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/moa_ops.h"
#include "moa_internal.h"
#include "moa_sync.h"

namespace moa {
namespace {

thread_local std::string g_error;
std::mutex g_ctx_mutex;
constexpr int kMaxDevices = 64;
DevCtx g_ctx[kMaxDevices];

int fail(int code, const std::string& msg) {
    g_error = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(MOA_ERROR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace

int set_error(int code, const char* msg) { return fail(code, msg); }

// Per device: a one-token call's bounded cross-workgroup wait expired (MOA_DEVERR_SPIN_TIMEOUT,
// seen by moa_device_errors), so that call's outputs may be partly written. Until the caller
// acknowledges it with moa_clear_device_state, every call that computes on that device and
// moa_init refuse with MOA_ERROR_DEVICE_STATE instead of building on those outputs.
namespace {
std::atomic<uint32_t> g_tripped[kMaxDevices];

// The current device's index for the tripped check; 0 when there is none (a failing HIP call
// then reports the device problem itself).
int current_device_or_0() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) dev = 0;
    return dev;
}

int tripped_fail(int dev) {
    return fail(MOA_ERROR_DEVICE_STATE,
                "device " + std::to_string(dev) + ": a one-token call's cross-workgroup wait expired "
                "(MOA_DEVERR_SPIN_TIMEOUT), so its outputs may be partly written; restore them, then call "
                "moa_clear_device_state(" + std::to_string(dev) + ")");
}
}  // namespace

DevCtx* existing_context(int dev) {
    std::lock_guard<std::mutex> lock(g_ctx_mutex);
    return g_ctx[dev].base ? &g_ctx[dev] : nullptr;
}

DevCtx* device_context(hipError_t* err) {
    int dev = 0;
    *err = hipGetDevice(&dev);
    if (*err != hipSuccess) return nullptr;
    if (dev < 0 || dev >= kMaxDevices) {
        *err = hipErrorInvalidDevice;
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_ctx_mutex);
    DevCtx& c = g_ctx[dev];
    if (c.base) return &c;
    size_t off = 0;
    auto carve = [&](size_t bytes) { size_t at = off; off = align_up(off + bytes, 256); return at; };
    const size_t t_tickets = carve(sizeof(uint32_t) * kTicketCount * kTicketStride);
    const size_t t_err = carve(sizeof(uint32_t) * 4);
    const size_t t_raw = carve(sizeof(uint16_t) * (size_t)kMaxChunkM * (kQs + 2 * kPs));
    const size_t t_p = carve(sizeof(uint16_t) * (size_t)kMaxChunkM * kL);
    const size_t t_h = carve(sizeof(uint16_t) * (size_t)kMaxChunkM * kH);
    const size_t t_f = carve(sizeof(float) * kChunkPartFloats);
    const size_t t_part = carve(sizeof(uint64_t) * kFfnSlotWords);
    const size_t t_opart = carve(sizeof(uint64_t) * kFfnSlotWords);
    const size_t t_ofnpart = carve(sizeof(uint64_t) * kFfnSlotWords * kOfnCopies);
    const size_t t_qpart = carve(sizeof(uint64_t) * kQkvSlotWords);
    const size_t t_ptag = carve(sizeof(uint64_t) * (kL / 2));
    const size_t t_rflag = carve(sizeof(uint64_t) * kRowsFlagWords);
    const size_t t_attn = carve(sizeof(float) * kAttnPartFloats);
    const size_t t_fattn = carve(sizeof(float) * kFattnPartFloats);
    int cus = 0;
    *err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (*err != hipSuccess) return nullptr;
    void* base = nullptr;
    *err = hipMalloc(&base, off);
    if (*err != hipSuccess) return nullptr;
    *err = hipMemset(base, 0, off);
    if (*err == hipSuccess) *err = hipDeviceSynchronize();
    if (*err != hipSuccess) {
        (void)hipFree(base);
        return nullptr;
    }
    char* b = static_cast<char*>(base);
    c.device = dev;
    c.cus = cus;
    c.tickets = reinterpret_cast<uint32_t*>(b + t_tickets);
    c.err = reinterpret_cast<uint32_t*>(b + t_err);
    c.raw_qkv = reinterpret_cast<uint16_t*>(b + t_raw);
    c.pbuf = reinterpret_cast<uint16_t*>(b + t_p);
    c.hbuf = reinterpret_cast<uint16_t*>(b + t_h);
    c.fbuf = reinterpret_cast<float*>(b + t_f);
    c.ffn_part = reinterpret_cast<uint64_t*>(b + t_part);
    c.o_part = reinterpret_cast<uint64_t*>(b + t_opart);
    c.ofn_part = reinterpret_cast<uint64_t*>(b + t_ofnpart);
    c.qkv_part = reinterpret_cast<uint64_t*>(b + t_qpart);
    c.ffn_ptag = reinterpret_cast<uint64_t*>(b + t_ptag);
    c.rows_flag = reinterpret_cast<uint64_t*>(b + t_rflag);
    c.attn_part = reinterpret_cast<float*>(b + t_attn);
    c.fattn_part = reinterpret_cast<float*>(b + t_fattn);
    c.base = base;
    return &c;
}

// ------------------------------------------------------------ the no-allocation entry point
// moa_decoder_feedforward_fp8_noalloc runs the same kernels as moa_decoder_feedforward_fp8 for
// 1..kMaxDecodeM rows, with every byte of scratch carved from `scratch` below instead of the
// hipMalloc'd per-device block: the epoch counters and hand-off words of the one-token kernel,
// and the normalised rows, GeGLU rows and down partial sums of the rows path. `scratch` is a
// static device array, so each GPU holds its own copy from the moment the code object loads
// (zero-filled, as static storage is) until the process ends. Its host-side name is not a device
// address: the set-up below asks HIP for the device address once per device and only that
// address ever reaches a kernel.
namespace {
constexpr size_t kNaTicketBytes = sizeof(uint32_t) * kTicketCount * kTicketStride;
constexpr size_t kNaErrBytes = 256;
constexpr size_t kNaPartBytes = sizeof(uint64_t) * kFfnSlotWords;
constexpr size_t kNaPtagBytes = sizeof(uint64_t) * (kL / 2);
constexpr size_t kNaHBytes = sizeof(uint16_t) * kMaxDecodeM * kH;
constexpr size_t kNaPBytes = sizeof(uint16_t) * kMaxDecodeM * kL;
constexpr size_t kNaFBytes = sizeof(float) * 4 * kMaxDecodeM * kH;  // 4 down splits of the rows path
constexpr size_t kNaRowsFlagBytes = sizeof(uint64_t) * kRowsFlagWords;
constexpr size_t na_up(size_t v) { return (v + 255) / 256 * 256; }
constexpr size_t kNaTicketOff = 0;
constexpr size_t kNaErrOff = kNaTicketOff + na_up(kNaTicketBytes);
constexpr size_t kNaPartOff = kNaErrOff + na_up(kNaErrBytes);
constexpr size_t kNaPtagOff = kNaPartOff + na_up(kNaPartBytes);
constexpr size_t kNaHOff = kNaPtagOff + na_up(kNaPtagBytes);
constexpr size_t kNaPOff = kNaHOff + na_up(kNaHBytes);
constexpr size_t kNaFOff = kNaPOff + na_up(kNaPBytes);
constexpr size_t kNaRowsFlagOff = kNaFOff + na_up(kNaFBytes);
constexpr size_t kNaBytes = kNaRowsFlagOff + na_up(kNaRowsFlagBytes);  // 1.93 MB
static_assert(kNaBytes < (2u << 20), "the no-allocation scratch stays under 2 MiB");

static __device__ __align__(256) unsigned char scratch[kNaBytes];

std::mutex g_na_mutex;
DevCtx g_na_ctx[kMaxDevices];  // per device: pointers into that device's copy of `scratch`

// Once per device, with that device current: the device address of its `scratch`, carved into a
// context of the layout above. Allocates nothing. nullptr (and *code set) on failure.
DevCtx* noalloc_context(int* code) {
    if (g_tripped[current_device_or_0()].load()) { *code = tripped_fail(current_device_or_0()); return nullptr; }
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) { *code = hip_fail(e, "hipGetDevice"); return nullptr; }
    if (dev < 0 || dev >= kMaxDevices) { *code = fail(MOA_ERROR_NO_DEVICE, "device index out of range"); return nullptr; }
    std::lock_guard<std::mutex> lock(g_na_mutex);
    DevCtx& c = g_na_ctx[dev];
    if (c.base) return &c;
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
        *code = hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
        return nullptr;
    }
    int cus = 0;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) { *code = hip_fail(e, "hipDeviceGetAttribute"); return nullptr; }
    char* b = static_cast<char*>(ptr);
    c.device = dev;
    c.cus = cus;
    c.tickets = reinterpret_cast<uint32_t*>(b + kNaTicketOff);
    c.err = reinterpret_cast<uint32_t*>(b + kNaErrOff);
    c.ffn_part = reinterpret_cast<uint64_t*>(b + kNaPartOff);
    c.ffn_ptag = reinterpret_cast<uint64_t*>(b + kNaPtagOff);
    c.hbuf = reinterpret_cast<uint16_t*>(b + kNaHOff);
    c.pbuf = reinterpret_cast<uint16_t*>(b + kNaPOff);
    c.fbuf = reinterpret_cast<float*>(b + kNaFOff);
    c.rows_flag = reinterpret_cast<uint64_t*>(b + kNaRowsFlagOff);
    c.base = ptr;
    return &c;
}
}  // namespace

}  // namespace moa

using namespace moa;

namespace {

struct Check {
    int code = MOA_SUCCESS;
    // Required pointer with the given alignment.
    Check& ptr(const void* p, const char* name, size_t align = 16) {
        if (code) return *this;
        if (!p) { code = fail(MOA_ERROR_INVALID_VALUE, std::string(name) + " is NULL"); return *this; }
        if (reinterpret_cast<uintptr_t>(p) % align) {
            code = fail(MOA_ERROR_MISALIGNED, std::string(name) + " is not " + std::to_string(align) + "-byte aligned");
        }
        return *this;
    }
    // Optional pointer: NULL allowed.
    Check& opt(const void* p, const char* name, size_t align = 16) {
        if (code || !p) return *this;
        return ptr(p, name, align);
    }
    Check& rows(int M) {
        if (code) return *this;
        if (M < 1 || M > (1 << 20)) code = fail(MOA_ERROR_INVALID_VALUE, "M must be in [1, 2^20], got " + std::to_string(M));
        return *this;
    }
};

DevCtx* ctx_or_fail(int* code) {
    if (g_tripped[current_device_or_0()].load()) { *code = tripped_fail(current_device_or_0()); return nullptr; }
    hipError_t e;
    DevCtx* c = device_context(&e);
    if (!c) *code = hip_fail(e, "allocating the per-device scratch");
    return c;
}

int finish(hipError_t e, const char* what) {
    if (e != hipSuccess) return hip_fail(e, what);
    return MOA_SUCCESS;
}

int qkv_common(const QkvParams& p, int M, void* stream) {
    Check c;
    c.ptr(p.x, "x").ptr(p.qw, "q_weight").ptr(p.kw, "k_weight").ptr(p.vw, "v_weight");
    const size_t sa = p.scale_kind == ScaleKind::F32 ? 4 : 2;
    c.ptr(p.qs, "q_weight_scale", sa).ptr(p.ks, "k_weight_scale", sa).ptr(p.vs, "v_weight_scale", sa);
    c.ptr(p.in_rms, "input_rms_weight").ptr(p.q_rms, "q_rms_weight").ptr(p.k_rms, "k_rms_weight");
    c.ptr(p.kv_off, "kv_offset", 4).ptr(p.rope_off, "rope_offset", 4).ptr(p.cos, "cos").ptr(p.sin, "sin");
    c.ptr(p.k_cache, "k_cache").ptr(p.v_cache, "v_cache").ptr(p.q_out, "q_out").rows(M);
    if (c.code) return c.code;
    int code = MOA_SUCCESS;
    DevCtx* ctx = ctx_or_fail(&code);
    if (!ctx) return code;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (M <= kMaxDecodeM) return finish(launch_qkv_decode(p, M, s, ctx), "sliding_project_qkv launch");
    for (int m0 = 0; m0 < M; m0 += kMaxChunkM) {
        const int e = finish(launch_qkv_chunk(p, m0, M - m0 < kMaxChunkM ? M - m0 : kMaxChunkM, s, ctx),
                             "sliding_project_qkv launch");
        if (e) return e;
    }
    return MOA_SUCCESS;
}

int o_check(const OParams& p, int M) {
    Check c;
    c.ptr(p.x, "x").ptr(p.post_rms, "post_attn_rms_weight").ptr(p.ow, "o_weight");
    c.ptr(p.os, "o_weight_scale", p.scale_kind == ScaleKind::F32 ? 4 : 2).ptr(p.residual, "residual").rows(M);
    return c.code;
}

int o_launch(const OParams& p, int M, hipStream_t s, DevCtx* ctx) {
    if (M <= kMaxDecodeM) return finish(launch_o_decode(p, M, s, ctx), "sliding_attention_output launch");
    for (int m0 = 0; m0 < M; m0 += kMaxChunkM) {
        const int e = finish(launch_o_chunk(p, m0, M - m0 < kMaxChunkM ? M - m0 : kMaxChunkM, s, ctx),
                             "sliding_attention_output launch");
        if (e) return e;
    }
    return MOA_SUCCESS;
}

int o_common(const OParams& p, int M, void* stream) {
    if (const int bad = o_check(p, M)) return bad;
    int code = MOA_SUCCESS;
    DevCtx* ctx = ctx_or_fail(&code);
    if (!ctx) return code;
    return o_launch(p, M, static_cast<hipStream_t>(stream), ctx);
}

int ffn_check(const FfnParams& p, int M) {
    Check c;
    c.ptr(p.residual, "residual").ptr(p.pre_rms, "pre_ff_rms_weight");
    c.ptr(p.up, "up_weight").ptr(p.gate, "gate_weight").ptr(p.down, "down_weight");
    if (p.fmt == FfnFormat::FP8) {
        const size_t sa = p.scale_kind == ScaleKind::F32 ? 4 : 2;
        c.ptr(p.up_s, "up_weight_scale", sa).ptr(p.gate_s, "gate_weight_scale", sa).ptr(p.down_s, "down_weight_scale", sa);
    } else {
        const size_t sa = 4;  // FP4 block-scale codes: read a dword at a time
        c.ptr(p.up_s, "up_weight_scale", sa).ptr(p.gate_s, "gate_weight_scale", sa).ptr(p.down_s, "down_weight_scale", sa);
    }
    if (p.fmt == FfnFormat::NVFP4) {
        c.ptr(p.up_g, "up_global_scale", 4).ptr(p.gate_g, "gate_global_scale", 4).ptr(p.down_g, "down_global_scale", 4);
        c.ptr(p.post_rms, "post_ff_rms_weight").ptr(p.layer_scalar, "layer_scalar", 2);
    } else {
        c.opt(p.post_rms, "post_ff_rms_weight").opt(p.layer_scalar, "layer_scalar", 2);
    }
    c.rows(M);
    return c.code;
}

int ffn_launch(const FfnParams& p, int M, hipStream_t s, DevCtx* ctx) {
    // More than kMaxDecodeM rows take the MFMA path (every weight format).
    if (M <= kMaxDecodeM) return finish(launch_ffn_decode(p, M, s, ctx), "decoder_feedforward launch");
    for (int m0 = 0; m0 < M; m0 += kMaxChunkM) {
        const int e = finish(launch_ffn_chunk(p, m0, M - m0 < kMaxChunkM ? M - m0 : kMaxChunkM, s, ctx),
                             "decoder_feedforward launch");
        if (e) return e;
    }
    return MOA_SUCCESS;
}

int ffn_common(const FfnParams& p, int M, void* stream) {
    if (const int bad = ffn_check(p, M)) return bad;
    int code = MOA_SUCCESS;
    DevCtx* ctx = ctx_or_fail(&code);
    if (!ctx) return code;
    return ffn_launch(p, M, static_cast<hipStream_t>(stream), ctx);
}

// sliding_attention_output then decoder_feedforward on one residual: one launch for a token row
// when a single-launch kernel covers the operand types; from kRowsProjMinM rows on, O's last row
// kernel also writes the FFN's normalised input (one kernel fewer than the two operators); else
// (two rows) the two operators in turn.
int o_ffn_common(const OParams& o, const FfnParams& p, int M, void* stream) {
    if (const int bad = o_check(o, M)) return bad;
    if (const int bad = ffn_check(p, M)) return bad;
    int code = MOA_SUCCESS;
    DevCtx* ctx = ctx_or_fail(&code);
    if (!ctx) return code;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e = hipSuccess;
    if (M == 1 && launch_o_ffn_fused(o, p, s, ctx, &e))
        return finish(e, "sliding_attention_output_feedforward launch");
    if (M > kMaxDecodeM) {  // the MFMA path: O's post rows write the FFN's normalised input too
        for (int m0 = 0; m0 < M; m0 += kMaxChunkM) {
            const int bad = finish(launch_o_ffn_chunk(o, p, m0, M - m0 < kMaxChunkM ? M - m0 : kMaxChunkM, s, ctx),
                                   "sliding_attention_output_feedforward launch");
            if (bad) return bad;
        }
        return MOA_SUCCESS;
    }
    if (M >= kRowsProjMinM)  // the rows path: O's post rows write the FFN's normalised input too
        return finish(launch_o_ffn_rows(o, p, 0, M, s, ctx), "sliding_attention_output_feedforward launch");
    if (const int bad = o_launch(o, M, s, ctx)) return bad;
    return ffn_launch(p, M, s, ctx);
}

}  // namespace

extern "C" {

const char* moa_version(void) { return "moa-gfx950 0.1.0"; }

const char* moa_last_error_string(void) { return g_error.c_str(); }

int moa_init(int device) {
    if (device >= 0 && device < kMaxDevices && g_tripped[device].load()) return tripped_fail(device);
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) return fail(MOA_ERROR_NO_DEVICE, "no HIP device visible");
    if (device < 0 || device >= n) return fail(MOA_ERROR_INVALID_VALUE, "device index out of range");
    e = hipSetDevice(device);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    int code = MOA_SUCCESS;
    if (!ctx_or_fail(&code)) return code;
    return noalloc_context(&code) ? MOA_SUCCESS : code;
}

int moa_device_errors(void* stream, uint32_t* bits) {
    if (!bits) return fail(MOA_ERROR_INVALID_VALUE, "bits is NULL");
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(MOA_ERROR_NO_DEVICE, "device index out of range");
    hipStream_t s = static_cast<hipStream_t>(stream);
    // The error words of whichever scratch exists on this device: the hipMalloc'd one of the
    // other entry points and the static one of the no-allocation entry point. Neither is created
    // here, so a caller that cannot allocate reads its calls' errors without allocating.
    const DevCtx* ctxs[2] = {existing_context(dev), nullptr};
    {
        std::lock_guard<std::mutex> lock(g_na_mutex);
        if (g_na_ctx[dev].base) ctxs[1] = &g_na_ctx[dev];
    }
    uint32_t host[2] = {0, 0};
    for (int i = 0; i < 2 && e == hipSuccess; ++i) {
        if (!ctxs[i]) continue;
        e = hipMemcpyAsync(&host[i], ctxs[i]->err, sizeof(uint32_t), hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipMemsetAsync(ctxs[i]->err, 0, sizeof(uint32_t), s);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, "reading device error bits");
    *bits = host[0] | host[1];
    if (*bits & kErrSpinTimeout) g_tripped[dev].store(1u);
    return MOA_SUCCESS;
}

int moa_clear_device_state(int device) {
    if (device < 0 || device >= kMaxDevices) return fail(MOA_ERROR_INVALID_VALUE, "device index out of range");
    g_tripped[device].store(0u);
    return MOA_SUCCESS;
}

int moa_sliding_project_qkv(const uint16_t* x, const uint8_t* q_weight, const uint8_t* k_weight,
                            const uint8_t* v_weight, const float* q_weight_scale,
                            const float* k_weight_scale, const float* v_weight_scale,
                            const uint16_t* input_rms_weight, const uint16_t* q_rms_weight,
                            const uint16_t* k_rms_weight, const int32_t* kv_offset,
                            const int32_t* rope_offset, const uint16_t* cos, const uint16_t* sin,
                            uint16_t* k_cache, uint16_t* v_cache, uint16_t* q_out, int M, void* stream) {
    QkvParams p{x, q_weight, k_weight, v_weight, q_weight_scale, k_weight_scale, v_weight_scale, ScaleKind::F32,
                input_rms_weight, q_rms_weight, k_rms_weight, kv_offset, rope_offset, cos, sin,
                k_cache, v_cache, q_out};
    return qkv_common(p, M, stream);
}

int moa_sliding_project_qkv_bf16_scales(
    const uint16_t* x, const uint8_t* q_weight, const uint8_t* k_weight, const uint8_t* v_weight,
    const uint16_t* q_weight_scale, const uint16_t* k_weight_scale, const uint16_t* v_weight_scale,
    const uint16_t* input_rms_weight, const uint16_t* q_rms_weight, const uint16_t* k_rms_weight,
    const int32_t* kv_offset, const int32_t* rope_offset, const uint16_t* cos, const uint16_t* sin,
    uint16_t* k_cache, uint16_t* v_cache, uint16_t* q_out, int M, void* stream) {
    QkvParams p{x, q_weight, k_weight, v_weight, q_weight_scale, k_weight_scale, v_weight_scale, ScaleKind::BF16,
                input_rms_weight, q_rms_weight, k_rms_weight, kv_offset, rope_offset, cos, sin,
                k_cache, v_cache, q_out};
    return qkv_common(p, M, stream);
}

int moa_sliding_attention_output(const uint16_t* x, const uint16_t* post_attn_rms_weight,
                                 const uint8_t* o_weight, const float* o_weight_scale,
                                 uint16_t* residual, int M, void* stream) {
    OParams p{x, post_attn_rms_weight, o_weight, o_weight_scale, ScaleKind::F32, residual};
    return o_common(p, M, stream);
}

int moa_sliding_attention_output_bf16_scales(const uint16_t* x, const uint16_t* post_attn_rms_weight,
                                             const uint8_t* o_weight, const uint16_t* o_weight_scale,
                                             uint16_t* residual, int M, void* stream) {
    OParams p{x, post_attn_rms_weight, o_weight, o_weight_scale, ScaleKind::BF16, residual};
    return o_common(p, M, stream);
}

int moa_decoder_feedforward(uint16_t* residual, const uint16_t* pre_ff_rms_weight,
                            const uint8_t* up_weight_packed, const uint8_t* gate_weight_packed,
                            const uint8_t* down_weight_packed, const uint8_t* up_weight_scale,
                            const uint8_t* gate_weight_scale, const uint8_t* down_weight_scale,
                            const float* up_global_scale, const float* gate_global_scale,
                            const float* down_global_scale, const uint16_t* post_ff_rms_weight,
                            const uint16_t* layer_scalar, int M, void* stream) {
    FfnParams p{FfnFormat::NVFP4, residual, pre_ff_rms_weight, up_weight_packed, gate_weight_packed,
                down_weight_packed, up_weight_scale, gate_weight_scale, down_weight_scale, ScaleKind::F32,
                up_global_scale, gate_global_scale, down_global_scale, post_ff_rms_weight, layer_scalar};
    return ffn_common(p, M, stream);
}

int moa_decoder_feedforward_fp8(uint16_t* residual, const uint16_t* pre_ff_rms_weight,
                                const uint8_t* up_weight, const uint8_t* gate_weight,
                                const uint8_t* down_weight, const float* up_weight_scale,
                                const float* gate_weight_scale, const float* down_weight_scale,
                                const uint16_t* post_ff_rms_weight, const uint16_t* layer_scalar,
                                int M, void* stream) {
    FfnParams p{FfnFormat::FP8, residual, pre_ff_rms_weight, up_weight, gate_weight, down_weight,
                up_weight_scale, gate_weight_scale, down_weight_scale, ScaleKind::F32,
                nullptr, nullptr, nullptr, post_ff_rms_weight, layer_scalar};
    return ffn_common(p, M, stream);
}

int moa_decoder_feedforward_fp8_noalloc(uint16_t* residual, const uint16_t* pre_ff_rms_weight,
                                        const uint8_t* up_weight, const uint8_t* gate_weight,
                                        const uint8_t* down_weight, const float* up_weight_scale,
                                        const float* gate_weight_scale, const float* down_weight_scale,
                                        const uint16_t* post_ff_rms_weight, const uint16_t* layer_scalar,
                                        int M, void* stream) {
    FfnParams p{FfnFormat::FP8, residual, pre_ff_rms_weight, up_weight, gate_weight, down_weight,
                up_weight_scale, gate_weight_scale, down_weight_scale, ScaleKind::F32,
                nullptr, nullptr, nullptr, post_ff_rms_weight, layer_scalar};
    if (const int bad = ffn_check(p, M)) return bad;
    if (M > kMaxDecodeM)
        return fail(MOA_ERROR_INVALID_VALUE, "M must be in [1, " + std::to_string(kMaxDecodeM) +
                                                 "] for the no-allocation entry point, got " + std::to_string(M));
    int code = MOA_SUCCESS;
    DevCtx* ctx = noalloc_context(&code);
    if (!ctx) return code;
    return finish(launch_ffn_decode(p, M, static_cast<hipStream_t>(stream), ctx), "decoder_feedforward_fp8_noalloc launch");
}

int moa_decoder_feedforward_mxfp4(uint16_t* residual, const uint16_t* pre_ff_rms_weight,
                                  const uint8_t* up_weight_packed, const uint8_t* gate_weight_packed,
                                  const uint8_t* down_weight_packed, const uint8_t* up_weight_scale,
                                  const uint8_t* gate_weight_scale, const uint8_t* down_weight_scale,
                                  const uint16_t* post_ff_rms_weight, const uint16_t* layer_scalar,
                                  int M, void* stream) {
    FfnParams p{FfnFormat::MXFP4, residual, pre_ff_rms_weight, up_weight_packed, gate_weight_packed,
                down_weight_packed, up_weight_scale, gate_weight_scale, down_weight_scale, ScaleKind::F32,
                nullptr, nullptr, nullptr, post_ff_rms_weight, layer_scalar};
    return ffn_common(p, M, stream);
}

int moa_sliding_attention_output_feedforward(
    const uint16_t* x, const uint16_t* post_attn_rms_weight, const uint8_t* o_weight, const uint16_t* o_weight_scale,
    uint16_t* residual, const uint16_t* pre_ff_rms_weight, const uint8_t* up_weight_packed,
    const uint8_t* gate_weight_packed, const uint8_t* down_weight_packed, const uint8_t* up_weight_scale,
    const uint8_t* gate_weight_scale, const uint8_t* down_weight_scale, const float* up_global_scale,
    const float* gate_global_scale, const float* down_global_scale, const uint16_t* post_ff_rms_weight,
    const uint16_t* layer_scalar, int M, void* stream) {
    OParams o{x, post_attn_rms_weight, o_weight, o_weight_scale, ScaleKind::BF16, residual};
    FfnParams p{FfnFormat::NVFP4, residual, pre_ff_rms_weight, up_weight_packed, gate_weight_packed,
                down_weight_packed, up_weight_scale, gate_weight_scale, down_weight_scale, ScaleKind::F32,
                up_global_scale, gate_global_scale, down_global_scale, post_ff_rms_weight, layer_scalar};
    return o_ffn_common(o, p, M, stream);
}

int moa_sliding_attention_output_feedforward_fp8(
    const uint16_t* x, const uint16_t* post_attn_rms_weight, const uint8_t* o_weight, const float* o_weight_scale,
    uint16_t* residual, const uint16_t* pre_ff_rms_weight, const uint8_t* up_weight, const uint8_t* gate_weight,
    const uint8_t* down_weight, const float* up_weight_scale, const float* gate_weight_scale,
    const float* down_weight_scale, const uint16_t* post_ff_rms_weight, const uint16_t* layer_scalar, int M,
    void* stream) {
    OParams o{x, post_attn_rms_weight, o_weight, o_weight_scale, ScaleKind::F32, residual};
    FfnParams p{FfnFormat::FP8, residual, pre_ff_rms_weight, up_weight, gate_weight, down_weight,
                up_weight_scale, gate_weight_scale, down_weight_scale, ScaleKind::F32,
                nullptr, nullptr, nullptr, post_ff_rms_weight, layer_scalar};
    return o_ffn_common(o, p, M, stream);
}

int moa_sliding_attention_output_feedforward_mxfp4(
    const uint16_t* x, const uint16_t* post_attn_rms_weight, const uint8_t* o_weight, const float* o_weight_scale,
    uint16_t* residual, const uint16_t* pre_ff_rms_weight, const uint8_t* up_weight_packed,
    const uint8_t* gate_weight_packed, const uint8_t* down_weight_packed, const uint8_t* up_weight_scale,
    const uint8_t* gate_weight_scale, const uint8_t* down_weight_scale, const uint16_t* post_ff_rms_weight,
    const uint16_t* layer_scalar, int M, void* stream) {
    OParams o{x, post_attn_rms_weight, o_weight, o_weight_scale, ScaleKind::F32, residual};
    FfnParams p{FfnFormat::MXFP4, residual, pre_ff_rms_weight, up_weight_packed, gate_weight_packed,
                down_weight_packed, up_weight_scale, gate_weight_scale, down_weight_scale, ScaleKind::F32,
                nullptr, nullptr, nullptr, post_ff_rms_weight, layer_scalar};
    return o_ffn_common(o, p, M, stream);
}

int moa_sliding_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* mask, uint16_t* out,
                          int M, void* stream) {
    Check c;
    c.ptr(q, "q").ptr(k, "k").ptr(v, "v").ptr(mask, "mask", 4).ptr(out, "out").rows(M);
    if (c.code) return c.code;
    int code = MOA_SUCCESS;
    DevCtx* ctx = ctx_or_fail(&code);
    if (!ctx) return code;
    return finish(launch_sliding_attention(q, k, v, mask, out, M, static_cast<hipStream_t>(stream), ctx),
                  "sliding_attention launch");
}

int moa_full_project_qkv(const uint16_t* x, const uint8_t* q_weight, const uint8_t* k_weight,
                         const uint16_t* q_weight_scale, const uint16_t* k_weight_scale,
                         const uint16_t* input_rms_weight, const uint16_t* q_rms_weight, const uint16_t* k_rms_weight,
                         const int32_t* kv_offset, const int32_t* rope_offset, const uint16_t* cos, const uint16_t* sin,
                         uint16_t* k_cache, uint16_t* v_cache, uint16_t* q_out, int M, void* stream) {
    Check c;
    c.ptr(x, "x").ptr(q_weight, "q_weight").ptr(k_weight, "k_weight");
    c.ptr(q_weight_scale, "q_weight_scale", 2).ptr(k_weight_scale, "k_weight_scale", 2);
    c.ptr(input_rms_weight, "input_rms_weight").ptr(q_rms_weight, "q_rms_weight").ptr(k_rms_weight, "k_rms_weight");
    c.ptr(kv_offset, "kv_offset", 4).ptr(rope_offset, "rope_offset", 4).ptr(cos, "cos").ptr(sin, "sin");
    c.ptr(k_cache, "k_cache").ptr(v_cache, "v_cache").ptr(q_out, "q_out").rows(M);
    if (c.code) return c.code;
    int code = MOA_SUCCESS;
    DevCtx* ctx = ctx_or_fail(&code);
    if (!ctx) return code;
    QkvParams p{x, q_weight, k_weight, nullptr, q_weight_scale, k_weight_scale, nullptr, ScaleKind::BF16,
                input_rms_weight, q_rms_weight, k_rms_weight, kv_offset, rope_offset, cos, sin, k_cache, v_cache, q_out};
    return finish(launch_full_qkv(p, M, static_cast<hipStream_t>(stream), ctx), "full_project_qkv launch");
}

static int full_page(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* mask, float* running_max,
                     float* running_sum, uint16_t* out, int M, bool first, void* stream) {
    Check c;
    c.ptr(q, "q").ptr(k, "k").ptr(v, "v").ptr(mask, "mask", 4).ptr(running_max, "running_max", 4);
    c.ptr(running_sum, "running_sum", 4).ptr(out, "out").rows(M);
    if (c.code) return c.code;
    int code = MOA_SUCCESS;
    DevCtx* ctx = ctx_or_fail(&code);
    if (!ctx) return code;
    return finish(launch_full_attention_page(q, k, v, mask, running_max, running_sum, out, M, first,
                                             static_cast<hipStream_t>(stream), ctx),
                  first ? "full_attention_first_page launch" : "full_attention_page launch");
}

int moa_full_attention_first_page(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* mask,
                                  float* running_max, float* running_sum, uint16_t* out, int M, void* stream) {
    return full_page(q, k, v, mask, running_max, running_sum, out, M, true, stream);
}

int moa_full_attention_page(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* mask,
                            float* running_max, float* running_sum, uint16_t* out, int M, void* stream) {
    return full_page(q, k, v, mask, running_max, running_sum, out, M, false, stream);
}

int moa_full_attention(const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages, const float* masks, int P,
                       float* running_max, float* running_sum, uint16_t* out, int M, void* stream) {
    Check c;
    c.ptr(q, "q").ptr(k_pages, "k_pages").ptr(v_pages, "v_pages").ptr(masks, "masks", 4);
    c.ptr(running_max, "running_max", 4).ptr(running_sum, "running_sum", 4).ptr(out, "out").rows(M);
    if (c.code) return c.code;
    if (P < 1 || P > kCf) return fail(MOA_ERROR_INVALID_VALUE, "P must be in [1, 64], got " + std::to_string(P));
    int code = MOA_SUCCESS;
    DevCtx* ctx = ctx_or_fail(&code);
    if (!ctx) return code;
    return finish(launch_full_attention(q, k_pages, v_pages, masks, P, running_max, running_sum, out, M,
                                        static_cast<hipStream_t>(stream), ctx),
                  "full_attention launch");
}

int moa_full_attention_output(const uint16_t* x, const float* running_sum, const uint16_t* post_attn_rms_weight,
                              const uint8_t* o_weight, const uint16_t* o_weight_scale, uint16_t* residual, int M,
                              void* stream) {
    Check c;
    c.ptr(x, "x").ptr(running_sum, "running_sum", 4).ptr(post_attn_rms_weight, "post_attn_rms_weight");
    c.ptr(o_weight, "o_weight").ptr(o_weight_scale, "o_weight_scale", 2).ptr(residual, "residual").rows(M);
    if (c.code) return c.code;
    int code = MOA_SUCCESS;
    DevCtx* ctx = ctx_or_fail(&code);
    if (!ctx) return code;
    OParams p{x, post_attn_rms_weight, o_weight, o_weight_scale, ScaleKind::BF16, residual, running_sum};
    return finish(launch_full_o(p, M, static_cast<hipStream_t>(stream), ctx), "full_attention_output launch");
}

int moa_final_norm_and_logits(const uint16_t* input, const uint16_t* rms_weight, const uint16_t* lm_head_weight,
                              uint16_t* out, int M, void* stream) {
    Check c;
    c.ptr(input, "input").ptr(rms_weight, "rms_weight").ptr(lm_head_weight, "lm_head_weight").ptr(out, "out").rows(M);
    if (c.code) return c.code;
    if (g_tripped[current_device_or_0()].load()) return tripped_fail(current_device_or_0());
    return finish(launch_final_norm_and_logits(input, rms_weight, lm_head_weight, out, M, static_cast<hipStream_t>(stream)),
                  "final_norm_and_logits launch");
}

int moa_fp8_scaled_projection(const uint16_t* x, const uint8_t* w, const float* scale, uint16_t* out,
                              int M, int N, int K, void* stream) {
    Check c;
    c.ptr(x, "x").ptr(w, "w").ptr(scale, "scale", 4).ptr(out, "out", 2).rows(M);
    if (c.code) return c.code;
    if (N < 1 || K < 16 || K % 16) return fail(MOA_ERROR_INVALID_VALUE, "need N >= 1 and K a positive multiple of 16");
    if (M > 65535) return fail(MOA_ERROR_INVALID_VALUE, "M must be <= 65535 for the projection");
    if (g_tripped[current_device_or_0()].load()) return tripped_fail(current_device_or_0());
    ProjParams p{x, w, scale, ScaleKind::F32, out, N, K};
    return finish(launch_proj_decode(p, M, static_cast<hipStream_t>(stream)), "fp8_scaled_projection launch");
}

int moa_test_epoch_layout(int kernel, int* counters, int* per) {
    if (!counters || !per) return fail(MOA_ERROR_INVALID_VALUE, "counters and per must not be NULL");
    switch (kernel) {
        case 0: *counters = kQkvEpochCounters; *per = kQkvEpochPer; return MOA_SUCCESS;
        case 1: *counters = kOEpochCounters; *per = kOEpochPer; return MOA_SUCCESS;
        case 2: *counters = kFfnEpochCounters; *per = kFfnEpochPer; return MOA_SUCCESS;
        case 3: *counters = kRowsEpochCounters; *per = kRowsEpochPer; return MOA_SUCCESS;
    }
    return fail(MOA_ERROR_INVALID_VALUE, "kernel must be 0 (QKV), 1 (O), 2 (FFN) or 3 (rows FFN)");
}

int moa_test_epoch_tag(int kernel, uint64_t old, uint32_t* tag) {
    if (!tag) return fail(MOA_ERROR_INVALID_VALUE, "tag is NULL");
    switch (kernel) {
        case 0: *tag = epoch_tag<kQkvEpochPer>(old); return MOA_SUCCESS;
        case 1: *tag = epoch_tag<kOEpochPer>(old); return MOA_SUCCESS;
        case 2: *tag = epoch_tag<kFfnEpochPer>(old); return MOA_SUCCESS;
        case 3: *tag = epoch_tag<kRowsEpochPer>(old); return MOA_SUCCESS;
    }
    return fail(MOA_ERROR_INVALID_VALUE, "kernel must be 0 (QKV), 1 (O), 2 (FFN) or 3 (rows FFN)");
}

int moa_test_preset_epochs(uint64_t launches) {
    int code = MOA_SUCCESS;
    DevCtx* ctx = ctx_or_fail(&code);
    if (!ctx) return code;
    hipError_t e = hipDeviceSynchronize();
    auto put64 = [&](int first, int n, uint64_t v) {
        for (int i = 0; i < n && e == hipSuccess; ++i)
            e = hipMemcpy(ctx->tickets + (size_t)(first + i) * kTicketStride, &v, sizeof v, hipMemcpyHostToDevice);
    };
    put64(kTicketQkvEpoch, kQkvEpochCounters, launches * kQkvEpochPer);
    put64(kTicketOEpoch, kOEpochCounters, launches * kOEpochPer);
    put64(kTicketFfnEpoch, kFfnEpochCounters, launches * kFfnEpochPer);
    put64(kTicketRowsEpoch, kRowsEpochCounters, launches * kRowsEpochPer);
    const uint32_t at = (uint32_t)(launches * 32u);
    for (int i = 0; i < kMaxDecodeM * kNs && e == hipSuccess; ++i)
        e = hipMemcpy(ctx->tickets + (size_t)(kTicketAttn + i) * kTicketStride, &at, sizeof at, hipMemcpyHostToDevice);
    return finish(e, "presetting the epoch counters");
}

int moa_test_set_stall(uint32_t steal_ticks, uint32_t hold_ticks, const int32_t* hold) {
    Stall st = {kStealTicks, 0, {-1, -1, -1, -1}};
    if (steal_ticks) {
        st.steal_ticks = steal_ticks;
        st.hold_ticks = hold ? hold_ticks : 0;
        for (int i = 0; i < 4 && hold; ++i) st.hold[i] = hold[i];
    }
    set_stall(st);
    return MOA_SUCCESS;
}

int moa_test_set_rows_one_launch(int on) {
    set_rows_one_launch(on != 0);
    return MOA_SUCCESS;
}

int moa_test_take_overs(uint32_t* count) {
    Check c;
    c.ptr(count, "count", 1);
    if (c.code) return c.code;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(MOA_ERROR_NO_DEVICE, "device index out of range");
    // both scratches' counters, as moa_device_errors reads both error words
    const DevCtx* ctxs[2] = {existing_context(dev), nullptr};
    {
        std::lock_guard<std::mutex> lock(g_na_mutex);
        if (g_na_ctx[dev].base) ctxs[1] = &g_na_ctx[dev];
    }
    e = hipDeviceSynchronize();
    uint32_t total = 0;
    const uint32_t zero = 0;
    for (int i = 0; i < 2 && e == hipSuccess; ++i) {
        if (!ctxs[i]) continue;
        uint32_t n = 0;
        e = hipMemcpy(&n, ctxs[i]->err + kErrTakeOvers, sizeof n, hipMemcpyDeviceToHost);
        if (e == hipSuccess) e = hipMemcpy(ctxs[i]->err + kErrTakeOvers, &zero, sizeof zero, hipMemcpyHostToDevice);
        total += n;
    }
    if (e == hipSuccess) *count = total;
    return finish(e, "reading the take-over count");
}

int moa_test_trip_device_state(int device) {
    if (device < 0 || device >= kMaxDevices) return fail(MOA_ERROR_INVALID_VALUE, "device index out of range");
    g_tripped[device].store(1u);
    return MOA_SUCCESS;
}

int moa_test_scratch_state(uint32_t* state) {
    Check c;
    c.ptr(state, "state", 4);
    if (c.code) return c.code;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(MOA_ERROR_NO_DEVICE, "device index out of range");
    uint32_t v = existing_context(dev) ? 1u : 0u;
    {
        std::lock_guard<std::mutex> lock(g_na_mutex);
        if (g_na_ctx[dev].base) v |= 2u;
    }
    *state = v;
    return MOA_SUCCESS;
}

int moa_format_selftest(uint32_t* out, void* stream) {
    Check c;
    c.ptr(out, "out", 4);
    if (c.code) return c.code;
    return finish(launch_format_selftest(out, static_cast<hipStream_t>(stream)), "format selftest launch");
}

}  // extern "C"
