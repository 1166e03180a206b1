// moa_ops.hpp -- C++ host interface over the C ABI (include/moa_ops.h), shaped like the reference
// crate's operator module (furiosa-opt-gemma4-12B/src/ops.rs, "FO/" below) and the tensor types
// its callers hold (FO/src/host/runtime.rs, FO/src/bin/test_kernels.rs).
//
//   Reference                                      Here
//   &mut Device                                     moa::Device& (a HIP device and one stream)
//   HbmTensor<bf16 | f8e4m3 | f4e2m1 | f32 | i32,   moa::HbmTensor<bf16 | f8e4m3 | f4e2m1x2 | e8m0 |
//             Chip, m![shape]>                                     float | int32_t> (runtime shape)
//   HostTensor::to_hbm / read back                  HbmTensor::from_host / HbmTensor::to_host
//   ops::<name>(device, args...) + launch().await   moa::ops::<name>(device, args...)
//   Result<_, Error>, unwrapped by the harness       moa::Error thrown on a rejected call
//
// Every operator keeps the reference's name, argument order and in-place outputs. Shapes are
// compile-time types in the reference; here each tensor carries its shape and the operator
// checks element counts before the C call (a mismatch throws moa::Error with
// MOA_ERROR_INVALID_VALUE, and nothing is launched). The leading dimension of the activation
// tensors is the number of token rows M (the reference passes exactly one).
//
// Work is ordered on the device's stream and the operators return without synchronising;
// to_host() synchronises. Header-only; link with libmoa_gfx950.so and the HIP runtime.
#ifndef MOA_OPS_HPP
#define MOA_OPS_HPP

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <numeric>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

#include "moa_ops.h"

namespace moa {

// Element types of the reference's tensors. Each is the raw storage unit the C ABI takes.
struct bf16 { uint16_t bits; };      // bfloat16 bit pattern
struct f8e4m3 { uint8_t code; };     // one E4M3FN code
struct f4e2m1x2 { uint8_t codes; };  // two E2M1 codes, the even element in the low nibble
struct e8m0 { uint8_t code; };       // one E8M0 block scale (MXFP4)

// Shapes (FO/src/axes.rs:3-29).
constexpr size_t kH = 3840, kL = 15360, kNs = 8, kGs = 2, kDs = 256, kQs = 4096, kPs = 2048, kTs = 1024;
constexpr size_t kE = 32768, kGf = 16, kDf = 512, kQf = 8192, kPf = 512, kTf = 512, kW = 262144;

// A rejected call: code is the MOA_ERROR_* value, what() the library's reason.
class Error : public std::runtime_error {
  public:
    Error(int code, const std::string& what) : std::runtime_error(what), code_(code) {}
    int code() const { return code_; }

  private:
    int code_;
};

inline void check(int rc, const char* what) {
    if (rc != MOA_SUCCESS) throw Error(rc, std::string(what) + ": " + moa_last_error_string());
}

inline void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess) throw Error(MOA_ERROR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

// The reference's Device: one accelerator with one ordered queue. A HIP device index and a
// stream created on it (default priority); moa_init sets up the library's per-device scratch.
class Device {
  public:
    explicit Device(int index = 0) : index_(index) {
        check_hip(hipSetDevice(index_), "hipSetDevice");
        check(moa_init(index_), "moa_init");
        check_hip(hipStreamCreate(&stream_), "hipStreamCreate");
    }
    ~Device() {
        if (stream_) {
            (void)hipSetDevice(index_);
            (void)hipStreamSynchronize(stream_);
            (void)hipStreamDestroy(stream_);
        }
    }
    Device(const Device&) = delete;
    Device& operator=(const Device&) = delete;

    int index() const { return index_; }
    hipStream_t stream() const { return stream_; }
    // The calling thread's current device must be this one for every library call.
    void make_current() const { check_hip(hipSetDevice(index_), "hipSetDevice"); }
    void synchronize() const {
        make_current();
        check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize");
    }
    // The device error word (MOA_DEVERR_* bits), synchronising the stream.
    uint32_t device_errors() const {
        make_current();
        uint32_t bits = 0;
        check(moa_device_errors(stream_, &bits), "moa_device_errors");
        return bits;
    }

  private:
    int index_;
    hipStream_t stream_ = nullptr;
};

// A device buffer of T with a shape, owned: hipMalloc'd at construction, hipFree'd at destruction
// (hipFree waits for the device's outstanding work, so a tensor may go out of scope right after an
// operator that uses it).
template <class T>
class HbmTensor {
    static_assert(std::is_trivially_copyable<T>::value, "device tensors hold plain values");

  public:
    HbmTensor() = default;
    // A zero-filled tensor (the reference harness's zeros(device)).
    HbmTensor(const Device& d, std::vector<size_t> shape) : shape_(std::move(shape)) {
        n_ = std::accumulate(shape_.begin(), shape_.end(), size_t{1}, [](size_t a, size_t b) { return a * b; });
        d.make_current();
        check_hip(hipMalloc(reinterpret_cast<void**>(&ptr_), bytes()), "hipMalloc");
        try {
            check_hip(hipMemsetAsync(ptr_, 0, bytes(), d.stream()), "hipMemsetAsync");
            check_hip(hipStreamSynchronize(d.stream()), "hipStreamSynchronize");
        } catch (...) {  // no destructor runs for a constructor that throws
            (void)hipFree(ptr_);
            throw;
        }
    }
    // The host values, uploaded (HostTensor::to_hbm).
    static HbmTensor from_host(const Device& d, const std::vector<T>& host, std::vector<size_t> shape) {
        HbmTensor t(d, std::move(shape));
        if (host.size() != t.n_) throw Error(MOA_ERROR_INVALID_VALUE, "from_host: host data does not match the shape");
        check_hip(hipMemcpyAsync(t.ptr_, host.data(), t.bytes(), hipMemcpyHostToDevice, d.stream()), "hipMemcpyAsync");
        check_hip(hipStreamSynchronize(d.stream()), "hipStreamSynchronize");
        return t;
    }
    // The values, read back after everything queued on the device's stream.
    std::vector<T> to_host(const Device& d) const {
        std::vector<T> host(n_);
        d.make_current();
        check_hip(hipMemcpyAsync(host.data(), ptr_, bytes(), hipMemcpyDeviceToHost, d.stream()), "hipMemcpyAsync");
        check_hip(hipStreamSynchronize(d.stream()), "hipStreamSynchronize");
        return host;
    }
    ~HbmTensor() {
        if (ptr_) (void)hipFree(ptr_);
    }
    HbmTensor(HbmTensor&& o) noexcept : ptr_(o.ptr_), n_(o.n_), shape_(std::move(o.shape_)) { o.ptr_ = nullptr; o.n_ = 0; }
    HbmTensor& operator=(HbmTensor&& o) noexcept {
        if (this != &o) {
            if (ptr_) (void)hipFree(ptr_);
            ptr_ = o.ptr_;
            n_ = o.n_;
            shape_ = std::move(o.shape_);
            o.ptr_ = nullptr;
            o.n_ = 0;
        }
        return *this;
    }
    HbmTensor(const HbmTensor&) = delete;
    HbmTensor& operator=(const HbmTensor&) = delete;

    T* data() { return ptr_; }
    const T* data() const { return ptr_; }
    size_t size() const { return n_; }
    size_t bytes() const { return n_ * sizeof(T); }
    const std::vector<size_t>& shape() const { return shape_; }

  private:
    T* ptr_ = nullptr;
    size_t n_ = 0;
    std::vector<size_t> shape_;
};

namespace detail {
template <class T>
inline void want(const HbmTensor<T>& t, size_t n, const char* name) {
    if (t.size() != n || !t.data())
        throw Error(MOA_ERROR_INVALID_VALUE, std::string(name) + ": " + std::to_string(t.size()) +
                                                 " elements, the operator takes " + std::to_string(n));
}
// M token rows from an activation tensor of `per_row` elements per row.
template <class T>
inline int rows(const HbmTensor<T>& t, size_t per_row, const char* name) {
    if (t.size() == 0 || t.size() % per_row)
        throw Error(MOA_ERROR_INVALID_VALUE, std::string(name) + ": not a whole number of token rows");
    return static_cast<int>(t.size() / per_row);
}
inline const uint16_t* u16(const HbmTensor<bf16>& t) { return reinterpret_cast<const uint16_t*>(t.data()); }
inline uint16_t* u16(HbmTensor<bf16>& t) { return reinterpret_cast<uint16_t*>(t.data()); }
template <class T>
inline const uint8_t* u8(const HbmTensor<T>& t) {
    static_assert(sizeof(T) == 1, "byte codes");
    return reinterpret_cast<const uint8_t*>(t.data());
}
inline const uint16_t* opt_u16(const HbmTensor<bf16>* t) { return t ? u16(*t) : nullptr; }
}  // namespace detail

namespace ops {

// ops::sliding_project_qkv -- FO/src/ops.rs:37-76 (bf16 per-channel scales, as the reference).
inline void sliding_project_qkv(const Device& device, const HbmTensor<bf16>& x, const HbmTensor<f8e4m3>& q_weight,
                                const HbmTensor<f8e4m3>& k_weight, const HbmTensor<f8e4m3>& v_weight,
                                const HbmTensor<bf16>& q_weight_scale, const HbmTensor<bf16>& k_weight_scale,
                                const HbmTensor<bf16>& v_weight_scale, const HbmTensor<bf16>& input_rms_weight,
                                const HbmTensor<bf16>& q_rms_weight, const HbmTensor<bf16>& k_rms_weight,
                                const HbmTensor<int32_t>& kv_offset, const HbmTensor<int32_t>& rope_offset,
                                const HbmTensor<bf16>& cos, const HbmTensor<bf16>& sin, HbmTensor<bf16>& k_cache,
                                HbmTensor<bf16>& v_cache, HbmTensor<bf16>& q_out) {
    using namespace detail;
    const int M = rows(x, kH, "x");
    want(q_weight, kQs * kH, "q_weight"); want(k_weight, kPs * kH, "k_weight"); want(v_weight, kPs * kH, "v_weight");
    want(q_weight_scale, kQs, "q_weight_scale"); want(k_weight_scale, kPs, "k_weight_scale");
    want(v_weight_scale, kPs, "v_weight_scale"); want(input_rms_weight, kH, "input_rms_weight");
    want(q_rms_weight, kDs, "q_rms_weight"); want(k_rms_weight, kDs, "k_rms_weight");
    want(kv_offset, 1, "kv_offset"); want(rope_offset, 1, "rope_offset");
    want(cos, kE * kDs, "cos"); want(sin, kE * kDs, "sin");
    want(k_cache, kTs * kNs * kDs, "k_cache"); want(v_cache, kTs * kNs * kDs, "v_cache");
    want(q_out, M * kQs, "q_out");
    device.make_current();
    check(moa_sliding_project_qkv_bf16_scales(u16(x), u8(q_weight), u8(k_weight), u8(v_weight), u16(q_weight_scale),
                                              u16(k_weight_scale), u16(v_weight_scale), u16(input_rms_weight),
                                              u16(q_rms_weight), u16(k_rms_weight), kv_offset.data(),
                                              rope_offset.data(), u16(cos), u16(sin), u16(k_cache), u16(v_cache),
                                              u16(q_out), M, device.stream()),
          "sliding_project_qkv");
}

// The same with f32 per-channel scales.
inline void sliding_project_qkv(const Device& device, const HbmTensor<bf16>& x, const HbmTensor<f8e4m3>& q_weight,
                                const HbmTensor<f8e4m3>& k_weight, const HbmTensor<f8e4m3>& v_weight,
                                const HbmTensor<float>& q_weight_scale, const HbmTensor<float>& k_weight_scale,
                                const HbmTensor<float>& v_weight_scale, const HbmTensor<bf16>& input_rms_weight,
                                const HbmTensor<bf16>& q_rms_weight, const HbmTensor<bf16>& k_rms_weight,
                                const HbmTensor<int32_t>& kv_offset, const HbmTensor<int32_t>& rope_offset,
                                const HbmTensor<bf16>& cos, const HbmTensor<bf16>& sin, HbmTensor<bf16>& k_cache,
                                HbmTensor<bf16>& v_cache, HbmTensor<bf16>& q_out) {
    using namespace detail;
    const int M = rows(x, kH, "x");
    want(q_weight, kQs * kH, "q_weight"); want(k_weight, kPs * kH, "k_weight"); want(v_weight, kPs * kH, "v_weight");
    want(q_weight_scale, kQs, "q_weight_scale"); want(k_weight_scale, kPs, "k_weight_scale");
    want(v_weight_scale, kPs, "v_weight_scale"); want(input_rms_weight, kH, "input_rms_weight");
    want(q_rms_weight, kDs, "q_rms_weight"); want(k_rms_weight, kDs, "k_rms_weight");
    want(kv_offset, 1, "kv_offset"); want(rope_offset, 1, "rope_offset");
    want(cos, kE * kDs, "cos"); want(sin, kE * kDs, "sin");
    want(k_cache, kTs * kNs * kDs, "k_cache"); want(v_cache, kTs * kNs * kDs, "v_cache");
    want(q_out, M * kQs, "q_out");
    device.make_current();
    check(moa_sliding_project_qkv(u16(x), u8(q_weight), u8(k_weight), u8(v_weight), q_weight_scale.data(),
                                  k_weight_scale.data(), v_weight_scale.data(), u16(input_rms_weight),
                                  u16(q_rms_weight), u16(k_rms_weight), kv_offset.data(), rope_offset.data(), u16(cos),
                                  u16(sin), u16(k_cache), u16(v_cache), u16(q_out), M, device.stream()),
          "sliding_project_qkv");
}

// ops::sliding_attention -- FO/src/ops.rs:118-128.
inline void sliding_attention(const Device& device, const HbmTensor<bf16>& q, const HbmTensor<bf16>& k,
                              const HbmTensor<bf16>& v, const HbmTensor<float>& mask, HbmTensor<bf16>& out_hbm) {
    using namespace detail;
    const int M = rows(q, kQs, "q");
    want(k, kTs * kNs * kDs, "k"); want(v, kTs * kNs * kDs, "v");
    want(mask, M * kTs, "mask"); want(out_hbm, M * kQs, "out_hbm");
    device.make_current();
    check(moa_sliding_attention(u16(q), u16(k), u16(v), mask.data(), u16(out_hbm), M, device.stream()),
          "sliding_attention");
}

// ops::sliding_attention_output -- FO/src/ops.rs:130-146 (bf16 scales, as the reference).
inline void sliding_attention_output(const Device& device, const HbmTensor<bf16>& x,
                                     const HbmTensor<bf16>& post_attn_rms_weight, const HbmTensor<f8e4m3>& o_weight,
                                     const HbmTensor<bf16>& o_weight_scale, HbmTensor<bf16>& residual_hbm) {
    using namespace detail;
    const int M = rows(x, kQs, "x");
    want(post_attn_rms_weight, kH, "post_attn_rms_weight"); want(o_weight, kH * kQs, "o_weight");
    want(o_weight_scale, kH, "o_weight_scale"); want(residual_hbm, M * kH, "residual_hbm");
    device.make_current();
    check(moa_sliding_attention_output_bf16_scales(u16(x), u16(post_attn_rms_weight), u8(o_weight), u16(o_weight_scale),
                                                   u16(residual_hbm), M, device.stream()),
          "sliding_attention_output");
}

// The same with f32 per-channel scales.
inline void sliding_attention_output(const Device& device, const HbmTensor<bf16>& x,
                                     const HbmTensor<bf16>& post_attn_rms_weight, const HbmTensor<f8e4m3>& o_weight,
                                     const HbmTensor<float>& o_weight_scale, HbmTensor<bf16>& residual_hbm) {
    using namespace detail;
    const int M = rows(x, kQs, "x");
    want(post_attn_rms_weight, kH, "post_attn_rms_weight"); want(o_weight, kH * kQs, "o_weight");
    want(o_weight_scale, kH, "o_weight_scale"); want(residual_hbm, M * kH, "residual_hbm");
    device.make_current();
    check(moa_sliding_attention_output(u16(x), u16(post_attn_rms_weight), u8(o_weight), o_weight_scale.data(),
                                       u16(residual_hbm), M, device.stream()),
          "sliding_attention_output");
}

// ops::decoder_feedforward -- FO/src/ops.rs:201-239, NVFP4 weights as the reference: E2M1 codes,
// E4M3 block-16 scales, device f32 reciprocal global scales; layer_scalar bf16 [8].
inline void decoder_feedforward(const Device& device, HbmTensor<bf16>& residual_hbm,
                                const HbmTensor<bf16>& pre_ff_rms_weight, const HbmTensor<f4e2m1x2>& up_weight_packed,
                                const HbmTensor<f4e2m1x2>& gate_weight_packed,
                                const HbmTensor<f4e2m1x2>& down_weight_packed, const HbmTensor<f8e4m3>& up_weight_scale,
                                const HbmTensor<f8e4m3>& gate_weight_scale, const HbmTensor<f8e4m3>& down_weight_scale,
                                const HbmTensor<float>& up_global_scale, const HbmTensor<float>& gate_global_scale,
                                const HbmTensor<float>& down_global_scale, const HbmTensor<bf16>& post_ff_rms_weight,
                                const HbmTensor<bf16>& layer_scalar) {
    using namespace detail;
    const int M = rows(residual_hbm, kH, "residual_hbm");
    want(pre_ff_rms_weight, kH, "pre_ff_rms_weight");
    want(up_weight_packed, kL * kH / 2, "up_weight_packed"); want(gate_weight_packed, kL * kH / 2, "gate_weight_packed");
    want(down_weight_packed, kH * kL / 2, "down_weight_packed");
    want(up_weight_scale, kL * kH / 16, "up_weight_scale"); want(gate_weight_scale, kL * kH / 16, "gate_weight_scale");
    want(down_weight_scale, kH * kL / 16, "down_weight_scale");
    want(up_global_scale, 1, "up_global_scale"); want(gate_global_scale, 1, "gate_global_scale");
    want(down_global_scale, 1, "down_global_scale");
    want(post_ff_rms_weight, kH, "post_ff_rms_weight"); want(layer_scalar, 8, "layer_scalar");
    device.make_current();
    check(moa_decoder_feedforward(u16(residual_hbm), u16(pre_ff_rms_weight), u8(up_weight_packed),
                                  u8(gate_weight_packed), u8(down_weight_packed), u8(up_weight_scale),
                                  u8(gate_weight_scale), u8(down_weight_scale), up_global_scale.data(),
                                  gate_global_scale.data(), down_global_scale.data(), u16(post_ff_rms_weight),
                                  u16(layer_scalar), M, device.stream()),
          "decoder_feedforward");
}

// The FFN with FP8 weights and f32 per-row scales. post_ff_rms_weight and
// layer_scalar may be null (the post-norm, the scalar skipped).
inline void decoder_feedforward_fp8(const Device& device, HbmTensor<bf16>& residual_hbm,
                                    const HbmTensor<bf16>& pre_ff_rms_weight, const HbmTensor<f8e4m3>& up_weight,
                                    const HbmTensor<f8e4m3>& gate_weight, const HbmTensor<f8e4m3>& down_weight,
                                    const HbmTensor<float>& up_weight_scale, const HbmTensor<float>& gate_weight_scale,
                                    const HbmTensor<float>& down_weight_scale,
                                    const HbmTensor<bf16>* post_ff_rms_weight, const HbmTensor<bf16>* layer_scalar) {
    using namespace detail;
    const int M = rows(residual_hbm, kH, "residual_hbm");
    want(pre_ff_rms_weight, kH, "pre_ff_rms_weight");
    want(up_weight, kL * kH, "up_weight"); want(gate_weight, kL * kH, "gate_weight"); want(down_weight, kH * kL, "down_weight");
    want(up_weight_scale, kL, "up_weight_scale"); want(gate_weight_scale, kL, "gate_weight_scale");
    want(down_weight_scale, kH, "down_weight_scale");
    if (post_ff_rms_weight) want(*post_ff_rms_weight, kH, "post_ff_rms_weight");
    if (layer_scalar) want(*layer_scalar, 8, "layer_scalar");
    device.make_current();
    check(moa_decoder_feedforward_fp8(u16(residual_hbm), u16(pre_ff_rms_weight), u8(up_weight), u8(gate_weight),
                                      u8(down_weight), up_weight_scale.data(), gate_weight_scale.data(),
                                      down_weight_scale.data(), opt_u16(post_ff_rms_weight), opt_u16(layer_scalar), M,
                                      device.stream()),
          "decoder_feedforward_fp8");
}

// The FFN with MXFP4 weights: E2M1 codes and E8M0 block-32 scales.
inline void decoder_feedforward_mxfp4(const Device& device, HbmTensor<bf16>& residual_hbm,
                                      const HbmTensor<bf16>& pre_ff_rms_weight,
                                      const HbmTensor<f4e2m1x2>& up_weight_packed,
                                      const HbmTensor<f4e2m1x2>& gate_weight_packed,
                                      const HbmTensor<f4e2m1x2>& down_weight_packed, const HbmTensor<e8m0>& up_weight_scale,
                                      const HbmTensor<e8m0>& gate_weight_scale, const HbmTensor<e8m0>& down_weight_scale,
                                      const HbmTensor<bf16>* post_ff_rms_weight, const HbmTensor<bf16>* layer_scalar) {
    using namespace detail;
    const int M = rows(residual_hbm, kH, "residual_hbm");
    want(pre_ff_rms_weight, kH, "pre_ff_rms_weight");
    want(up_weight_packed, kL * kH / 2, "up_weight_packed"); want(gate_weight_packed, kL * kH / 2, "gate_weight_packed");
    want(down_weight_packed, kH * kL / 2, "down_weight_packed");
    want(up_weight_scale, kL * kH / 32, "up_weight_scale"); want(gate_weight_scale, kL * kH / 32, "gate_weight_scale");
    want(down_weight_scale, kH * kL / 32, "down_weight_scale");
    if (post_ff_rms_weight) want(*post_ff_rms_weight, kH, "post_ff_rms_weight");
    if (layer_scalar) want(*layer_scalar, 8, "layer_scalar");
    device.make_current();
    check(moa_decoder_feedforward_mxfp4(u16(residual_hbm), u16(pre_ff_rms_weight), u8(up_weight_packed),
                                        u8(gate_weight_packed), u8(down_weight_packed), u8(up_weight_scale),
                                        u8(gate_weight_scale), u8(down_weight_scale), opt_u16(post_ff_rms_weight),
                                        opt_u16(layer_scalar), M, device.stream()),
          "decoder_feedforward_mxfp4");
}

// sliding_attention_output then decoder_feedforward on one residual (the tail of the runtime's
// sliding-layer step, FO/src/host/runtime.rs:440-459 then 543-571), with the reference's operand
// types: the same bits as the two calls in turn, one launch for a token row.
inline void sliding_attention_output_feedforward(
    const Device& device, const HbmTensor<bf16>& x, const HbmTensor<bf16>& post_attn_rms_weight,
    const HbmTensor<f8e4m3>& o_weight, const HbmTensor<bf16>& o_weight_scale, HbmTensor<bf16>& residual_hbm,
    const HbmTensor<bf16>& pre_ff_rms_weight, const HbmTensor<f4e2m1x2>& up_weight_packed,
    const HbmTensor<f4e2m1x2>& gate_weight_packed, const HbmTensor<f4e2m1x2>& down_weight_packed,
    const HbmTensor<f8e4m3>& up_weight_scale, const HbmTensor<f8e4m3>& gate_weight_scale,
    const HbmTensor<f8e4m3>& down_weight_scale, const HbmTensor<float>& up_global_scale,
    const HbmTensor<float>& gate_global_scale, const HbmTensor<float>& down_global_scale,
    const HbmTensor<bf16>& post_ff_rms_weight, const HbmTensor<bf16>& layer_scalar) {
    using namespace detail;
    const int M = rows(x, kQs, "x");
    want(post_attn_rms_weight, kH, "post_attn_rms_weight"); want(o_weight, kH * kQs, "o_weight");
    want(o_weight_scale, kH, "o_weight_scale"); want(residual_hbm, M * kH, "residual_hbm");
    want(pre_ff_rms_weight, kH, "pre_ff_rms_weight");
    want(up_weight_packed, kL * kH / 2, "up_weight_packed"); want(gate_weight_packed, kL * kH / 2, "gate_weight_packed");
    want(down_weight_packed, kH * kL / 2, "down_weight_packed");
    want(up_weight_scale, kL * kH / 16, "up_weight_scale"); want(gate_weight_scale, kL * kH / 16, "gate_weight_scale");
    want(down_weight_scale, kH * kL / 16, "down_weight_scale");
    want(up_global_scale, 1, "up_global_scale"); want(gate_global_scale, 1, "gate_global_scale");
    want(down_global_scale, 1, "down_global_scale");
    want(post_ff_rms_weight, kH, "post_ff_rms_weight"); want(layer_scalar, 8, "layer_scalar");
    device.make_current();
    check(moa_sliding_attention_output_feedforward(
              u16(x), u16(post_attn_rms_weight), u8(o_weight), u16(o_weight_scale), u16(residual_hbm),
              u16(pre_ff_rms_weight), u8(up_weight_packed), u8(gate_weight_packed), u8(down_weight_packed),
              u8(up_weight_scale), u8(gate_weight_scale), u8(down_weight_scale), up_global_scale.data(),
              gate_global_scale.data(), down_global_scale.data(), u16(post_ff_rms_weight), u16(layer_scalar), M,
              device.stream()),
          "sliding_attention_output_feedforward");
}

// ops::full_project_qkv -- FO/src/ops.rs:78-116 (one KV head of 512, a 512-slot page).
inline void full_project_qkv(const Device& device, const HbmTensor<bf16>& x, const HbmTensor<f8e4m3>& q_weight,
                             const HbmTensor<f8e4m3>& k_weight, const HbmTensor<bf16>& q_weight_scale,
                             const HbmTensor<bf16>& k_weight_scale, const HbmTensor<bf16>& input_rms_weight,
                             const HbmTensor<bf16>& q_rms_weight, const HbmTensor<bf16>& k_rms_weight,
                             const HbmTensor<int32_t>& kv_offset, const HbmTensor<int32_t>& rope_offset,
                             const HbmTensor<bf16>& cos, const HbmTensor<bf16>& sin, HbmTensor<bf16>& k_cache,
                             HbmTensor<bf16>& v_cache, HbmTensor<bf16>& q_out) {
    using namespace detail;
    const int M = rows(x, kH, "x");
    want(q_weight, kQf * kH, "q_weight"); want(k_weight, kPf * kH, "k_weight");
    want(q_weight_scale, kQf, "q_weight_scale"); want(k_weight_scale, kPf, "k_weight_scale");
    want(input_rms_weight, kH, "input_rms_weight"); want(q_rms_weight, kDf, "q_rms_weight");
    want(k_rms_weight, kDf, "k_rms_weight"); want(kv_offset, 1, "kv_offset"); want(rope_offset, 1, "rope_offset");
    want(cos, kE * kDf, "cos"); want(sin, kE * kDf, "sin");
    want(k_cache, kTf * kDf, "k_cache"); want(v_cache, kTf * kDf, "v_cache"); want(q_out, M * kGf * kDf, "q_out");
    device.make_current();
    check(moa_full_project_qkv(u16(x), u8(q_weight), u8(k_weight), u16(q_weight_scale), u16(k_weight_scale),
                               u16(input_rms_weight), u16(q_rms_weight), u16(k_rms_weight), kv_offset.data(),
                               rope_offset.data(), u16(cos), u16(sin), u16(k_cache), u16(v_cache), u16(q_out), M,
                               device.stream()),
          "full_project_qkv");
}

// ops::full_attention_first_page / ops::full_attention_page -- FO/src/ops.rs:148-174.
inline void full_attention_first_page(const Device& device, const HbmTensor<bf16>& q, const HbmTensor<bf16>& k,
                                      const HbmTensor<bf16>& v, const HbmTensor<float>& mask,
                                      HbmTensor<float>& running_max, HbmTensor<float>& running_sum,
                                      HbmTensor<bf16>& out_hbm) {
    using namespace detail;
    const int M = rows(q, kGf * kDf, "q");
    want(k, kTf * kDf, "k"); want(v, kTf * kDf, "v"); want(mask, M * kTf, "mask");
    want(running_max, M * kGf, "running_max"); want(running_sum, M * kGf, "running_sum");
    want(out_hbm, M * kGf * kDf, "out_hbm");
    device.make_current();
    check(moa_full_attention_first_page(u16(q), u16(k), u16(v), mask.data(), running_max.data(), running_sum.data(),
                                        u16(out_hbm), M, device.stream()),
          "full_attention_first_page");
}

inline void full_attention_page(const Device& device, const HbmTensor<bf16>& q, const HbmTensor<bf16>& k,
                                const HbmTensor<bf16>& v, const HbmTensor<float>& mask, HbmTensor<float>& running_max,
                                HbmTensor<float>& running_sum, HbmTensor<bf16>& out_hbm) {
    using namespace detail;
    const int M = rows(q, kGf * kDf, "q");
    want(k, kTf * kDf, "k"); want(v, kTf * kDf, "v"); want(mask, M * kTf, "mask");
    want(running_max, M * kGf, "running_max"); want(running_sum, M * kGf, "running_sum");
    want(out_hbm, M * kGf * kDf, "out_hbm");
    device.make_current();
    check(moa_full_attention_page(u16(q), u16(k), u16(v), mask.data(), running_max.data(), running_sum.data(),
                                  u16(out_hbm), M, device.stream()),
          "full_attention_page");
}

// ops::full_attention_output -- FO/src/ops.rs:176-199.
inline void full_attention_output(const Device& device, const HbmTensor<bf16>& x, const HbmTensor<float>& running_sum,
                                  const HbmTensor<bf16>& post_attn_rms_weight, const HbmTensor<f8e4m3>& o_weight,
                                  const HbmTensor<bf16>& o_weight_scale, HbmTensor<bf16>& residual_hbm) {
    using namespace detail;
    const int M = rows(x, kGf * kDf, "x");
    want(running_sum, M * kGf, "running_sum"); want(post_attn_rms_weight, kH, "post_attn_rms_weight");
    want(o_weight, kH * kQf, "o_weight"); want(o_weight_scale, kH, "o_weight_scale");
    want(residual_hbm, M * kH, "residual_hbm");
    device.make_current();
    check(moa_full_attention_output(u16(x), running_sum.data(), u16(post_attn_rms_weight), u8(o_weight),
                                    u16(o_weight_scale), u16(residual_hbm), M, device.stream()),
          "full_attention_output");
}

// ops::final_norm_and_logits -- FO/src/ops.rs:241-298.
inline void final_norm_and_logits(const Device& device, const HbmTensor<bf16>& input, const HbmTensor<bf16>& rms_weight,
                                  const HbmTensor<bf16>& lm_head_weight, HbmTensor<bf16>& out) {
    using namespace detail;
    const int M = rows(input, kH, "input");
    want(rms_weight, kH, "rms_weight"); want(lm_head_weight, kW * kH, "lm_head_weight"); want(out, M * kW, "out");
    device.make_current();
    check(moa_final_norm_and_logits(u16(input), u16(rms_weight), u16(lm_head_weight), u16(out), M, device.stream()),
          "final_norm_and_logits");
}

}  // namespace ops
}  // namespace moa

#endif  // MOA_OPS_HPP
