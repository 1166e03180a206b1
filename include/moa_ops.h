/*
 * moa_ops.h -- C ABI of the MI355X (gfx950) decoder-layer hot path.
 *
 * Drop-in for the three Stage-1 operators of the reference crate
 * (furiosa-opt-gemma4-12B, "FO/" below). Each entry point keeps the argument order and
 * meaning of the reference's `#[device] fn` in FO/src/ops.rs, with the `device` handle
 * replaced by a trailing (M, stream) pair:
 *   - every tensor is a caller-owned device pointer (hipMalloc'd); the library never
 *     allocates per call (one per-device scratch block is made on first use or by moa_init);
 *   - `&mut` tensors of the reference (k_cache, v_cache, q_out, residual) are written in place;
 *   - bf16 tensors are raw uint16 bit patterns; E4M3FN/E2M1/E8M0 are uint8 codes;
 *   - M is the number of token rows (the reference processes exactly one, M = 1);
 *   - stream is a hipStream_t (NULL = the null stream); all work is ordered on it and the
 *     call returns without synchronising. Calls on one device must be issued from one
 *     stream at a time: the per-device scratch is shared.
 *   - the call is served by the scratch of the calling thread's current device (hipSetDevice),
 *     so the stream and every tensor must belong to that device.
 * Pointers must be 16-byte aligned except per-channel scales (natural alignment) and FP4
 * block-scale codes (4-byte aligned).
 *
 * Return value: MOA_SUCCESS or a negative MOA_ERROR_* code; moa_last_error_string() gives
 * the reason. Invalid arguments are rejected before anything is launched. Device-resident
 * offsets are validated by the kernel: a token row whose RoPE row or ring slot is out of range
 * writes nothing (the call's other rows are written) and raises a bit read back by
 * moa_device_errors().
 *
 * Shapes (FO/src/axes.rs:3-29): H=3840 hidden, L=15360 intermediate, 8 KV heads x 2 query
 * heads x 256 head_dim (Q=4096, K/V=2048), ring cache T=1024 slots, RoPE table E=32768 rows.
 */
#ifndef MOA_OPS_H
#define MOA_OPS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOA_SUCCESS 0
#define MOA_ERROR_INVALID_VALUE (-1) /* null pointer, bad M or shape */
#define MOA_ERROR_MISALIGNED (-2)    /* pointer not 16-byte aligned */
#define MOA_ERROR_HIP (-3)           /* a HIP runtime call failed */
#define MOA_ERROR_NO_DEVICE (-4)     /* no usable gfx950 device */
#define MOA_ERROR_DEVICE_STATE (-5)  /* a kernel flagged a bad device-resident argument, or the
                                        device's state is tripped (see moa_clear_device_state) */

#define MOA_DEVERR_ROPE_OFFSET 1u /* rope_offset not a multiple of 512 or past the table */
#define MOA_DEVERR_KV_OFFSET 2u   /* kv_offset not a multiple of 4096 or past the ring */
#define MOA_DEVERR_SPIN_TIMEOUT 4u /* a bounded cross-workgroup wait of a one-token call expired
                                      (another process held the CUs). The workgroups whose wait
                                      expired store nothing: with the post-norm, the residual rows
                                      behind an expired leader keep their input values, but rows of
                                      other leaders may hold the result, so restore the outputs
                                      from a copy before calling again. Once moa_device_errors has
                                      returned this bit, the device's state is tripped: every call
                                      that computes on it, and moa_init, return
                                      MOA_ERROR_DEVICE_STATE until moa_clear_device_state. */

/* Library version string. */
const char* moa_version(void);

/* Reason for the last non-zero return on this thread. */
const char* moa_last_error_string(void);

/* Allocates the per-device scratch of `device` (also done lazily by the first call) and sets up
 * the static scratch of moa_decoder_feedforward_fp8_noalloc. Call it before capturing calls into
 * a HIP graph. A caller that cannot allocate skips it: the no-allocation entry point sets itself
 * up on its first call without allocating. */
int moa_init(int device);

/* Synchronises `stream`, returns the OR of device-side error bits raised since the last call
 * (MOA_DEVERR_*) in *bits, and clears them. Reads the error word of each scratch that exists on
 * the current device and creates none, so it allocates nothing. MOA_DEVERR_SPIN_TIMEOUT among
 * the bits trips the device's state (see below). */
int moa_device_errors(void* stream, uint32_t* bits);

/* No counterpart in the reference, whose operators cannot fail (FO/src/bin/test_kernels.rs:536
 * unwraps). Acknowledges a tripped state of `device` -- a one-token call's wait expired and the
 * caller has restored that call's outputs -- so that calls compute again. Returns MOA_SUCCESS
 * whether or not the state was tripped. */
int moa_clear_device_state(int device);

/* ops::sliding_project_qkv -- FO/src/ops.rs:37-76.
 * x bf16 [M,3840]; q_weight E4M3 [4096,3840]; k_weight, v_weight E4M3 [2048,3840] (row =
 * output channel); *_weight_scale f32 per output channel; input_rms_weight bf16 [3840];
 * q_rms_weight, k_rms_weight bf16 [256]; kv_offset, rope_offset: device int32 BYTE offsets
 * for row 0 (slot*8*256*2 and pos*256*2, FO/src/bin/test_kernels.rs:520-527); row m uses
 * table row rope_offset/512+m and ring slot (kv_offset/4096+m) mod 1024; cos, sin bf16
 * [32768,256] (sin with its low half negated, FO/scripts/generate_references.py:200-210);
 * k_cache, v_cache bf16 [1024,8,256] (only the addressed slots are written); q_out bf16
 * [M,8,2,256]. */
int moa_sliding_project_qkv(const uint16_t* x, const uint8_t* q_weight, const uint8_t* k_weight,
                            const uint8_t* v_weight, const float* q_weight_scale,
                            const float* k_weight_scale, const float* v_weight_scale,
                            const uint16_t* input_rms_weight, const uint16_t* q_rms_weight,
                            const uint16_t* k_rms_weight, const int32_t* kv_offset,
                            const int32_t* rope_offset, const uint16_t* cos, const uint16_t* sin,
                            uint16_t* k_cache, uint16_t* v_cache, uint16_t* q_out, int M,
                            void* stream);

/* Same with bf16 per-channel scales, the exact operand types of FO/src/ops.rs:44-46. */
int moa_sliding_project_qkv_bf16_scales(
    const uint16_t* x, const uint8_t* q_weight, const uint8_t* k_weight, const uint8_t* v_weight,
    const uint16_t* q_weight_scale, const uint16_t* k_weight_scale, const uint16_t* v_weight_scale,
    const uint16_t* input_rms_weight, const uint16_t* q_rms_weight, const uint16_t* k_rms_weight,
    const int32_t* kv_offset, const int32_t* rope_offset, const uint16_t* cos, const uint16_t* sin,
    uint16_t* k_cache, uint16_t* v_cache, uint16_t* q_out, int M, void* stream);

/* ops::sliding_attention -- FO/src/ops.rs:118-128 (the step between QKV and O).
 * q bf16 [M,8,2,256] (query heads after head norm and RoPE, the q_out of sliding_project_qkv);
 * k, v bf16 [1024,8,256] (the ring caches); mask f32 [M,1024] (one row per token row: slot t takes
 * part when mask[t] != 0, as the runtime's 1.0 / 0.0 rows do, FO/src/host/runtime.rs:160);
 * out bf16 [M,8,2,256] = softmax over the valid slots of (q . k_t) (scale 1.0) times v
 * (FO/scripts/reference/gemma4.py:163-186). A row with no valid slot gives zeros. */
int moa_sliding_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* mask,
                          uint16_t* out, int M, void* stream);

/* ops::sliding_attention_output -- FO/src/ops.rs:130-146.
 * x bf16 [M,4096] (= [M,8,2,256]); post_attn_rms_weight bf16 [3840]; o_weight E4M3
 * [3840,4096]; o_weight_scale f32 [3840]; residual bf16 [M,3840], updated in place:
 * residual = bf16(residual + RMSNorm(bf16((x.W^T) * scale), post_attn_rms_weight)). */
int moa_sliding_attention_output(const uint16_t* x, const uint16_t* post_attn_rms_weight,
                                 const uint8_t* o_weight, const float* o_weight_scale,
                                 uint16_t* residual, int M, void* stream);

/* Same with bf16 scales (FO/src/ops.rs:136). */
int moa_sliding_attention_output_bf16_scales(const uint16_t* x, const uint16_t* post_attn_rms_weight,
                                             const uint8_t* o_weight, const uint16_t* o_weight_scale,
                                             uint16_t* residual, int M, void* stream);

/* ops::decoder_feedforward -- FO/src/ops.rs:201-239, NVFP4 weights exactly as the reference:
 * *_weight_packed E2M1 two per byte, low nibble first (up/gate [15360,1920], down [3840,7680]);
 * *_weight_scale E4M3 per 16 K-elements (up/gate [15360,240], down [3840,960]);
 * *_global_scale device f32 [1] holding the RECIPROCAL global scale (FO/src/host/load.rs:170-190);
 * pre/post_ff_rms_weight bf16 [3840]; layer_scalar bf16 [8] (element 0 used);
 * residual bf16 [M,3840] updated in place. */
int moa_decoder_feedforward(uint16_t* residual, const uint16_t* pre_ff_rms_weight,
                            const uint8_t* up_weight_packed, const uint8_t* gate_weight_packed,
                            const uint8_t* down_weight_packed, const uint8_t* up_weight_scale,
                            const uint8_t* gate_weight_scale, const uint8_t* down_weight_scale,
                            const float* up_global_scale, const float* gate_global_scale,
                            const float* down_global_scale, const uint16_t* post_ff_rms_weight,
                            const uint16_t* layer_scalar, int M, void* stream);

/* GeGLU FFN with FP8 E4M3 weights and per-output-channel f32 scales (no counterpart in the
 * reference's weights; same operator contract as FO/src/ops.rs:201-239 with each projection
 * computed as FO/scripts/generate_references.py:265-274 scaled_projection).
 * up, gate E4M3 [15360,3840]; down E4M3 [3840,15360]; scales f32 [15360],[15360],[3840].
 * post_ff_rms_weight and layer_scalar may be NULL (skip the post norm / the gate). */
int moa_decoder_feedforward_fp8(uint16_t* residual, const uint16_t* pre_ff_rms_weight,
                                const uint8_t* up_weight, const uint8_t* gate_weight,
                                const uint8_t* down_weight, const float* up_weight_scale,
                                const float* gate_weight_scale, const float* down_weight_scale,
                                const uint16_t* post_ff_rms_weight, const uint16_t* layer_scalar,
                                int M, void* stream);

/* No counterpart in the reference: for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The same operator as
 * moa_decoder_feedforward_fp8, the same kernels and the same bits, for 1 <= M <= 16 rows (larger
 * M is rejected with MOA_ERROR_INVALID_VALUE). Its scratch (about 1.9 MB: epoch counters,
 * hand-off words, normalised rows, GeGLU rows, down partial sums) is a static device array that
 * each GPU holds until the process ends; neither this call nor its set-up (done by its first
 * call on a device) allocates, and moa_device_errors reads its error bits without allocating. Every call on one device shares that array and it keeps the
 * last call's contents: calls that overlap on one device (different streams, no dependency)
 * race. Independent of the scratch of the other entry points. */
int moa_decoder_feedforward_fp8_noalloc(uint16_t* residual, const uint16_t* pre_ff_rms_weight,
                                        const uint8_t* up_weight, const uint8_t* gate_weight,
                                        const uint8_t* down_weight, const float* up_weight_scale,
                                        const float* gate_weight_scale, const float* down_weight_scale,
                                        const uint16_t* post_ff_rms_weight, const uint16_t* layer_scalar,
                                        int M, void* stream);

/* GeGLU FFN with MXFP4 weights: E2M1 two per byte (as NVFP4) with E8M0 scales per 32
 * K-elements (up/gate [15360,120], down [3840,480]); no global scale. Same contract
 * otherwise; post_ff_rms_weight and layer_scalar may be NULL. */
int moa_decoder_feedforward_mxfp4(uint16_t* residual, const uint16_t* pre_ff_rms_weight,
                                  const uint8_t* up_weight_packed, const uint8_t* gate_weight_packed,
                                  const uint8_t* down_weight_packed, const uint8_t* up_weight_scale,
                                  const uint8_t* gate_weight_scale, const uint8_t* down_weight_scale,
                                  const uint16_t* post_ff_rms_weight, const uint16_t* layer_scalar,
                                  int M, void* stream);

/* The tail of the reference's sliding-layer decode step, FO/src/host/runtime.rs:440-459 (the
 * ops::sliding_attention_output launch) followed by 543-571 (the ops::decoder_feedforward launch of
 * mlp) on the same residual: O projection, post-attention norm and residual add (FO/src/ops.rs:130-146),
 * then the GeGLU FFN (FO/src/ops.rs:201-239), with the reference's operand types (bf16 O scales,
 * NVFP4 FFN weights). Arguments are those of moa_sliding_attention_output_bf16_scales followed by
 * those of moa_decoder_feedforward after its residual. The residual afterwards has the same bits
 * as those two calls made in turn; at M = 1 it is one launch (the residual between the two
 * operators is never written to memory), and from 3 rows on O's last kernel also writes the FFN's
 * normalised input (one kernel fewer). */
int moa_sliding_attention_output_feedforward(
    const uint16_t* x, const uint16_t* post_attn_rms_weight, const uint8_t* o_weight, const uint16_t* o_weight_scale,
    uint16_t* residual, const uint16_t* pre_ff_rms_weight, const uint8_t* up_weight_packed,
    const uint8_t* gate_weight_packed, const uint8_t* down_weight_packed, const uint8_t* up_weight_scale,
    const uint8_t* gate_weight_scale, const uint8_t* down_weight_scale, const float* up_global_scale,
    const float* gate_global_scale, const float* down_global_scale, const uint16_t* post_ff_rms_weight,
    const uint16_t* layer_scalar, int M, void* stream);

/* The same with BASELINE's operand types: f32 O scales and the FP8 FFN of
 * moa_decoder_feedforward_fp8 (post_ff_rms_weight and layer_scalar may be NULL). The same bits as
 * moa_sliding_attention_output then moa_decoder_feedforward_fp8. */
int moa_sliding_attention_output_feedforward_fp8(
    const uint16_t* x, const uint16_t* post_attn_rms_weight, const uint8_t* o_weight, const float* o_weight_scale,
    uint16_t* residual, const uint16_t* pre_ff_rms_weight, const uint8_t* up_weight, const uint8_t* gate_weight,
    const uint8_t* down_weight, const float* up_weight_scale, const float* gate_weight_scale,
    const float* down_weight_scale, const uint16_t* post_ff_rms_weight, const uint16_t* layer_scalar, int M,
    void* stream);

/* The same with f32 O scales and the MXFP4 FFN of moa_decoder_feedforward_mxfp4. */
int moa_sliding_attention_output_feedforward_mxfp4(
    const uint16_t* x, const uint16_t* post_attn_rms_weight, const uint8_t* o_weight, const float* o_weight_scale,
    uint16_t* residual, const uint16_t* pre_ff_rms_weight, const uint8_t* up_weight_packed,
    const uint8_t* gate_weight_packed, const uint8_t* down_weight_packed, const uint8_t* up_weight_scale,
    const uint8_t* gate_weight_scale, const uint8_t* down_weight_scale, const uint16_t* post_ff_rms_weight,
    const uint16_t* layer_scalar, int M, void* stream);

/* ops::final_norm_and_logits -- FO/src/ops.rs:241-298 (oracle gemma4.py:256-261).
 * input bf16 [M,3840]; rms_weight bf16 [3840]; lm_head_weight bf16 [262144,3840]; out bf16
 * [M,262144] = bf16(tanh(l / 30) * 30) in f32, l = bf16(RMSNorm(input) . W_v). */
int moa_final_norm_and_logits(const uint16_t* input, const uint16_t* rms_weight, const uint16_t* lm_head_weight,
                              uint16_t* out, int M, void* stream);

/* ---- full-attention layers (every sixth layer): 16 query heads and one KV head of 512, a
 * cache of 512-slot pages (FO/src/axes.rs: Gf=16, Df=512, Qf=8192, Pf=512, Tf=512). ---- */

/* ops::full_project_qkv -- FO/src/ops.rs:78-116 (oracle gemma4.py:152-166, attention_k_eq_v).
 * x bf16 [M,3840]; q_weight E4M3 [8192,3840], k_weight E4M3 [512,3840] with bf16 per-row
 * scales; q_rms_weight, k_rms_weight bf16 [512]; cos/sin bf16 [32768,512] (sin's low half
 * negated). Row m: q_out[m] = RoPE(RMSNorm_q(q)) [16,512]; of the raw K projection, the page's
 * slot kv_offset/1024 + m gets K = RoPE(RMSNorm_k(k)) in k_cache [512,512] and the unweighted
 * norm V = RMSNorm(k) in v_cache [512,512]. RoPE row rope_offset/1024 + m. A row whose slot
 * falls past the page writes nothing and raises MOA_DEVERR_KV_OFFSET. */
int moa_full_project_qkv(const uint16_t* x, const uint8_t* q_weight, const uint8_t* k_weight,
                         const uint16_t* q_weight_scale, const uint16_t* k_weight_scale,
                         const uint16_t* input_rms_weight, const uint16_t* q_rms_weight, const uint16_t* k_rms_weight,
                         const int32_t* kv_offset, const int32_t* rope_offset, const uint16_t* cos, const uint16_t* sin,
                         uint16_t* k_cache, uint16_t* v_cache, uint16_t* q_out, int M, void* stream);

/* ops::full_attention_first_page / ops::full_attention_page -- FO/src/ops.rs:148-174
 * (FO/src/device/full/attention.rs:203-329). q bf16 [M,16,512]; one page's k, v bf16 [512,512];
 * mask f32 [M,512] (slot t takes part when non-zero); the running state running_max,
 * running_sum f32 [M,16] and out bf16 [M,16,512] (un-normalised: sum of exp(s - max) v).
 * first_page starts the state from this page; page folds this page into it (the old state is
 * rescaled by exp(old max - new max)). Scores use scale 1.0. A head with no valid slot so far
 * has max -inf, sum 0 and out 0. */
int moa_full_attention_first_page(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* mask,
                                  float* running_max, float* running_sum, uint16_t* out, int M, void* stream);
int moa_full_attention_page(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* mask,
                            float* running_max, float* running_sum, uint16_t* out, int M, void* stream);

/* The state that full_attention_first_page followed by full_attention_page over pages 1 .. P-1
 * leaves, in two launches whatever P is (no counterpart in the reference, whose runtime launches
 * one operator per page, FO/src/host/runtime.rs:496-517). k_pages, v_pages bf16 [P,512,512]
 * contiguous (page p at p * 512 * 512); masks f32 [P,M,512]; 1 <= P <= 64. Same outputs and
 * meaning as the per-page calls. */
int moa_full_attention(const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages, const float* masks, int P,
                       float* running_max, float* running_sum, uint16_t* out, int M, void* stream);

/* ops::full_attention_output -- FO/src/ops.rs:176-199. x bf16 [M,16,512] (the pages' out),
 * running_sum f32 [M,16]; residual bf16 [M,3840] updated in place:
 * r = bf16(r + RMSNorm(bf16(bf16(x / sum) . W_o) * s)) with o_weight E4M3 [3840,8192] and bf16
 * per-row scales (a zero sum gives a zero attention row). */
int moa_full_attention_output(const uint16_t* x, const float* running_sum, const uint16_t* post_attn_rms_weight,
                              const uint8_t* o_weight, const uint16_t* o_weight_scale, uint16_t* residual, int M,
                              void* stream);

/* The FP8 projection alone -- FO/scripts/generate_references.py:265-274 scaled_projection:
 * out[m,n] = bf16((x[m,:] . dec(w[n,:])) * scale[n]). x bf16 [M,K], w E4M3 [N,K], scale f32
 * [N], out bf16 [M,N]; K % 16 == 0. */
int moa_fp8_scaled_projection(const uint16_t* x, const uint8_t* w, const float* scale, uint16_t* out,
                              int M, int N, int K, void* stream);

/* Test support: decodes every E4M3 code, E2M1 byte, E8M0 code, bf16 GeLU input and bf16
 * final-logit softcap input, and rounds f32 values of every bf16 high half to bf16, with the
 * kernels' own device helpers into out (device uint32 [721924]; layout in moa_decode.hip). */
int moa_format_selftest(uint32_t* out, void* stream);

/* Test support for the launch epochs of the one-launch kernels (no counterpart in the reference).
 * The one-token QKV (kernel 0), O (1) and FFN (2) kernels and the FFN of 2..16 rows (3) tag their
 * cross-workgroup hand-off words with a per-launch tag derived from 64-bit epoch counters that
 * `per` workgroups of each launch advance by one. moa_test_epoch_layout gives the number of counters and `per`;
 * moa_test_epoch_tag computes, on the host, the tag a workgroup derives from the value `old` its
 * add returned (the same function the kernels run). Neither touches a device. */
int moa_test_epoch_layout(int kernel, int* counters, int* per);
int moa_test_epoch_tag(int kernel, uint64_t old, uint32_t* tag);

/* Test support: sets every epoch counter of the current device as if `launches` launches of each
 * one-launch kernel had run (counter = launches * per), and the sliding-attention tickets to
 * (launches * 32) mod 2^32, so that a test can cross counter wrap points without running
 * billions of launches. Synchronous; no call may be in flight on the device. */
int moa_test_preset_epochs(uint64_t launches);

/* Test support for the waits of the one-token QKV, O and FFN kernels (no counterpart in the
 * reference). A workgroup that has waited steal_ticks (100 MHz wall-clock ticks; 50000 by
 * default) for another workgroup of its launch computes that workgroup's share itself, so a call
 * completes with the same bits whether or not its whole grid is resident. With hold_ticks > 0,
 * workgroups hold[0..3] (-1: none) of every later launch wait hold_ticks at entry, before they read
 * or write anything -- as if they had been started late. Applies to calls issued after it;
 * steal_ticks 0 restores the defaults (no hold). */
int moa_test_set_stall(uint32_t steal_ticks, uint32_t hold_ticks, const int32_t* hold);

/* Test support (no counterpart in the reference): with on == 0, later decoder_feedforward calls of
 * 2..16 rows (and the rows path of sliding_attention_output_feedforward) run the up/gate and the
 * down contractions as two launches instead of one, so that a test can compare the two (they give
 * the same bits); on != 0 restores the default, one launch where its grid fits on the device. */
int moa_test_set_rows_one_launch(int on);

/* Test support: the number of take-overs (a wait that did another workgroup's share) on the
 * current device since the last call, in the scratch of every entry point that has run there
 * (the no-allocation entry point's included), then resets it. Synchronises the device. */
int moa_test_take_overs(uint32_t* count);

/* Test support: which scratch exists on the current device, without creating either: bit 0 the
 * hipMalloc'd scratch of the ordinary entry points, bit 1 the static scratch of
 * moa_decoder_feedforward_fp8_noalloc. Touches no device memory. */
int moa_test_scratch_state(uint32_t* state);

/* Test only: trips the state of `device` as a MOA_DEVERR_SPIN_TIMEOUT read by moa_device_errors
 * does (no device needed), so the refusal path can be tested where no wait expires. */
int moa_test_trip_device_state(int device);

#ifdef __cplusplus
}
#endif
#endif
