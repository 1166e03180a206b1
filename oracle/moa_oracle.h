/*
 * moa_oracle.h -- CPU restatement of the reference's algorithm for the Gemma-4-12B
 * decoder-layer hot path (QKV / attention-output / GeGLU FFN).
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: tests/, the smoke()
 * entry and bench.py's cpu_baseline leg call it. The product path (the HIP
 * library under moa-workspace_amd/) never links, loads or calls it.
 *
 * Every function cites the reference file:line it restates. Paths are relative
 * to the reference checkout; FO/ = furiosa-opt-gemma4-12B/.
 *
 * Numerical contract (FO/scripts/generate_references.py + FO/scripts/reference/gemma4.py):
 *   - bf16 values are stored as raw uint16 bits; bf16(v) is round-half-to-even of f32.
 *   - Each torch elementwise op on bf16 tensors computes in f32 and rounds to bf16.
 *   - Matrix products accumulate in f32.
 * The file is compiled with -ffp-contract=off so no multiply/add pair is fused
 * behind the restatement's back.
 *
 * Pinning status of each function (what checks it) is listed in oracle/README.md.
 */
#ifndef MOA_ORACLE_H
#define MOA_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- shapes (FO/src/axes.rs:3-29, FO/src/lib.rs:25) ---- */
enum {
    ORC_H = 3840, ORC_L = 15360, ORC_NS = 8, ORC_GS = 2, ORC_DS = 256,
    ORC_QS = 4096, ORC_PS = 2048, ORC_TS = 1024, ORC_E = 32768,
    ORC_GF = 16, ORC_DF = 512, ORC_QF = 8192, ORC_TF = 512 /* full-attention layers */
};
#define ORC_EPS 1e-6f

/* ---- formats ---- */
uint16_t orc_bf16_rne(float v);                 /* fixture_prng.py:80-90 (+NaN kept NaN) */
float    orc_bf16_to_f32(uint16_t b);
float    orc_e4m3_decode(uint8_t code);         /* E4M3FN, generate_references.py:152 (torch.float8_e4m3fn) */
uint8_t  orc_e4m3_encode_rne(float v);          /* RNE, saturating to +-448; NaN -> 0x7f */
float    orc_e2m1_decode(uint8_t nibble);       /* generate_references.py:69,154-163 */
uint8_t  orc_e2m1_encode_rne(float v);          /* RNE, saturating to +-6 */
float    orc_e8m0_decode(uint8_t e);            /* 2^(e-127); 0xff -> NaN (OCP MX) */

/* ---- reference PRNG (FO/scripts/fixture_prng.py:44-198 == FO/src/bin/test_kernels.rs:34-145) ---- */
uint64_t orc_name_hash(const char* name);                               /* fixture_prng.py:44-54 */
uint64_t orc_word(uint64_t seed, uint64_t index);                       /* fixture_prng.py:57-67 */
void orc_bf16_uniform(const char* name, size_t count, float lo, float hi, uint16_t* out); /* :94-103 */
void orc_f32_uniform(const char* name, size_t count, float lo, float hi, float* out);     /* :106-114 */
void orc_bf16_signs(const char* name, size_t count, float scale, uint16_t* out);         /* :115-125 */
void orc_f8_banded(const char* name, size_t count, int exp_min, int exp_max, int is_signed, uint8_t* out); /* :128-148 */
void orc_f4_nibbles(const char* name, size_t count, uint8_t* out_packed);               /* :151-166 */
uint32_t orc_checksum(const void* data, size_t nbytes);                                 /* :170-198 */
int orc_run_pos(int run);                                                               /* generate_references.py:79-90 */

/* cos/sin row for one position, f64 -> f32 (generate_references.py:184-197). Outputs f32. */
void orc_rope_row(int head_dim, double theta, double partial_rotary_factor, int pos,
                  float* cos_out, float* sin_out);

/* ---- primitives ---- */
/* gemma4.py:83-89: bf16((x * rsqrt(mean(x^2)+eps)) * w); w may be NULL (unweighted). One row of n. */
void orc_rmsnorm_row(const uint16_t* x, const uint16_t* w, int n, uint16_t* out);
/* torch gelu(approximate="tanh") on one f32 value (operator named at gemma4.py:197). */
float orc_gelu_tanh(float x);

/* generate_references.py:265-274: out[m,n] = bf16((f32(x[m,:]) . dec(W[n,:])) * f32(s[n])).
 * W is E4M3FN codes [N,K] row-major; scale f32 [N] (bf16 scales widen exactly). */
void orc_scaled_projection_fp8(const uint16_t* x, int M, int K, const uint8_t* w,
                               const float* scale, int N, uint16_t* out);

/* ---- the three operators (FO/src/ops.rs) ---- */

/* ops::sliding_project_qkv, FO/src/ops.rs:37-76; oracle generate_references.py:291-334.
 * x [M,3840] bf16; q/k/v weights E4M3 [4096|2048|2048, 3840]; scales f32 per row;
 * cos/sin: [E,256] bf16 tables as the kernel receives them (sin low half pre-negated,
 * generate_references.py:200-210); kv_offset/rope_offset are BYTE offsets for row 0
 * (FO/src/bin/test_kernels.rs:520-527); row m uses table row rope_offset/512 + m and
 * cache slot (kv_offset/4096 + m) mod 1024.  Writes q_out [M,16,256] and the K/V slots. */
void orc_sliding_project_qkv(const uint16_t* x, const uint8_t* q_w, const uint8_t* k_w,
                             const uint8_t* v_w, const float* q_s, const float* k_s,
                             const float* v_s, const uint16_t* in_rms, const uint16_t* q_rms,
                             const uint16_t* k_rms, int32_t kv_offset, int32_t rope_offset,
                             const uint16_t* cos_tab, const uint16_t* sin_tab,
                             uint16_t* k_cache, uint16_t* v_cache, uint16_t* q_out, int M);

/* ops::sliding_attention (FO/src/ops.rs:118-128): q, out [M][8][2][256] bf16; k, v [1024][8][256]
 * bf16; mask [M][1024] f32 (slot t takes part when mask != 0). */
void orc_sliding_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* mask,
                           uint16_t* out, int M);
/* ops::sliding_attention_output, FO/src/ops.rs:130-146; oracle generate_references.py:337-355.
 * x [M,4096]; o_w [3840,4096]; residual [M,3840] updated in place. */
void orc_sliding_attention_output(const uint16_t* x, const uint16_t* post_rms, const uint8_t* o_w,
                                  const float* o_s, uint16_t* residual, int M);

/* ops::full_project_qkv (FO/src/ops.rs:78-116; gemma4.py:152-166 with attention_k_eq_v):
 * x [M,3840]; q_w [8192,3840], k_w [512,3840] E4M3 with f32 row scales; q_rms, k_rms [512];
 * cos/sin [E][512] (sin's low half negated). Row m: q_out [M][16][512]; slot kv_offset/1024 + m
 * of the page gets K = RoPE(RMSNorm(k_raw, k_rms)) in k_page and V = RMSNorm(k_raw) in v_page
 * ([512][512] each); RoPE row rope_offset/1024 + m. */
void orc_full_project_qkv(const uint16_t* x, const uint8_t* q_w, const uint8_t* k_w, const float* q_s,
                          const float* k_s, const uint16_t* in_rms, const uint16_t* q_rms, const uint16_t* k_rms,
                          int32_t kv_offset, int32_t rope_offset, const uint16_t* cos_tab, const uint16_t* sin_tab,
                          uint16_t* k_page, uint16_t* v_page, uint16_t* q_out, int M);
/* The running state of full_attention_first_page + full_attention_page over P pages
 * (FO/src/ops.rs:148-174) computed at once in f64: the softmax of the CPU reference (gemma4.py:
 * 180-184, scale 1.0) over the valid slots (mask != 0). q [M][16][512]; k_pages, v_pages
 * [P][512][512]; masks [P][M][512]. running_max / running_sum [M][16]: the largest valid score
 * and sum of exp(s - max); out [M][16][512] = bf16(sum of exp(s - max) v). No valid slot: -inf,
 * 0 and zeros. */
void orc_full_attention_pages(const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages,
                              const float* masks, int P, float* running_max, float* running_sum, uint16_t* out,
                              int M);
/* ops::full_attention_output (FO/src/ops.rs:176-199): x' = bf16(x / running_sum[head]) (0 for a
 * zero sum), then as sliding_attention_output with K = 8192: residual += RMSNorm(bf16(x'.W_o^T * s)). */
void orc_full_attention_output(const uint16_t* x, const float* running_sum, const uint16_t* post_rms,
                               const uint8_t* o_w, const float* o_s, uint16_t* residual, int M);

/* Gemma's final-logit softcap of a bf16 logit l (FO/src/ops.rs:256-293; gemma4.py:260-261):
 * tanh(l / 30) * 30 in f64, rounded once to bf16. */
uint16_t orc_softcap30(uint16_t l);
/* ops::final_norm_and_logits (FO/src/ops.rs:241-298): RMSNorm of each input row, the bf16 linear
 * over the W rows of lm_head given ([W][3840], any run of vocabulary rows), then the softcap.
 * x [M][3840]; out [M][W]. */
void orc_final_norm_and_logits(const uint16_t* x, const uint16_t* rms_w, const uint16_t* lm_head, int W,
                               uint16_t* out, int M);

/* ops::decoder_feedforward, FO/src/ops.rs:201-239; oracle generate_references.py:375-414.
 * Weight format selects the projection rule:
 *   ORC_FFN_NVFP4: packed e2m1 [N,K/2] + e4m3 block-16 scales [N,K/16] + f32 reciprocal global;
 *                  proj = bf16(bf16(h.W) * inv_g)               (GloballyScaled, :358-372)
 *   ORC_FFN_FP8:   e4m3 [N,K] + f32 per-row scale; proj = bf16((h.W) * s_row)  (scaled_projection)
 *   ORC_FFN_MXFP4: packed e2m1 [N,K/2] + e8m0 block-32 scales [N,K/32]; proj = bf16(h.W)
 * post_rms / layer_scalar may be NULL (skip the post-FF norm / the gate multiply). */
enum { ORC_FFN_NVFP4 = 0, ORC_FFN_FP8 = 1, ORC_FFN_MXFP4 = 2 };
typedef struct {
    int format;
    const uint8_t* up;   const uint8_t* gate;   const uint8_t* down;
    const void* up_scale; const void* gate_scale; const void* down_scale; /* u8 codes or f32 */
    float up_inv_global, gate_inv_global, down_inv_global;             /* NVFP4 only */
} orc_ffn_weights;

void orc_decoder_feedforward(uint16_t* residual, const uint16_t* pre_rms, const orc_ffn_weights* w,
                             const uint16_t* post_rms, const uint16_t* layer_scalar, int M);

/* GeGLU projection pieces, exposed for tests: h [M,3840] -> p [M,15360] (bf16), and
 * p -> d [M,3840] (bf16) using the same projection rule as above. */
void orc_ffn_up_gate(const uint16_t* h, const orc_ffn_weights* w, uint16_t* p, int M);
void orc_ffn_down(const uint16_t* p, const orc_ffn_weights* w, uint16_t* d, int M);

/* OpenMP threads used by the heavy loops (0 = runtime default). Returns the count in effect. */
int orc_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
