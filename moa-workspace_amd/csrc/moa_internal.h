// moa_internal.h -- host-side declarations shared by the C-ABI and the kernel launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "moa_shapes.h"

namespace moa {

// Rows handled by the decode (GEMV) kernels in one launch; larger M goes to the MFMA path.
constexpr int kMaxDecodeM = 16;
// Calls of at least this many rows (and at most kMaxDecodeM) run QKV and O, sliding and full, on
// the matrix-core rows path (moa_rows.hip), which reads the weights once instead of once per row
// (full-attention O from two rows). At two rows the per-row kernels are as fast.
constexpr int kRowsProjMinM = 3;
// Rows handled by one call of the MFMA (M > kMaxDecodeM) path; larger calls are tiled by the host.
constexpr int kMaxChunkM = 1024;
// QKV projection rows (Q | K | V).
constexpr int kQkvRowsTotal = kQs + 2 * kPs;
// f32 split-K partial sums of the MFMA path: splits x M x N never exceeds one chunk of QKV columns
constexpr size_t kChunkPartFloats = (size_t)kMaxChunkM * kQkvRowsTotal;

// Arrival counters. Each counter owns a 256-byte line: device-scope atomics to one line
// serialise (~15 ns each), so counters never share a line and each kernel arrives once per
// workgroup. Layout (in counters): [0, 32*kMaxDecodeM) QKV per (row, head);
// then per row a 17-counter tree (16 leaves + 1 root) for O.
constexpr int kTicketStride = 64;  // uint32 per counter (256 bytes)
constexpr int kTreeLeaves = 16;
constexpr int kTreeCounters = kTreeLeaves + 1;
constexpr int kTicketQkv = 0;
constexpr int kTicketO = kTicketQkv + 32 * kMaxDecodeM;
// 64-bit epoch counters of the single-launch O (15 counters of 16 workgroups), QKV (one per head,
// 8 workgroups) and FFN (15 of 16) kernels: monotonic, never reset; a workgroup adds one at entry
// and divides what it read by the workgroups per counter (epoch_tag, moa_sync.h).
constexpr int kTicketOEpoch = kTicketO + kTreeCounters * kMaxDecodeM;
constexpr int kTicketQkvEpoch = kTicketOEpoch + 16;
constexpr int kTicketFfnEpoch = kTicketQkvEpoch + 32;
constexpr int kOEpochCounters = 15, kOEpochPer = 16;
constexpr int kQkvEpochCounters = 32, kQkvEpochPer = 8;
constexpr int kFfnEpochCounters = 15, kFfnEpochPer = 16;
// sliding_attention: one counter per (row, head) of a launch, 32 arrivals per launch, never reset
constexpr int kTicketRowsEpoch = kTicketFfnEpoch + 16;  // the one-launch rows FFN (16 of 16)
constexpr int kRowsEpochCounters = 16, kRowsEpochPer = 16;
constexpr int kTicketAttn = kTicketRowsEpoch + 16;
constexpr int kTicketCount = kTicketAttn + kMaxDecodeM * kNs;
// sliding_attention partials: [kMaxDecodeM][kNs][32 chunks][kGs][max, sum, o[kDs]]
constexpr size_t kAttnPartFloats = (size_t)kMaxDecodeM * kNs * 32 * kGs * (4 + kDs);
// full-attention page partials: per token row and 64-slot chunk, 16 maxima, 16 sums, out [16][512]
constexpr int kFaChunks = 8;
constexpr int kFaDimBlocks = 4;
constexpr int kFaRec = 2 * kGf + kGf * kDf;
constexpr int kFaMaxRecords = 256;                        // records per row of the fused pass
constexpr int kFaSplitPages = 8;                           // the fused pass splits dims up to 8 pages
constexpr int kFattnRecords = 256;                         // records of scratch (>= kMaxDecodeM * kFaChunks)
constexpr size_t kFattnPartFloats = (size_t)kFattnRecords * kFaRec;

// Tagged hand-off words of the single-launch FFN (per workgroup a partial sum, 8 output words and
// a claim word; never shared with another kernel).
constexpr int kFfnPartSlots = 256;
constexpr int kFfnSlotWords = kFfnPartSlots * 10;
constexpr int kQkvSlotWords = 32 * 8;
constexpr int kOfnCopies = 8;  // copies of O's post-norm words in the single-launch O -> FFN kernel
// Tagged flags of the one-launch rows FFN (moa_rows.hip rows_fused_kernel): one per GeGLU block,
// one per block of down partial sums, one per normalised row.
constexpr int kRowsFlagWords = 512;

// Device-side error bits (OR-ed by kernels; read back by moa_device_errors()).
constexpr uint32_t kErrRopeOffset = 1u;
constexpr uint32_t kErrKvOffset = 2u;
constexpr uint32_t kErrSpinTimeout = 4u;
constexpr int kErrTakeOvers = 1;  // err[1]: waits of the one-token kernels that took work over (tests)

// Per-device persistent scratch, allocated once on first use (never per call).
struct DevCtx {
    int device = -1;
    uint32_t* tickets = nullptr;  // kTicketCount * kTicketStride, zero between calls (self-resetting)
    uint32_t* err = nullptr;      // 4 words
    uint16_t* raw_qkv = nullptr;  // [kMaxChunkM, 8192] bf16 raw projections
    uint16_t* pbuf = nullptr;     // [kMaxChunkM, 15360] bf16 (O: [M,3840]; FFN: GeGLU output)
    uint16_t* hbuf = nullptr;     // [kMaxChunkM, 3840] bf16 (normalised activations, MFMA path)
    float* fbuf = nullptr;        // [splits][M][N] f32 split-K partial sums (MFMA path), kChunkPartFloats
    uint64_t* ffn_part = nullptr;  // tagged hand-off words of the single-launch FFN (kFfnSlotWords)
    uint64_t* ffn_ptag = nullptr;  // [kL / 2] tagged GeGLU pairs of the single-launch FP8 FFN (only it writes them)
    uint64_t* o_part = nullptr;   // the same for the single-launch O (kFfnSlotWords)
    uint64_t* ofn_part = nullptr; // O's post-norm words of the single-launch O -> FFN (kOfnCopies x kFfnSlotWords)
    uint64_t* qkv_part = nullptr; // tagged per-head partial sums of the single-launch QKV (kQkvSlotWords)
    uint64_t* rows_flag = nullptr; // tagged flags of the one-launch rows FFN (kRowsFlagWords)
    float* attn_part = nullptr;   // sliding_attention split partials (kAttnPartFloats)
    float* fattn_part = nullptr;  // full-attention page partials (kFattnPartFloats)
    void* base = nullptr;
    int cus = 0;                  // compute units of the device
    int8_t ffn_fused[6] = {-1, -1, -1, -1, -1, -1};  // per (format, scale kind): grid fits resident? (-1 unknown)
    int8_t o_fused[2] = {-1, -1};                    // per scale kind
    int8_t qkv_fused[2] = {-1, -1};                  // per scale kind
    int8_t full_o_fused[2] = {-1, -1};               // the same for full_attention_output
    int8_t o_ffn_fused[3] = {-1, -1, -1};            // the single-launch O -> FFN, per FFN format
    int8_t rows_fused[18] = {-1, -1, -1, -1, -1, -1, -1, -1, -1,  // the one-launch rows FFN, per (format,
                             -1, -1, -1, -1, -1, -1, -1, -1, -1}; // scale kind, O post step kind)
};

// Returns the context of the current device, allocating it on first use. nullptr on failure.
DevCtx* device_context(hipError_t* err);

// Records `msg` as this thread's last error (moa_last_error_string) and returns `code`.
int set_error(int code, const char* msg);

enum class ScaleKind { F32, BF16 };
enum class FfnFormat { FP8, NVFP4, MXFP4 };

struct QkvParams {
    const uint16_t* x; const uint8_t* qw; const uint8_t* kw; const uint8_t* vw;
    const void* qs; const void* ks; const void* vs; ScaleKind scale_kind;
    const uint16_t* in_rms; const uint16_t* q_rms; const uint16_t* k_rms;
    const int32_t* kv_off; const int32_t* rope_off; const uint16_t* cos; const uint16_t* sin;
    uint16_t* k_cache; uint16_t* v_cache; uint16_t* q_out;
};

struct OParams {
    const uint16_t* x; const uint16_t* post_rms; const uint8_t* ow; const void* os; ScaleKind scale_kind;
    uint16_t* residual;
    const float* div = nullptr;  // full-attention layers: running softmax sums [M][16] that divide x
};

// Waits of the single-launch kernels (a kernel argument). A workgroup that has waited steal_ticks
// (100 MHz wall clock) for another workgroup of its grid does that workgroup's work itself, so the
// kernels finish with correct results even when part of the grid cannot be resident (another
// process holding CUs). Test only: workgroups hold[0..3] of each launch wait hold_ticks at entry,
// before they read or write anything, as if they had started late.
struct Stall {
    uint32_t steal_ticks;
    uint32_t hold_ticks;
    int32_t hold[4];
};
constexpr uint32_t kStealTicks = 50000;  // 500 us: far beyond any wait of a resident grid
void set_stall(const Stall& st);           // the Stall every later single-launch call passes (tests)
void set_rows_one_launch(bool on);         // the rows FFN's up/gate and down in one launch (default) or two (tests)

struct FfnParams {
    FfnFormat fmt;
    uint16_t* residual; const uint16_t* pre_rms;
    const uint8_t* up; const uint8_t* gate; const uint8_t* down;
    const void* up_s; const void* gate_s; const void* down_s;  // FP8: f32|bf16 per row; FP4: u8 codes
    ScaleKind scale_kind;                                        // FP8 only
    const float* up_g; const float* gate_g; const float* down_g; // NVFP4 reciprocal globals (device)
    const uint16_t* post_rms; const uint16_t* layer_scalar;      // nullable
};

struct ProjParams {  // raw FP8 projection out[m,n] = bf16((x[m].W[n]) * s[n])
    const uint16_t* x; const uint8_t* w; const void* s; ScaleKind scale_kind; uint16_t* out;
    int N, K;
};

hipError_t launch_qkv_decode(const QkvParams& p, int M, hipStream_t s, DevCtx* ctx);
hipError_t launch_o_decode(const OParams& p, int M, hipStream_t s, DevCtx* ctx);
hipError_t launch_ffn_decode(const FfnParams& p, int M, hipStream_t s, DevCtx* ctx);
hipError_t launch_proj_decode(const ProjParams& p, int M, hipStream_t s);
// One token row of sliding_attention_output followed by decoder_feedforward on the same residual
// (o.residual == p.residual), in one launch. Returns false, launching nothing, when that grid cannot
// be resident at once or no single-launch kernel covers the operand types (FP8 FFN with f32 O
// scales, NVFP4 with bf16 O scales, MXFP4 with f32 O scales); *e is the launch's status otherwise.
bool launch_o_ffn_fused(const OParams& o, const FfnParams& p, hipStream_t s, DevCtx* ctx, hipError_t* e);

// Full-attention layers: ops::full_project_qkv (QkvParams with vw / vs unused; k_cache / v_cache
// are the position's page) and ops::full_attention_output (OParams with div set).
hipError_t launch_full_qkv(const QkvParams& p, int M, hipStream_t s, DevCtx* ctx);
hipError_t launch_full_o(const OParams& p, int M, hipStream_t s, DevCtx* ctx);
// ops::full_attention_first_page (first) / ops::full_attention_page for M token rows: q / out
// [M][16][512], the page's K and V [512][512], mask [M][512], running max / sum [M][16].
hipError_t launch_full_attention_page(const uint16_t* q, const uint16_t* k_page, const uint16_t* v_page,
                                      const float* mask, float* running_max, float* running_sum, uint16_t* out,
                                      int M, bool first, hipStream_t s, DevCtx* ctx);
// The state over pages 0 .. P - 1 (k_pages / v_pages [P][512][512], masks [P][M][512]) at once.
hipError_t launch_full_attention(const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages,
                                 const float* masks, int P, float* running_max, float* running_sum, uint16_t* out,
                                 int M, hipStream_t s, DevCtx* ctx);

// MFMA path for one chunk of 1..kMaxChunkM token rows starting at row m0 of the call.
hipError_t launch_qkv_chunk(const QkvParams& p, int m0, int M, hipStream_t s, DevCtx* ctx);
hipError_t launch_o_chunk(const OParams& p, int m0, int M, hipStream_t s, DevCtx* ctx);
hipError_t launch_ffn_chunk(const FfnParams& p, int m0, int M, hipStream_t s, DevCtx* ctx);  // every format
// sliding_attention_output then decoder_feedforward on one residual (o.residual == p.residual)
hipError_t launch_o_ffn_chunk(const OParams& o, const FfnParams& p, int m0, int M, hipStream_t s, DevCtx* ctx);
// decoder_feedforward for 1..kMaxDecodeM rows on the matrix cores (every format; moa_rows.hip), and its
// last step: the sum of `splits` f32 partials [splits][M][kH] of the down projection, the format's
// commit, post-RMSNorm, residual and layer scalar into res [M][kH].
hipError_t launch_ffn_rows(const FfnParams& p, int m0, int M, hipStream_t s, DevCtx* ctx);
hipError_t launch_ffn_post_rows(const FfnParams& p, const float* part, int splits, int M, uint16_t* res, hipStream_t s);
// out[m] = bf16(RMSNorm(x[m]) * w) for M rows of kH, row-major (gemma4.py:83-89).
hipError_t launch_rmsnorm_rows(const uint16_t* x, const uint16_t* w, uint16_t* out, int M, hipStream_t s);
// The row kernels after a split-K contraction of M rows (partials [splits][M][N] f32): the QKV heads
// (scale, head RMSNorm, RoPE, q_out / ring-cache stores) and the O post (scale, post-RMSNorm, residual).
hipError_t launch_qkv_heads(const QkvParams& p, int m0, int M, const float* part, int splits, hipStream_t s, DevCtx* ctx);
hipError_t launch_post_rows(const float* part, int splits, int M, const void* scale, ScaleKind sk, const uint16_t* w_post,
                            uint16_t* res, const uint16_t* ls, hipStream_t s);
// The O post rows with the FFN's pre-norm behind them (splits <= 4): the new residual rows into res,
// and bf16(RMSNorm(new residual) * w_pre) row-major into hout [M][kH].
hipError_t launch_post_pre_rows(const float* part, int splits, int M, const void* scale, ScaleKind sk,
                                const uint16_t* w_post, uint16_t* res, const uint16_t* w_pre, uint16_t* hout, hipStream_t s);
// sliding_project_qkv and sliding / full attention output for 2..kMaxDecodeM rows on the matrix cores
// (moa_rows.hip).
hipError_t launch_qkv_rows(const QkvParams& p, int m0, int M, hipStream_t s, DevCtx* ctx);
hipError_t launch_o_rows(const OParams& p, int m0, int M, hipStream_t s, DevCtx* ctx);
// sliding_attention_output then decoder_feedforward on one residual for 2..kMaxDecodeM rows: O's post
// rows also write the FFN's normalised input, so the FFN starts at its up/gate contraction (two
// launches where the one-launch rows FFN fits: O's contraction, then the FFN with O's post rows).
hipError_t launch_o_ffn_rows(const OParams& o, const FfnParams& p, int m0, int M, hipStream_t s, DevCtx* ctx);
hipError_t launch_full_qkv_rows(const QkvParams& p, int m0, int M, hipStream_t s, DevCtx* ctx);

// ops::final_norm_and_logits for M token rows (input [M][kH], out [M][kW]).
hipError_t launch_final_norm_and_logits(const uint16_t* input, const uint16_t* rms_w, const uint16_t* w, uint16_t* out,
                                        int M, hipStream_t s);

// ops::sliding_attention for M token rows (q / out [M][kNs][kGs][kDs], mask [M][kTs]).
hipError_t launch_sliding_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, const float* mask,
                                    uint16_t* out, int M, hipStream_t s, DevCtx* ctx);

hipError_t launch_format_selftest(uint32_t* out, hipStream_t s);

}  // namespace moa
