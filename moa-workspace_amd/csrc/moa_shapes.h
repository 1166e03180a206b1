// moa_shapes.h -- model shapes of the hot path (FO/src/axes.rs:3-29; EPS FO/src/lib.rs:25).
#pragma once

namespace moa {
constexpr int kH = 3840;    // hidden
constexpr int kL = 15360;   // FFN intermediate
constexpr int kNs = 8;      // KV heads (sliding layers)
constexpr int kGs = 2;      // query heads per KV head
constexpr int kDs = 256;    // head_dim
constexpr int kQs = 4096;   // kNs * kGs * kDs
constexpr int kPs = 2048;   // kNs * kDs
constexpr int kTs = 1024;   // ring-cache slots
constexpr int kE = 32768;   // RoPE table rows
constexpr int kW = 262144;  // vocabulary rows of lm_head (FO/src/axes.rs: W)
// full-attention layers (every sixth): 16 query heads and one KV head of 512, a cache of pages
constexpr int kGf = 16;     // query heads
constexpr int kDf = 512;    // head_dim
constexpr int kQf = 8192;   // kGf * kDf
constexpr int kPf = 512;    // K projection rows (V is the unweighted norm of raw K)
constexpr int kTf = 512;    // slots per cache page
constexpr int kCf = 64;     // pages (FO/src/axes.rs: C)
constexpr float kEps = 1e-6f;
}  // namespace moa
