/*
 * moa_oracle.c -- CPU restatement of the reference's hot-path algorithm.
 *
 * TEST INFRASTRUCTURE ONLY (the checker; never the product path). See moa_oracle.h
 * for the contract and oracle/README.md for what pins each function.
 * Build: oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off).
 */
#include "moa_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ formats */

static inline uint32_t f32_bits(float v) { uint32_t u; memcpy(&u, &v, 4); return u; }
static inline float bits_f32(uint32_t u) { float v; memcpy(&v, &u, 4); return v; }

/* fixture_prng.py:80-90 (round half to even on the raw bits). The reference never
 * feeds NaN; NaN maps to the canonical quiet NaN as torch's bf16 conversion does. */
uint16_t orc_bf16_rne(float v) {
    uint32_t b = f32_bits(v);
    if ((b & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    uint32_t rounding = 0x7fffu + ((b >> 16) & 1u);
    return (uint16_t)((b + rounding) >> 16);
}

float orc_bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

/* E4M3FN (OCP): bias 7, no infinities, S.1111.111 is NaN, subnormal m * 2^-9.
 * The reference widens codes with torch.float8_e4m3fn (generate_references.py:152). */
float orc_e4m3_decode(uint8_t c) {
    int e = (c >> 3) & 15, m = c & 7;
    float v;
    if (e == 15 && m == 7) return NAN;
    if (e == 0) v = ldexpf((float)m, -9);
    else v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return (c & 0x80) ? -v : v;
}

/* Round-to-nearest-even encoder, saturating at +-448 (the quantisers never exceed it). */
uint8_t orc_e4m3_encode_rne(float v) {
    if (isnan(v)) return 0x7f;
    uint8_t sign = signbit(v) ? 0x80 : 0;
    float a = fabsf(v);
    if (a >= 464.0f) return sign | 0x7e; /* 448 */
    int e;
    float quantum;
    if (a < 0x1p-6f) quantum = 0x1p-9f;
    else { frexpf(a, &e); quantum = ldexpf(1.0f, e - 1 - 3); }
    float r = nearbyintf(a / quantum) * quantum; /* exact scaling by a power of two */
    if (r == 0.0f) return sign;
    if (r < 0x1p-6f) return sign | (uint8_t)(r / 0x1p-9f);
    frexpf(r, &e); /* r = f * 2^e, f in [0.5,1) */
    int exp_field = e - 1 + 7;
    int mant = (int)((ldexpf(r, -(e - 1)) - 1.0f) * 8.0f);
    if (exp_field > 15 || (exp_field == 15 && mant == 7)) return sign | 0x7e;
    return sign | (uint8_t)(exp_field << 3) | (uint8_t)mant;
}

static const float kE2M1[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};

/* generate_references.py:69,162: magnitude table indexed by code & 7, bit 3 = sign. */
float orc_e2m1_decode(uint8_t n) {
    float v = kE2M1[n & 7];
    return (n & 8) ? -v : v;
}

/* RNE onto {0,.5,1,1.5,2,3,4,6}; ties go to the even code. Saturates at 6. */
uint8_t orc_e2m1_encode_rne(float v) {
    uint8_t sign = signbit(v) ? 8 : 0;
    float a = fabsf(v);
    uint8_t c;
    if (isnan(a)) return 7 | sign;
    if (a <= 0.25f) c = 0;
    else if (a < 0.75f) c = 1;
    else if (a <= 1.25f) c = 2;
    else if (a < 1.75f) c = 3;
    else if (a <= 2.5f) c = 4;
    else if (a < 3.5f) c = 5;
    else if (a <= 5.0f) c = 6;
    else c = 7;
    return c | sign;
}

float orc_e8m0_decode(uint8_t e) {
    if (e == 0xff) return NAN;
    return ldexpf(1.0f, (int)e - 127);
}

/* --------------------------------------------------------------------- PRNG */

#define FNV_OFFSET 0xcbf29ce484222325ull
#define FNV_PRIME 0x00000100000001b3ull
#define GOLDEN 0x9e3779b97f4a7c15ull
#define MIX_A 0xbf58476d1ce4e5b9ull
#define MIX_B 0x94d049bb133111ebull

/* fixture_prng.py:44-54: FNV-1a over the UTF-8 name. */
uint64_t orc_name_hash(const char* name) {
    uint64_t h = FNV_OFFSET;
    for (const unsigned char* p = (const unsigned char*)name; *p; ++p) h = (h ^ *p) * FNV_PRIME;
    return h;
}

/* fixture_prng.py:57-67: splitmix64's finaliser applied to (seed ^ index) + golden. */
uint64_t orc_word(uint64_t seed, uint64_t index) {
    uint64_t x = (seed ^ index) + GOLDEN;
    x = (x ^ (x >> 30)) * MIX_A;
    x = (x ^ (x >> 27)) * MIX_B;
    return x ^ (x >> 31);
}

/* fixture_prng.py:71-77: the top 24 bits as an exact f32 in [0,1). */
static inline float u01(uint64_t w) { return (float)(uint32_t)(w >> 40) / 16777216.0f; }

void orc_bf16_uniform(const char* name, size_t count, float lo, float hi, uint16_t* out) {
    uint64_t seed = orc_name_hash(name);
    float span = hi - lo;
    for (size_t i = 0; i < count; ++i) {
        float t = span * u01(orc_word(seed, i));
        out[i] = orc_bf16_rne(lo + t);
    }
}

void orc_f32_uniform(const char* name, size_t count, float lo, float hi, float* out) {
    uint64_t seed = orc_name_hash(name);
    float span = hi - lo;
    for (size_t i = 0; i < count; ++i) {
        float t = span * u01(orc_word(seed, i));
        out[i] = lo + t;
    }
}

void orc_bf16_signs(const char* name, size_t count, float scale, uint16_t* out) {
    uint64_t seed = orc_name_hash(name);
    uint16_t mag = orc_bf16_rne(fabsf(scale));
    for (size_t i = 0; i < count; ++i)
        out[i] = (orc_word(seed, i) >> 63) ? (uint16_t)(mag | 0x8000u) : mag;
}

void orc_f8_banded(const char* name, size_t count, int exp_min, int exp_max, int is_signed,
                   uint8_t* out) {
    uint64_t seed = orc_name_hash(name);
    uint64_t span = (uint64_t)(exp_max - exp_min + 1);
    for (size_t i = 0; i < count; ++i) {
        uint64_t w = orc_word(seed, i);
        uint8_t e = (uint8_t)(exp_min + (int)((w >> 32) % span));
        uint8_t m = (uint8_t)((w >> 56) & 7u);
        uint8_t s = is_signed ? (uint8_t)((w >> 63) << 7) : 0;
        out[i] = s | (uint8_t)(e << 3) | m;
    }
}

void orc_f4_nibbles(const char* name, size_t count, uint8_t* out_packed) {
    uint64_t seed = orc_name_hash(name);
    for (size_t i = 0; i + 1 < count; i += 2) {
        uint8_t lo = (uint8_t)(orc_word(seed, i) >> 60) & 0xf;
        uint8_t hi = (uint8_t)(orc_word(seed, i + 1) >> 60) & 0xf;
        out_packed[i / 2] = lo | (uint8_t)(hi << 4);
    }
}

/* fixture_prng.py:170-198: sum of word * (2*index+1) mod 2^32 over zero-padded u32 words. */
uint32_t orc_checksum(const void* data, size_t nbytes) {
    const uint8_t* p = (const uint8_t*)data;
    uint32_t total = 0;
    size_t words = (nbytes + 3) / 4;
    for (size_t i = 0; i < words; ++i) {
        uint8_t b[4] = {0, 0, 0, 0};
        for (int j = 0; j < 4; ++j)
            if (4 * i + j < nbytes) b[j] = p[4 * i + j];
        uint32_t w = (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) |
                     ((uint32_t)b[3] << 24);
        total += w * ((uint32_t)i * 2u + 1u);
    }
    return total;
}

int orc_run_pos(int run) {
    char name[64];
    snprintf(name, sizeof name, "run%d.global.pos", run);
    return 1 + (int)(orc_word(orc_name_hash(name), 0) % 2047u);
}

/* generate_references.py:184-197 (== test_kernels.rs:393-409): f64 angles, narrowed to f32. */
void orc_rope_row(int head_dim, double theta, double factor, int pos, float* cos_out,
                  float* sin_out) {
    int angles = (int)floor(factor * head_dim / 2.0);
    int half = head_dim / 2;
    for (int i = 0; i < head_dim; ++i) {
        int j = i % half;
        double inv = j < angles ? 1.0 / pow(theta, (double)(2 * j) / (double)head_dim) : 0.0;
        double a = (double)pos * inv;
        cos_out[i] = (float)cos(a);
        sin_out[i] = (float)sin(a);
    }
}

/* --------------------------------------------------------------- primitives */

/* Sums of the reference's f32 accumulations: the reference adds in f32 in an unspecified
 * order (torch CPU), so the oracle computes the value every order approximates, the exactly
 * rounded f32 sum: eight interleaved f64 partial sums (each term -- a square of a bf16 value
 * or a bf16 x fp8/fp4 product -- is exact in f64, and the sums of these few thousand terms
 * are too), combined pairwise and rounded once to f32. Exact-dyadic known answers do not
 * depend on this choice; on random inputs it keeps the oracle within one f32 rounding of the
 * ideal, so a tolerance gate measures each implementation against the same anchor. */
#define LANES 8
static inline float reduce_lanes(double* acc) {
    for (int w = LANES / 2; w >= 1; w /= 2)
        for (int i = 0; i < w; ++i) acc[i] = acc[i] + acc[i + w];
    return (float)acc[0];
}

void orc_rmsnorm_row(const uint16_t* x, const uint16_t* w, int n, uint16_t* out) {
    double acc[LANES] = {0};
    for (int i = 0; i < n; ++i) {
        double v = orc_bf16_to_f32(x[i]);
        acc[i % LANES] += v * v;
    }
    float mean = reduce_lanes(acc) / (float)n;
    float inv = 1.0f / sqrtf(mean + ORC_EPS); /* torch.rsqrt on CPU = 1/sqrt, both rounded */
    for (int i = 0; i < n; ++i) {
        float y = orc_bf16_to_f32(x[i]) * inv;
        if (w) y = y * orc_bf16_to_f32(w[i]);
        out[i] = orc_bf16_rne(y);
    }
}

/* torch's gelu(approximate="tanh"): 0.5*x*(1+tanh(sqrt(2/pi)*(x+0.044715*x^3))) evaluated
 * in f32 (opmath for bf16 inputs), left to right. */
float orc_gelu_tanh(float x) {
    const float kBeta = (float)(0.7978845608028654); /* sqrt(2/pi) */
    const float kKappa = 0.044715f;
    float cube = x * x * x;
    float inner = kBeta * (x + kKappa * cube);
    return 0.5f * x * (1.0f + tanhf(inner));
}

static float e4m3_lut[256];
static float e2m1_lut[16];
static float e8m0_lut[256];
static int luts_ready = 0;
static void init_luts(void) {
    if (luts_ready) return;
    for (int i = 0; i < 256; ++i) e4m3_lut[i] = orc_e4m3_decode((uint8_t)i);
    for (int i = 0; i < 16; ++i) e2m1_lut[i] = orc_e2m1_decode((uint8_t)i);
    for (int i = 0; i < 256; ++i) e8m0_lut[i] = orc_e8m0_decode((uint8_t)i);
    luts_ready = 1;
}

static inline float dot_fp8_row(const float* xf, const uint8_t* row, int K) {
    double acc[LANES] = {0};
    for (int k = 0; k < K; ++k) acc[k % LANES] += (double)xf[k] * e4m3_lut[row[k]];
    return reduce_lanes(acc);
}

void orc_scaled_projection_fp8(const uint16_t* x, int M, int K, const uint8_t* w,
                               const float* scale, int N, uint16_t* out) {
    init_luts();
    float* xf = (float*)malloc(sizeof(float) * (size_t)K * (size_t)M);
    for (size_t i = 0; i < (size_t)K * (size_t)M; ++i) xf[i] = orc_bf16_to_f32(x[i]);
    for (int m = 0; m < M; ++m) {
#pragma omp parallel for schedule(static)
        for (int n = 0; n < N; ++n) {
            float d = dot_fp8_row(xf + (size_t)m * K, w + (size_t)n * K, K);
            out[(size_t)m * N + n] = orc_bf16_rne(d * scale[n]);
        }
    }
    free(xf);
}

/* --------------------------------------------------------------------- QKV */

static void rope_head_n(const uint16_t* xin, const uint16_t* cos_row, const uint16_t* sin_dev,
                        uint16_t* out, int n) {
    /* generate_references.py:213-220 with gemma4.py:120-122: y = x*cos + rotate_half(x)*sin,
     * every op rounded to bf16, over a head of n elements. The table holds sin with the low half
     * negated (generate_references.py:200-210; runtime.rs:298-322); undo that exactly to recover
     * the reference sin. */
    for (int i = 0; i < n; ++i) {
        float s = orc_bf16_to_f32(sin_dev[i]);
        if (i < n / 2) s = -s;
        float xi = orc_bf16_to_f32(xin[i]);
        float rot = i < n / 2 ? -orc_bf16_to_f32(xin[i + n / 2]) : orc_bf16_to_f32(xin[i - n / 2]);
        float a = orc_bf16_to_f32(orc_bf16_rne(xi * orc_bf16_to_f32(cos_row[i])));
        float b = orc_bf16_to_f32(orc_bf16_rne(rot * orc_bf16_to_f32(orc_bf16_rne(s))));
        out[i] = orc_bf16_rne(a + b);
    }
}

static void rope_head(const uint16_t* xin, const uint16_t* cos_row, const uint16_t* sin_dev, uint16_t* out) {
    rope_head_n(xin, cos_row, sin_dev, out, ORC_DS);
}

void orc_sliding_project_qkv(const uint16_t* x, const uint8_t* q_w, const uint8_t* k_w,
                             const uint8_t* v_w, const float* q_s, const float* k_s,
                             const float* v_s, const uint16_t* in_rms, const uint16_t* q_rms,
                             const uint16_t* k_rms, int32_t kv_offset, int32_t rope_offset,
                             const uint16_t* cos_tab, const uint16_t* sin_tab,
                             uint16_t* k_cache, uint16_t* v_cache, uint16_t* q_out, int M) {
    uint16_t h[ORC_H];
    uint16_t* q_raw = (uint16_t*)malloc(2 * ORC_QS);
    uint16_t* k_raw = (uint16_t*)malloc(2 * ORC_PS);
    uint16_t* v_raw = (uint16_t*)malloc(2 * ORC_PS);
    uint16_t tmp[ORC_DS];
    int slot0 = kv_offset / (ORC_NS * ORC_DS * 2);
    int row0 = rope_offset / (ORC_DS * 2);
    for (int m = 0; m < M; ++m) {
        orc_rmsnorm_row(x + (size_t)m * ORC_H, in_rms, ORC_H, h);
        orc_scaled_projection_fp8(h, 1, ORC_H, q_w, q_s, ORC_QS, q_raw);
        orc_scaled_projection_fp8(h, 1, ORC_H, k_w, k_s, ORC_PS, k_raw);
        orc_scaled_projection_fp8(h, 1, ORC_H, v_w, v_s, ORC_PS, v_raw);
        const uint16_t* cos_row = cos_tab + (size_t)(row0 + m) * ORC_DS;
        const uint16_t* sin_row = sin_tab + (size_t)(row0 + m) * ORC_DS;
        int slot = (slot0 + m) % ORC_TS;
        for (int hd = 0; hd < ORC_NS * ORC_GS; ++hd) {
            orc_rmsnorm_row(q_raw + hd * ORC_DS, q_rms, ORC_DS, tmp);
            rope_head(tmp, cos_row, sin_row, q_out + ((size_t)m * ORC_QS + hd * ORC_DS));
        }
        for (int hd = 0; hd < ORC_NS; ++hd) {
            size_t at = ((size_t)slot * ORC_NS + hd) * ORC_DS;
            orc_rmsnorm_row(k_raw + hd * ORC_DS, k_rms, ORC_DS, tmp);
            rope_head(tmp, cos_row, sin_row, k_cache + at);
            orc_rmsnorm_row(v_raw + hd * ORC_DS, NULL, ORC_DS, v_cache + at);
        }
    }
    free(q_raw);
    free(k_raw);
    free(v_raw);
}

/* ------------------------------------------------------ full-attention layer */

void orc_full_project_qkv(const uint16_t* x, const uint8_t* q_w, const uint8_t* k_w, const float* q_s,
                          const float* k_s, const uint16_t* in_rms, const uint16_t* q_rms, const uint16_t* k_rms,
                          int32_t kv_offset, int32_t rope_offset, const uint16_t* cos_tab, const uint16_t* sin_tab,
                          uint16_t* k_page, uint16_t* v_page, uint16_t* q_out, int M) {
    uint16_t h[ORC_H];
    uint16_t* q_raw = (uint16_t*)malloc(2 * ORC_QF);
    uint16_t k_raw[ORC_DF], tmp[ORC_DF];
    const int slot0 = kv_offset / (ORC_DF * 2);
    const int row0 = rope_offset / (ORC_DF * 2);
    for (int m = 0; m < M; ++m) {
        orc_rmsnorm_row(x + (size_t)m * ORC_H, in_rms, ORC_H, h);
        orc_scaled_projection_fp8(h, 1, ORC_H, q_w, q_s, ORC_QF, q_raw);
        orc_scaled_projection_fp8(h, 1, ORC_H, k_w, k_s, ORC_DF, k_raw);
        const uint16_t* cos_row = cos_tab + (size_t)(row0 + m) * ORC_DF;
        const uint16_t* sin_row = sin_tab + (size_t)(row0 + m) * ORC_DF;
        for (int hd = 0; hd < ORC_GF; ++hd) {
            orc_rmsnorm_row(q_raw + hd * ORC_DF, q_rms, ORC_DF, tmp);
            rope_head_n(tmp, cos_row, sin_row, q_out + ((size_t)m * ORC_QF + hd * ORC_DF), ORC_DF);
        }
        const size_t at = (size_t)(slot0 + m) * ORC_DF;
        orc_rmsnorm_row(k_raw, k_rms, ORC_DF, tmp);
        rope_head_n(tmp, cos_row, sin_row, k_page + at, ORC_DF);
        orc_rmsnorm_row(k_raw, NULL, ORC_DF, v_page + at); /* V: the unweighted norm of raw K */
    }
    free(q_raw);
}

void orc_full_attention_pages(const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages,
                              const float* masks, int P, float* running_max, float* running_sum, uint16_t* out,
                              int M) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int m = 0; m < M; ++m)
        for (int hd = 0; hd < ORC_GF; ++hd) {
            const uint16_t* qr = q + ((size_t)m * ORC_GF + hd) * ORC_DF;
            double* s = (double*)malloc(sizeof(double) * (size_t)P * ORC_TF);
            double mx = -INFINITY;
            for (int pg = 0; pg < P; ++pg)
                for (int t = 0; t < ORC_TF; ++t) {
                    const size_t at = (size_t)pg * ORC_TF + t;
                    if (masks[((size_t)pg * M + m) * ORC_TF + t] == 0.0f) continue;
                    const uint16_t* kr = k_pages + at * ORC_DF;
                    double a = 0.0;
                    for (int d = 0; d < ORC_DF; ++d) a += (double)orc_bf16_to_f32(qr[d]) * orc_bf16_to_f32(kr[d]);
                    s[at] = a;
                    if (a > mx) mx = a;
                }
            double l = 0.0, o[ORC_DF];
            for (int d = 0; d < ORC_DF; ++d) o[d] = 0.0;
            if (mx != -INFINITY) {
                for (int pg = 0; pg < P; ++pg)
                    for (int t = 0; t < ORC_TF; ++t) {
                        const size_t at = (size_t)pg * ORC_TF + t;
                        if (masks[((size_t)pg * M + m) * ORC_TF + t] == 0.0f) continue;
                        const double e = exp(s[at] - mx);
                        l += e;
                        const uint16_t* vr = v_pages + at * ORC_DF;
                        for (int d = 0; d < ORC_DF; ++d) o[d] += e * orc_bf16_to_f32(vr[d]);
                    }
            }
            running_max[(size_t)m * ORC_GF + hd] = (float)mx;
            running_sum[(size_t)m * ORC_GF + hd] = (float)l;
            uint16_t* orow = out + ((size_t)m * ORC_GF + hd) * ORC_DF;
            for (int d = 0; d < ORC_DF; ++d) orow[d] = orc_bf16_rne((float)o[d]);
            free(s);
        }
}

void orc_full_attention_output(const uint16_t* x, const float* running_sum, const uint16_t* post_rms,
                               const uint8_t* o_w, const float* o_s, uint16_t* residual, int M) {
    uint16_t* xd = (uint16_t*)malloc(2 * ORC_QF);
    uint16_t p[ORC_H], n[ORC_H];
    for (int m = 0; m < M; ++m) {
        for (int i = 0; i < ORC_QF; ++i) {
            const float sm = running_sum[(size_t)m * ORC_GF + i / ORC_DF];
            xd[i] = orc_bf16_rne(sm > 0.0f ? orc_bf16_to_f32(x[(size_t)m * ORC_QF + i]) / sm : 0.0f);
        }
        orc_scaled_projection_fp8(xd, 1, ORC_QF, o_w, o_s, ORC_H, p);
        orc_rmsnorm_row(p, post_rms, ORC_H, n);
        uint16_t* r = residual + (size_t)m * ORC_H;
        for (int i = 0; i < ORC_H; ++i) r[i] = orc_bf16_rne(orc_bf16_to_f32(r[i]) + orc_bf16_to_f32(n[i]));
    }
    free(xd);
}

/* ---------------------------------------------------------------------- O */

void orc_sliding_attention_output(const uint16_t* x, const uint16_t* post_rms, const uint8_t* o_w,
                                  const float* o_s, uint16_t* residual, int M) {
    uint16_t p[ORC_H], n[ORC_H];
    for (int m = 0; m < M; ++m) {
        orc_scaled_projection_fp8(x + (size_t)m * ORC_QS, 1, ORC_QS, o_w, o_s, ORC_H, p);
        orc_rmsnorm_row(p, post_rms, ORC_H, n);
        uint16_t* r = residual + (size_t)m * ORC_H;
        for (int i = 0; i < ORC_H; ++i)
            r[i] = orc_bf16_rne(orc_bf16_to_f32(r[i]) + orc_bf16_to_f32(n[i]));
    }
}

/* --------------------------------------------------------------- attention */

/* ops::sliding_attention (FO/src/ops.rs:118-128) against its CPU reference, gemma4.py:163-186:
 * scaled_dot_product_attention(q, k, v, attn_mask, scale=1.0) for one query position, the mask
 * being the runtime's 1.0 / 0.0 row over the ring slots (FO/src/host/runtime.rs:160, 409).
 * Computed in f64 (every bf16 x bf16 product is exact); the output is rounded to f32, then to bf16. A row
 * with no valid slot gives zeros (the RNGD kernel's sum + 1e-6 gives 0 / 1e-6 = 0 too).
 * q, out [M][8][2][256]; k, v [1024][8][256]; mask [M][1024]. */
void orc_sliding_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* mask,
                           uint16_t* out, int M) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int m = 0; m < M; ++m)
        for (int hq = 0; hq < ORC_NS * ORC_GS; ++hq) {
            const int n = hq / ORC_GS;
            const uint16_t* qr = q + ((size_t)m * ORC_NS * ORC_GS + hq) * ORC_DS;
            const float* mr = mask + (size_t)m * ORC_TS;
            double s[ORC_TS];
            double mx = -INFINITY;
            for (int t = 0; t < ORC_TS; ++t) {
                if (mr[t] == 0.0f) continue;
                const uint16_t* kr = k + ((size_t)t * ORC_NS + n) * ORC_DS;
                double a = 0.0;
                for (int d = 0; d < ORC_DS; ++d) a += (double)orc_bf16_to_f32(qr[d]) * orc_bf16_to_f32(kr[d]);
                s[t] = a;
                if (a > mx) mx = a;
            }
            double l = 0.0, o[ORC_DS];
            for (int d = 0; d < ORC_DS; ++d) o[d] = 0.0;
            for (int t = 0; t < ORC_TS; ++t) {
                if (mr[t] == 0.0f) continue;
                const double p = exp(s[t] - mx);
                l += p;
                const uint16_t* vr = v + ((size_t)t * ORC_NS + n) * ORC_DS;
                for (int d = 0; d < ORC_DS; ++d) o[d] += p * orc_bf16_to_f32(vr[d]);
            }
            uint16_t* orow = out + ((size_t)m * ORC_NS * ORC_GS + hq) * ORC_DS;
            for (int d = 0; d < ORC_DS; ++d) orow[d] = orc_bf16_rne(l > 0.0 ? (float)(o[d] / l) : 0.0f);
        }
}

/* ------------------------------------------------------------------ logits */

/* f64 -> bf16 with one rounding (to nearest even). The f32 step can only land on a bf16 tie that
 * the f64 value does not sit on; such a tie is moved one f32 step toward the f64 value first. */
static uint16_t bf16_rne_f64(double d) {
    float f = (float)d;
    uint32_t u;
    memcpy(&u, &f, 4);
    if (isfinite(f) && (u & 0xffffu) == 0x8000u && (double)f != d) f = nextafterf(f, d > (double)f ? INFINITY : -INFINITY);
    return orc_bf16_rne(f);
}

uint16_t orc_softcap30(uint16_t l) {
    const double v = orc_bf16_to_f32(l);
    return bf16_rne_f64(tanh(v / 30.0) * 30.0);
}

void orc_final_norm_and_logits(const uint16_t* x, const uint16_t* rms_w, const uint16_t* lm_head, int W,
                               uint16_t* out, int M) {
    for (int m = 0; m < M; ++m) {
        uint16_t h[ORC_H];
        float hf[ORC_H];
        orc_rmsnorm_row(x + (size_t)m * ORC_H, rms_w, ORC_H, h);
        for (int i = 0; i < ORC_H; ++i) hf[i] = orc_bf16_to_f32(h[i]);
#pragma omp parallel for schedule(static)
        for (int r = 0; r < W; ++r) {
            const uint16_t* wr = lm_head + (size_t)r * ORC_H;
            double acc[LANES] = {0};
            for (int k = 0; k < ORC_H; ++k) acc[k % LANES] += (double)hf[k] * orc_bf16_to_f32(wr[k]);
            /* the lm_head linear's bf16 output feeds the softcap */
            out[(size_t)m * W + r] = orc_softcap30(orc_bf16_rne(reduce_lanes(acc)));
        }
    }
}

/* --------------------------------------------------------------------- FFN */

/* One output row of a projection with the format's rounding rule. xf: f32 activation. */
static uint16_t ffn_proj_row(const orc_ffn_weights* w, int which, const float* xf, int K, int n) {
    const uint8_t* mat = which == 0 ? w->up : which == 1 ? w->gate : w->down;
    const void* sc = which == 0 ? w->up_scale : which == 1 ? w->gate_scale : w->down_scale;
    float inv_g = which == 0 ? w->up_inv_global : which == 1 ? w->gate_inv_global : w->down_inv_global;
    double acc[LANES] = {0};
    if (w->format == ORC_FFN_FP8) {
        float d = dot_fp8_row(xf, mat + (size_t)n * K, K);
        return orc_bf16_rne(d * ((const float*)sc)[n]);
    }
    const uint8_t* row = mat + (size_t)n * (K / 2);
    const uint8_t* srow = (const uint8_t*)sc + (size_t)n * (K / (w->format == ORC_FFN_NVFP4 ? 16 : 32));
    for (int k = 0; k < K; ++k) {
        uint8_t byte = row[k / 2];
        uint8_t nib = (k & 1) ? (byte >> 4) : (byte & 0xf);
        /* The reference folds the block scale into the weight before the bf16 linear
         * (generate_references.py:398,407); the product is exact in f32 and in bf16. */
        float wv = w->format == ORC_FFN_NVFP4 ? e2m1_lut[nib] * e4m3_lut[srow[k / 16]]
                                               : e2m1_lut[nib] * e8m0_lut[srow[k / 32]];
        wv = orc_bf16_to_f32(orc_bf16_rne(wv));
        acc[k % LANES] += (double)xf[k] * wv;
    }
    float d = reduce_lanes(acc);
    if (w->format == ORC_FFN_NVFP4) /* bf16 nn.Linear output, then GloballyScaled (:371-372) */
        return orc_bf16_rne(orc_bf16_to_f32(orc_bf16_rne(d)) * inv_g);
    return orc_bf16_rne(d); /* MXFP4: plain bf16 linear */
}

void orc_ffn_up_gate(const uint16_t* h, const orc_ffn_weights* w, uint16_t* p, int M) {
    init_luts();
    float* xf = (float*)malloc(sizeof(float) * ORC_H);
    for (int m = 0; m < M; ++m) {
        for (int i = 0; i < ORC_H; ++i) xf[i] = orc_bf16_to_f32(h[(size_t)m * ORC_H + i]);
#pragma omp parallel for schedule(static)
        for (int n = 0; n < ORC_L; ++n) {
            float up = orc_bf16_to_f32(ffn_proj_row(w, 0, xf, ORC_H, n));
            float gate = orc_bf16_to_f32(ffn_proj_row(w, 1, xf, ORC_H, n));
            /* gemma4.py:197: gelu(gate) (bf16 out) * up (bf16 out) */
            float a = orc_bf16_to_f32(orc_bf16_rne(orc_gelu_tanh(gate)));
            p[(size_t)m * ORC_L + n] = orc_bf16_rne(a * up);
        }
    }
    free(xf);
}

void orc_ffn_down(const uint16_t* p, const orc_ffn_weights* w, uint16_t* d, int M) {
    init_luts();
    float* xf = (float*)malloc(sizeof(float) * ORC_L);
    for (int m = 0; m < M; ++m) {
        for (int i = 0; i < ORC_L; ++i) xf[i] = orc_bf16_to_f32(p[(size_t)m * ORC_L + i]);
#pragma omp parallel for schedule(static)
        for (int n = 0; n < ORC_H; ++n) d[(size_t)m * ORC_H + n] = ffn_proj_row(w, 2, xf, ORC_L, n);
    }
    free(xf);
}

void orc_decoder_feedforward(uint16_t* residual, const uint16_t* pre_rms, const orc_ffn_weights* w,
                             const uint16_t* post_rms, const uint16_t* layer_scalar, int M) {
    if (M <= 0) return;
    uint16_t* h = (uint16_t*)malloc(2 * (size_t)ORC_H * M);
    uint16_t* p = (uint16_t*)malloc(2 * (size_t)ORC_L * M);
    uint16_t* d = (uint16_t*)malloc(2 * (size_t)ORC_H * M);
    uint16_t n[ORC_H];
    for (int m = 0; m < M; ++m) orc_rmsnorm_row(residual + (size_t)m * ORC_H, pre_rms, ORC_H, h + (size_t)m * ORC_H);
    orc_ffn_up_gate(h, w, p, M);
    orc_ffn_down(p, w, d, M);
    for (int m = 0; m < M; ++m) {
        const uint16_t* dm = d + (size_t)m * ORC_H;
        if (post_rms) orc_rmsnorm_row(dm, post_rms, ORC_H, n);
        else memcpy(n, dm, sizeof n);
        uint16_t* r = residual + (size_t)m * ORC_H;
        for (int i = 0; i < ORC_H; ++i) {
            /* generate_references.py:413: bf16(bf16(r + n) * layer_scalar[0]) */
            uint16_t s = orc_bf16_rne(orc_bf16_to_f32(r[i]) + orc_bf16_to_f32(n[i]));
            if (layer_scalar) s = orc_bf16_rne(orc_bf16_to_f32(s) * orc_bf16_to_f32(layer_scalar[0]));
            r[i] = s;
        }
    }
    free(h);
    free(p);
    free(d);
}

int orc_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
    return omp_get_max_threads();
#else
    (void)n;
    return 1;
#endif
}
