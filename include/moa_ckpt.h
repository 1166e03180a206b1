/*
 * moa_ckpt.h -- C ABI of the checkpoint reader: the reference's on-disk format
 * (FO/src/host/load.rs), one safetensors file, read into caller-owned device buffers.
 *
 * A handle maps the file read-only and parses its header once. The typed loaders check a
 * tensor's dtype and shape the way load.rs does before anything is copied, then copy it to
 * `dst` (device memory) through two pinned staging buffers on `stream`, returning when the
 * bytes are on the device. A handle is used by one thread at a time.
 *
 * Return value: MOA_SUCCESS or a negative MOA_ERROR_* code (moa_ops.h); moa_last_error_string()
 * names the tensor and the mismatch. MOA_ERROR_NOT_FOUND: no tensor of that name;
 * MOA_ERROR_FORMAT: a malformed file or a tensor of another dtype or shape.
 */
#ifndef MOA_CKPT_H
#define MOA_CKPT_H

#include <stdint.h>

#include "moa_ops.h"

#ifdef __cplusplus
extern "C" {
#endif

#define MOA_ERROR_NOT_FOUND (-6) /* no tensor of that name in the checkpoint */
#define MOA_ERROR_FORMAT (-7)    /* malformed file, or a dtype / shape other than the one required */
#define MOA_ERROR_IO (-8)        /* the file cannot be opened or mapped */

typedef struct moa_ckpt moa_ckpt;

/* Maps `path` and parses the safetensors header (8-byte little-endian length, JSON table of
 * dtype, shape and data_offsets per tensor). Every tensor's byte range must lie in the file and
 * match its dtype and shape. Replaces safetensors::SafeTensors::deserialize over the mmap in
 * load_model (FO/src/host/load.rs:356-360). */
int moa_ckpt_open(const char* path, moa_ckpt** out);
/* Unmaps the file and frees the staging buffers. */
int moa_ckpt_close(moa_ckpt* ckpt);

/* Number of tensors, and the name of tensor `index` (in header order; valid until close). */
int moa_ckpt_count(const moa_ckpt* ckpt, int* count);
int moa_ckpt_name(const moa_ckpt* ckpt, int index, const char** name);
/* dtype string as stored ("BF16", "F8_E4M3", "U8", "F32", ...; valid until close), up to 8
 * dims into shape[], their count and the byte size. Replaces tensors.tensor(name)?. */
int moa_ckpt_info(const moa_ckpt* ckpt, const char* name, const char** dtype, int64_t* shape, int* ndim,
                  uint64_t* nbytes);
/* Copies the raw bytes of `name` to host memory; nbytes must equal the tensor's size. */
int moa_ckpt_read(const moa_ckpt* ckpt, const char* name, void* host_dst, uint64_t nbytes);

/* load_bf16 (load.rs:93-101): BF16 of exactly `shape` (ndim <= 8). */
int moa_ckpt_load_bf16(moa_ckpt* ckpt, const char* name, const int64_t* shape, int ndim, void* dst, void* stream);
/* load_bf16_column (load.rs:117-135): BF16 [n, 1] (per-channel FP8 weight scales). */
int moa_ckpt_load_bf16_column(moa_ckpt* ckpt, const char* name, int64_t n, void* dst, void* stream);
/* load_f8 (load.rs:131-140): F8_E4M3 [rows, cols] (FP8 weights, NVFP4 block scales). */
int moa_ckpt_load_f8(moa_ckpt* ckpt, const char* name, int64_t rows, int64_t cols, void* dst, void* stream);
/* load_f4 (load.rs:142-160): E2M1 codes packed two per byte, low nibble first, stored as
 * U8 [rows, cols / 2]. */
int moa_ckpt_load_f4(moa_ckpt* ckpt, const char* name, int64_t rows, int64_t cols, void* dst, void* stream);
/* load_scalar_bf16 (load.rs:103-115): a BF16 [1] value written 8 times (the layer scalar's
 * 16-byte operand). */
int moa_ckpt_load_scalar_bf16(moa_ckpt* ckpt, const char* name, void* dst, void* stream);
/* reciprocal_global_scale (load.rs:162-179): the F32 scalar g of an NVFP4 projection, returned
 * as 1 / g; g = 0 or a non-finite g is MOA_ERROR_FORMAT. */
int moa_ckpt_global_scale(const moa_ckpt* ckpt, const char* name, float* reciprocal);
/* load_global_scale (load.rs:181-190): 1 / g stored as one f32 on the device. */
int moa_ckpt_load_global_scale(moa_ckpt* ckpt, const char* name, void* dst, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOA_CKPT_H */
