/*
 * bmx.h -- C ABI of the MI355X-native (gfx950) implementation of
 * base-mlx's 4-bit affine quantized matmul path (MLX format: uint32-packed
 * nibbles, group_size 64, bf16 per-group scales and biases) and the ops of
 * a Qwen3 decode step around it.
 *
 * Conventions (every entry point):
 *  - All tensor pointers are DEVICE pointers owned by the caller, row-major
 *    and contiguous unless a stride is given.  bf16 tensors are passed as
 *    raw 16-bit patterns (bmx_bf16).
 *  - `stream` is a hipStream_t (NULL = the default stream).  Calls enqueue
 *    work and return without synchronising.
 *  - Return value: 0 on success, a negative BMX_E_* code for an argument or
 *    shape error (nothing is enqueued), or a positive hipError_t.  The text
 *    for the last failure on the calling thread is bmx_last_error().  This
 *    mirrors mlx-c's `int` return, so a wrapper written like the reference's
 *    mlx_ext::slice_update (crates/base-mlx-core/src/mlx_ext.rs:58-61) maps
 *    rc != 0 to Error::Inference(String) unchanged.
 *  - No call aborts.  Calls are thread-compatible, not thread-safe per
 *    stream, like the reference's single-threaded model use
 *    (crates/base-mlx-server/src/state.rs:1-19).
 */
#ifndef BMX_H
#define BMX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t bmx_bf16;

#define BMX_OK 0
#define BMX_E_ARG (-1)         /* null pointer or invalid argument */
#define BMX_E_SHAPE (-2)       /* shape / size mismatch */
#define BMX_E_UNSUPPORTED (-3) /* bits != 4 or group_size != 64 */
#define BMX_E_KV_CAPACITY (-4) /* offset + M exceeds the KV capacity */
#define BMX_E_ALLOC (-5)       /* device allocation failed */
#define BMX_E_ALIGN (-6)       /* pointer alignment requirement not met */

/* Text of the last failure on this thread ("" if none). */
const char *bmx_last_error(void);
/* ABI version: (major << 16) | minor. */
int bmx_abi_version(void);

/* ------------------------------------------------------------------ */
/* Quantized matmul                                                    */
/* ------------------------------------------------------------------ */

/* y[M,N] = x[M,K] . dequant(w, scales, biases)^T   (transpose = true)
 * w: [N, K*bits/32] uint32; scales, biases: [N, K/group_size] bf16;
 * x, y bf16; fp32 accumulation.  bits must be 4 and group_size 64.
 * M <= 8 runs the streaming GEMV (qmv); larger M the MFMA GEMM (qmm).
 * x and w must be 16-byte aligned.
 * Replaces: mlx_rs::ops::quantized_matmul(x, w, scales, biases, true, 64, 4)
 *   as called by QLinear::forward (crates/base-mlx-core/src/model/qwen3.rs:30-41),
 *   QEmbedding::lm_head (qwen3.rs:80-91) and qkv_block / mlp_block
 *   (crates/base-mlx-core/src/model/kernels.rs:42-44, 69-75). */
int bmx_qmatmul_affine(const bmx_bf16 *x, const uint32_t *w, const bmx_bf16 *scales,
                       const bmx_bf16 *biases, bmx_bf16 *y, int64_t M, int64_t N, int64_t K,
                       int group_size, int bits, void *stream);

/* out[N,K] = scales * q + biases (fp32, rounded to bf16).
 * Replaces: mlx_rs::ops::dequantize(w, s, b, group_size, bits)
 *   (crates/base-mlx-core/src/model/qwen3.rs:75). */
int bmx_dequantize_affine(const uint32_t *w, const bmx_bf16 *scales, const bmx_bf16 *biases,
                          bmx_bf16 *out, int64_t N, int64_t K, int group_size, int bits,
                          void *stream);

/* out[m,:] = dequantize(row ids[m] of (w, scales, biases)), m < M.
 * ids are int32 token ids in [0, rows); an id outside that range yields a
 * zero row.
 * Replaces: QEmbedding::lookup = index(tokens) + dequantize
 *   (crates/base-mlx-core/src/model/qwen3.rs:67-76). */
int bmx_dequant_gather(const int32_t *ids, int64_t M, int64_t rows, const uint32_t *w,
                       const bmx_bf16 *scales, const bmx_bf16 *biases, bmx_bf16 *out, int64_t K,
                       int group_size, int bits, void *stream);

/* ------------------------------------------------------------------ */
/* Seeded random initialisation (the benchmark workloads use random-init */
/* weights; these kernels are bit-identical to the CPU generator).      */
/* No counterpart in the reference, which loads weights from            */
/* safetensors (crates/base-mlx-core/src/model/qwen3.rs:194-295).       */
/* ------------------------------------------------------------------ */

/* Element (n,k) = t * c with t the centred sum of the four 16-bit fields
 * of rand64(seed, n*K + k) (approx normal), quantized to MLX affine 4-bit
 * gs64 with the documented formula evaluated exactly on the integers t:
 * q = rne(15 (t - tmin) / (tmax - tmin)), s = (tmax - tmin) c / 15,
 * b = tmin c (the group minimum). */
int bmx_init_qlinear(uint64_t seed, int64_t N, int64_t K, float c, uint32_t *w,
                     bmx_bf16 *scales, bmx_bf16 *biases, void *stream);
/* out[i] = bf16(approx-normal(seed, i) * c) */
int bmx_fill_normal_bf16(uint64_t seed, int64_t n, float c, bmx_bf16 *out, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* BMX_H */
