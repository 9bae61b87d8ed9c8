/*
 * bmx_oracle.h -- CPU restatement of base-mlx's 4-bit affine quantized
 * matmul path (MLX format) and of the Qwen3 forward that calls it.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library under
 * base-mlx_amd/) links, loads or calls this code.  It is used by tests/ as
 * the parity checker, by __graft_entry__.smoke() as the checker, and by
 * bench.py's cpu_baseline leg as the timed CPU restatement.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the reference checkout).  Arithmetic that lives inside
 * MLX itself (not vendored in the reference) follows MLX's documented
 * semantics and is marked [MLX upstream].
 *
 * Conventions: bf16 values are passed as raw uint16_t bit patterns; all
 * arrays are row-major and contiguous; fp32 accumulation, bf16 outputs
 * rounded to nearest-even, as the reference's bf16 models produce.
 *
 * Pinning.  The reference holds no tests or golden vectors for this path
 * and cannot be built or imported here (Rust over mlx-rs; MLX's kernels are
 * Metal), so each function is checked against closed forms, library
 * routines and invariants (tests/test_oracle_*.py) and against the
 * closed-form fixtures of tests/golden/ (tests/test_golden.py).  Parity
 * unpinned -- only an MLX import could pin these bits: the exact output of
 * MLX's own quantizer (orc_quantize_affine follows the documented formula;
 * op parity does not depend on it since both sides consume the same packed
 * tensors), the accumulation order inside MLX's quantized_matmul, the
 * internal precision of MLX's fast::rms_norm / rope / SDPA, MLX's
 * end-to-end logits and its argmax tie-break.
 */
#ifndef BMX_ORACLE_H
#define BMX_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalars -------------------------------------------------------- */
uint16_t orc_f2bf(float f);
float orc_bf2f(uint16_t h);

/* ---- seeded counter-based generator (shared bit-exactly with the GPU) - */
uint64_t orc_rand64(uint64_t seed, uint64_t idx);
uint64_t orc_tensor_seed(uint64_t model_seed, int layer, int slot);
/* Approximately normal deviate t*c with t = (sum of the four 16-bit fields
 * of orc_rand64(seed, idx)) - 131070; c = sigma / 37837.2262.. */
float orc_normal_at(uint64_t seed, uint64_t idx, float c);
float orc_sigma_to_c(double sigma);
void orc_fill_normal_bf16(uint64_t seed, int64_t n, float c, uint16_t *out);
void orc_fill_normal_f32(uint64_t seed, int64_t n, float c, float *out);
void orc_fill_tokens(uint64_t seed, int64_t n, uint32_t vocab, uint32_t *out);

/* ---- MLX affine quantization format --------------------------------- */
int orc_quantize_affine(const float *w, int64_t N, int64_t K, int gs, int bits,
                        uint32_t *wq, uint16_t *s, uint16_t *b);
void orc_init_qlinear(uint64_t seed, int64_t N, int64_t K, float c,
                      uint32_t *wq, uint16_t *s, uint16_t *b);
int orc_dequantize(const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                   int64_t N, int64_t K, int gs, int bits, uint16_t *out);
int orc_dequant_gather(const uint32_t *ids, int64_t M, int64_t rows,
                       const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                       int64_t K, int gs, int bits, uint16_t *out);
int orc_qmatmul(const uint16_t *x, const uint32_t *wq, const uint16_t *s,
                const uint16_t *b, uint16_t *y, int64_t M, int64_t N, int64_t K,
                int gs, int bits);
int orc_qmm_dequant(const uint16_t *x, const uint32_t *wq, const uint16_t *s,
                    const uint16_t *b, uint16_t *y, int64_t M, int64_t N,
                    int64_t K, int gs, int bits);
int orc_qlinear(const uint16_t *x, const uint32_t *wq, const uint16_t *s,
                const uint16_t *b, uint16_t *y, int64_t M, int64_t N, int64_t K,
                int gs, int bits);
int orc_gather_qmm(const uint16_t *x, const uint32_t *wq, const uint16_t *s,
                   const uint16_t *b, const uint32_t *rhs, uint16_t *y,
                   int64_t R, int64_t x_bcast, int64_t E, int64_t M, int64_t N,
                   int64_t K, int gs, int bits);
int orc_qmatmul_f64(const uint16_t *x, const uint32_t *wq, const uint16_t *s,
                    const uint16_t *b, double *y, int64_t M, int64_t N,
                    int64_t K, int gs, int bits);

/* ---- ops around the matmul ------------------------------------------ */
void orc_rms_norm(const uint16_t *x, const uint16_t *w, uint16_t *y,
                  int64_t rows, int64_t dim, float eps);
void orc_rope(const uint16_t *x, uint16_t *y, int64_t H, int64_t T, int64_t D,
              float theta, int64_t offset);
int orc_slice_update(uint16_t *src, int ndim, const int64_t *shape,
                     const uint16_t *update, const int64_t *start,
                     const int64_t *stop, const int64_t *strides);
void orc_sdpa(const uint16_t *q, const uint16_t *k, const uint16_t *v,
              uint16_t *out, int64_t Hq, int64_t Hkv, int64_t M, int64_t L,
              int64_t D, int64_t kv_stride, int64_t offset, int causal,
              float scale);
void orc_silu_mul(const uint16_t *g, const uint16_t *u, uint16_t *y, int64_t n);
void orc_add(const uint16_t *a, const uint16_t *b, uint16_t *y, int64_t n);
void orc_argmax_rows(const uint16_t *x, int64_t rows, int64_t n, uint32_t *out);
/* Test knob: reverse the order of every fp32 reduction (GEMV, GEMM, SDPA,
 * RMSNorm): measures the spread summation order alone causes.  Default off. */
void orc_set_reverse_accumulation(int on);

/* ---- Qwen3 model ----------------------------------------------------- */
typedef struct {
  int hidden, inter, layers, n_heads, n_kv_heads, head_dim, vocab;
  int tied, group_size, bits;
  float eps, rope_theta;
} orc_qwen3_config;

typedef struct orc_qwen3 orc_qwen3;
typedef struct orc_kv orc_kv;

orc_qwen3 *orc_qwen3_create_random(const orc_qwen3_config *cfg, uint64_t seed,
                                   double sigma);
void orc_qwen3_free(orc_qwen3 *m);
int orc_qwen3_qlinear(orc_qwen3 *m, int layer, int slot, uint32_t **w,
                      uint16_t **s, uint16_t **b, int *N, int *K);
uint16_t *orc_qwen3_norm(orc_qwen3 *m, int layer, int which);

orc_kv *orc_kv_create(const orc_qwen3 *m, int capacity);
void orc_kv_free(orc_kv *kv);
int orc_kv_seq_len(const orc_kv *kv);
int orc_kv_capacity(const orc_kv *kv);
void orc_kv_reset(orc_kv *kv);
void orc_kv_truncate(orc_kv *kv, int target);
uint16_t *orc_kv_data(orc_kv *kv);
void orc_kv_fill_synthetic(orc_kv *kv, uint64_t seed, int seq_len);

int orc_qwen3_forward(orc_qwen3 *m, orc_kv *kv, const uint32_t *tokens, int M,
                      int all_logits, uint16_t *logits);
int orc_generate_greedy(orc_qwen3 *m, orc_kv *kv, const uint32_t *prompt,
                        int P, int max_new, const uint32_t *eos, int n_eos,
                        uint32_t *out, int *n_out);
int orc_speculative_generate(orc_qwen3 *target, orc_kv *tkv, orc_qwen3 *draft,
                             orc_kv *dkv, const uint32_t *prompt, int P,
                             int max_new, int spec_k, const uint32_t *eos,
                             int n_eos, uint32_t *out, int *n_out,
                             int64_t *stats);

/* host measurement helpers for the CPU baseline */
int orc_num_threads(void);
double orc_stream_triad_gbs(int64_t n, int reps);

/* error codes shared with the HIP library */
#define ORC_OK 0
#define ORC_E_ARG (-1)
#define ORC_E_SHAPE (-2)
#define ORC_E_UNSUPPORTED (-3)
#define ORC_E_KV_CAPACITY (-4)
#define ORC_E_ALLOC (-5)

#ifdef __cplusplus
}
#endif
#endif
