/*
 * bmx_oracle.c -- CPU restatement (C11 + OpenMP) of base-mlx's quantized
 * matmul path and Qwen3 forward.  TEST INFRASTRUCTURE ONLY: used by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the
 * product library.
 *
 * Reference behaviour restated here (paths relative to the reference tree):
 *   QLinear::forward -> quantized_matmul(x, W, s, b, transpose=true, 64, 4)
 *       crates/base-mlx-core/src/model/qwen3.rs:18-42
 *   QEmbedding::lookup / lm_head        qwen3.rs:57-92
 *   RmsNorm::forward (fast::rms_norm)   qwen3.rs:44-55
 *   qkv_block / mlp_block               crates/base-mlx-core/src/model/kernels.rs:28-78
 *   KvCache + truncate                  qwen3.rs:109-162
 *   forward_internal                    qwen3.rs:314-563
 *   causal_mask_offset                  qwen3.rs:629-653
 *   mlx_ext::slice_update               crates/base-mlx-core/src/mlx_ext.rs:21-64
 *   greedy decode loop / pick_next      crates/base-mlx-core/src/engine.rs:89-202
 *   speculative::generate               crates/base-mlx-core/src/speculative.rs:57-293
 *
 * Built with -ffp-contract=off so that every float operation rounds once,
 * exactly as written; the generator and quantizer below are therefore
 * bit-identical to the HIP kernels that restate them.
 */
#include "bmx_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* bf16 <-> f32                                                        */
/* ------------------------------------------------------------------ */
static inline float bf2f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static inline uint16_t f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u); /* round to nearest even */
  return (uint16_t)(u >> 16);
}
uint16_t orc_f2bf(float f) { return f2bf(f); }
float orc_bf2f(uint16_t h) { return bf2f(h); }

/* ------------------------------------------------------------------ */
/* Counter-based generator.  Weights in the benchmark configurations   */
/* are seeded random-init; this generator is restated bit-exactly by   */
/* the device init kernels so CPU and GPU hold identical tensors.      */
/* ------------------------------------------------------------------ */
static inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
uint64_t orc_rand64(uint64_t seed, uint64_t idx) {
  return mix64(mix64(seed) + (idx + 1u) * 0x9E3779B97F4A7C15ull);
}
uint64_t orc_tensor_seed(uint64_t model_seed, int layer, int slot) {
  return mix64(model_seed * 0xD1B54A32D192ED03ull +
               (uint64_t)(int64_t)(layer + 16) * 64u + (uint64_t)slot);
}
static inline int32_t irwin4(uint64_t r) {
  return (int32_t)((r & 0xffffu) + ((r >> 16) & 0xffffu) +
                   ((r >> 32) & 0xffffu) + ((r >> 48) & 0xffffu)) -
         131070;
}
/* standard deviation of the sum of four uniform 16-bit integers */
#define IRWIN4_STD 37837.226523565 /* sqrt((65536^2 - 1) / 3) */
float orc_sigma_to_c(double sigma) { return (float)(sigma / IRWIN4_STD); }
float orc_normal_at(uint64_t seed, uint64_t idx, float c) {
  return (float)irwin4(orc_rand64(seed, idx)) * c;
}
void orc_fill_normal_bf16(uint64_t seed, int64_t n, float c, uint16_t *out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; i++) out[i] = f2bf(orc_normal_at(seed, (uint64_t)i, c));
}
void orc_fill_normal_f32(uint64_t seed, int64_t n, float c, float *out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; i++) out[i] = orc_normal_at(seed, (uint64_t)i, c);
}
void orc_fill_tokens(uint64_t seed, int64_t n, uint32_t vocab, uint32_t *out) {
  for (int64_t i = 0; i < n; i++)
    out[i] = (uint32_t)(orc_rand64(seed, (uint64_t)i) % (uint64_t)vocab);
}

/* ------------------------------------------------------------------ */
/* MLX affine quantization [MLX upstream, documented formula]:         */
/*   per group of gs consecutive weights along K:                      */
/*   alpha = max w, beta = min w, s = (alpha - beta) / (2^bits - 1),   */
/*   q = clip(round_half_even((w - beta) / s), 0, 2^bits - 1), b = beta */
/*   W packs element k of a row into word k / (32/bits) at bit         */
/*   offset bits * (k mod (32/bits)), lowest bits first.               */
/* Shapes follow the reference's packed-shape relation                 */
/*   bits = W_last * 32 / (S_last * gs)   (gemma.rs:760-779)           */
/* ------------------------------------------------------------------ */
static void quantize_group(const float *w, int gs, uint32_t *wq, uint16_t *s,
                           uint16_t *b) {
  float hi = w[0], lo = w[0];
  for (int i = 1; i < gs; i++) {
    hi = w[i] > hi ? w[i] : hi;
    lo = w[i] < lo ? w[i] : lo;
  }
  float sc = (hi - lo) / 15.0f;
  if (!(sc > 0.0f)) sc = 1e-7f;
  for (int i = 0; i < gs / 8; i++) wq[i] = 0;
  for (int i = 0; i < gs; i++) {
    float qf = rintf((w[i] - lo) / sc);
    int q = (int)qf;
    q = q < 0 ? 0 : (q > 15 ? 15 : q);
    wq[i >> 3] |= (uint32_t)q << (4 * (i & 7));
  }
  *s = f2bf(sc);
  *b = f2bf(lo);
}

int orc_quantize_affine(const float *w, int64_t N, int64_t K, int gs, int bits,
                        uint32_t *wq, uint16_t *s, uint16_t *b) {
  if (bits != 4) return ORC_E_UNSUPPORTED;
  if (gs <= 0 || gs % 8 || K % gs) return ORC_E_SHAPE;
  int64_t G = K / gs;
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; n++)
    for (int64_t g = 0; g < G; g++)
      quantize_group(w + n * K + g * gs, gs, wq + n * (K / 8) + g * (gs / 8),
                     s + n * G + g, b + n * G + g);
  return ORC_OK;
}

/* Random-init projection.  Element (n, k) is the deviate t * c with
 * t = irwin4(rand64(seed, n*K + k)) (approx N(0, sigma) for
 * c = sigma / IRWIN4_STD).  The documented affine formula is evaluated
 * exactly on the integer deviates, so the CPU and GPU agree bit for bit:
 *   q    = round_half_even(15 (t - tmin) / (tmax - tmin))   (integer)
 *   s    = bf16(float((tmax - tmin) * c * (1/15)))           (double math)
 *   b    = bf16(tmin * c)                                    (= group min) */
static void quantize_group_int(const int32_t *t, float c, uint32_t *wq,
                               uint16_t *s, uint16_t *b) {
  int32_t hi = t[0], lo = t[0];
  for (int i = 1; i < 64; i++) {
    hi = t[i] > hi ? t[i] : hi;
    lo = t[i] < lo ? t[i] : lo;
  }
  const int32_t den = hi - lo;
  for (int i = 0; i < 8; i++) wq[i] = 0;
  for (int i = 0; i < 64; i++) {
    int32_t q = 0;
    if (den > 0) {
      int32_t num = 15 * (t[i] - lo);
      q = num / den;
      int32_t r = num - q * den;
      if (2 * r > den || (2 * r == den && (q & 1))) q++;
    }
    wq[i >> 3] |= (uint32_t)q << (4 * (i & 7));
  }
  double sd = den > 0 ? (double)den * (double)c * (1.0 / 15.0) : 1e-7;
  *s = f2bf((float)sd);
  *b = f2bf((float)lo * c);
}

void orc_init_qlinear(uint64_t seed, int64_t N, int64_t K, float c,
                      uint32_t *wq, uint16_t *s, uint16_t *b) {
  int64_t G = K / 64;
  uint64_t ms = mix64(seed);
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; n++) {
    int32_t tmp[64];
    for (int64_t g = 0; g < G; g++) {
      uint64_t base = (uint64_t)(n * K + g * 64);
      for (int i = 0; i < 64; i++)
        tmp[i] = irwin4(mix64(ms + (base + (uint64_t)i + 1u) * 0x9E3779B97F4A7C15ull));
      quantize_group_int(tmp, c, wq + n * (K / 8) + g * 8, s + n * G + g, b + n * G + g);
    }
  }
}

static inline float dq_elem(const uint32_t *row, const uint16_t *srow,
                            const uint16_t *brow, int64_t k, int gs) {
  uint32_t q = (row[k >> 3] >> (4 * (k & 7))) & 0xfu;
  /* s*q is exact in fp32 (8-bit by 4-bit significands), one rounding */
  return bf2f(srow[k / gs]) * (float)q + bf2f(brow[k / gs]);
}

/* mlx_rs::ops::dequantize as called by QEmbedding::lookup (qwen3.rs:69-76):
 * value = s * q + b in fp32, rounded to the bf16 output dtype. */
int orc_dequantize(const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                   int64_t N, int64_t K, int gs, int bits, uint16_t *out) {
  if (bits != 4) return ORC_E_UNSUPPORTED;
  if (gs <= 0 || gs % 8 || K % gs) return ORC_E_SHAPE;
  int64_t G = K / gs;
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; n++)
    for (int64_t k = 0; k < K; k++)
      out[n * K + k] = f2bf(dq_elem(wq + n * (K / 8), s + n * G, b + n * G, k, gs));
  return ORC_OK;
}

/* QEmbedding::lookup (qwen3.rs:67-76): gather rows by id, then dequantize. */
int orc_dequant_gather(const uint32_t *ids, int64_t M, int64_t rows,
                       const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                       int64_t K, int gs, int bits, uint16_t *out) {
  if (bits != 4) return ORC_E_UNSUPPORTED;
  if (gs <= 0 || gs % 8 || K % gs) return ORC_E_SHAPE;
  int64_t G = K / gs;
  for (int64_t m = 0; m < M; m++)
    if ((int64_t)ids[m] >= rows) return ORC_E_ARG;
  for (int64_t m = 0; m < M; m++) {
    int64_t n = ids[m];
    for (int64_t k = 0; k < K; k++)
      out[m * K + k] = f2bf(dq_elem(wq + n * (K / 8), s + n * G, b + n * G, k, gs));
  }
  return ORC_OK;
}

/* Accumulation-order variant, for measuring the end-to-end spread that fp32
 * summation order alone causes (a test measures the oracle against itself
 * with this on): every fp32 reduction runs in the opposite order -- the
 * GEMV adds its groups last to first, the GEMM its 8-wide k blocks, SDPA its
 * keys and RMSNorm (incl. the per-head QK-norm) its squares.  Off by
 * default; not thread-safe to toggle while a call runs. */
static int g_reverse = 0;
void orc_set_reverse_accumulation(int on) { g_reverse = on ? 1 : 0; }

/* quantized_matmul(x, W, s, b, transpose=true, gs, 4) [MLX upstream]:
 *   y[m, n] = sum_g ( s[n,g] * sum_{k in g} q[n,k] x[m,k]
 *                    + b[n,g] * sum_{k in g} x[m,k] )
 * fp32 accumulation, bf16 result.  Call sites: qwen3.rs:30-41, 80-91;
 * kernels.rs:42-44, 69-75. */
int orc_qmatmul(const uint16_t *x, const uint32_t *wq, const uint16_t *s,
                const uint16_t *b, uint16_t *y, int64_t M, int64_t N, int64_t K,
                int gs, int bits) {
  if (bits != 4) return ORC_E_UNSUPPORTED;
  if (gs != 64 || K % 64) return ORC_E_SHAPE;
  const int64_t G = K / 64;
  float *xf = (float *)malloc(sizeof(float) * (size_t)(M * K));
  float *sx = (float *)malloc(sizeof(float) * (size_t)(M * G));
  if (!xf || !sx) {
    free(xf);
    free(sx);
    return ORC_E_ALLOC;
  }
  for (int64_t i = 0; i < M * K; i++) xf[i] = bf2f(x[i]);
  for (int64_t m = 0; m < M; m++)
    for (int64_t g = 0; g < G; g++) {
      float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      const float *xp = xf + m * K + g * 64;
      for (int i = 0; i < 64; i += 8)
        for (int j = 0; j < 8; j++) a[j] += xp[i + j];
      sx[m * G + g] = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
    }
#pragma omp parallel for schedule(dynamic, 16)
  for (int64_t n = 0; n < N; n++) {
    const uint32_t *row = wq + n * (K / 8);
    float qrow[64];
    for (int64_t m = 0; m < M; m++) {
      float acc = 0.0f;
      for (int64_t gi = 0; gi < G; gi++) {
        const int64_t g = g_reverse ? G - 1 - gi : gi;
        const uint32_t *wg = row + g * 8;
        for (int i = 0; i < 8; i++) {
          uint32_t w = wg[i];
          for (int j = 0; j < 8; j++) qrow[i * 8 + j] = (float)((w >> (4 * j)) & 0xfu);
        }
        const float *xp = xf + m * K + g * 64;
        float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int i = 0; i < 64; i += 8)
          for (int j = 0; j < 8; j++) a[j] += qrow[i + j] * xp[i + j];
        float dq = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
        acc += bf2f(s[n * G + g]) * dq;
        acc += bf2f(b[n * G + g]) * sx[m * G + g];
      }
      y[m * N + n] = f2bf(acc);
    }
  }
  free(xf);
  free(sx);
  return ORC_OK;
}

/* The matrix path of quantized_matmul (MLX runs its qmm kernel for
 * matrices and its qmv kernel for a few rows; the HIP library takes this
 * path for M > 8 rows): every weight row is dequantized to bf16 -- the bits
 * orc_dequantize returns, s*q + b with one rounding -- and y = x w^T
 * accumulates in fp32, rounded to bf16 [MLX upstream: the Metal qmm loader
 * dequantizes each weight tile to the input dtype in threadgroup memory
 * before its GEMM].  Parity unpinned at one bf16 ulp of w: MLX's loader
 * rounds s*q and the sum separately. */
int orc_qmm_dequant(const uint16_t *x, const uint32_t *wq, const uint16_t *s,
                    const uint16_t *b, uint16_t *y, int64_t M, int64_t N,
                    int64_t K, int gs, int bits) {
  if (bits != 4) return ORC_E_UNSUPPORTED;
  if (gs != 64 || K % 64) return ORC_E_SHAPE;
  const int64_t G = K / 64;
  float *xf = (float *)malloc(sizeof(float) * (size_t)(M * K));
  if (!xf) return ORC_E_ALLOC;
  for (int64_t i = 0; i < M * K; i++) xf[i] = bf2f(x[i]);
  int fail = 0;
#pragma omp parallel
  {
    float *wrow = (float *)malloc(sizeof(float) * (size_t)K);
    if (!wrow) {
#pragma omp atomic write
      fail = 1;
    } else {
#pragma omp for schedule(dynamic, 16)
      for (int64_t n = 0; n < N; n++) {
        for (int64_t k = 0; k < K; k++)
          wrow[k] = bf2f(f2bf(dq_elem(wq + n * (K / 8), s + n * G, b + n * G, k, 64)));
        for (int64_t m = 0; m < M; m++) {
          const float *xp = xf + m * K;
          float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
          for (int64_t ki = 0; ki < K; ki += 8) {
            const int64_t k = g_reverse ? K - 8 - ki : ki;
            for (int j = 0; j < 8; j++) a[j] += wrow[k + j] * xp[k + j];
          }
          y[m * N + n] = f2bf(((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7])));
        }
      }
      free(wrow);
    }
  }
  free(xf);
  return fail ? ORC_E_ALLOC : ORC_OK;
}

/* QLinear::forward (qwen3.rs:30-41) as the HIP library evaluates it: the
 * group-decomposition GEMV for up to 8 rows of x, the dequantizing GEMM
 * beyond. */
int orc_qlinear(const uint16_t *x, const uint32_t *wq, const uint16_t *s,
                const uint16_t *b, uint16_t *y, int64_t M, int64_t N, int64_t K,
                int gs, int bits) {
  if (M <= 8) return orc_qmatmul(x, wq, s, b, y, M, N, K, gs, bits);
  return orc_qmm_dequant(x, wq, s, b, y, M, N, K, gs, bits);
}

/* gather_qmm (mlx_ext.rs:66-117) as QSwitchLinear::forward calls it
 * (granite.rs:74-88): route r multiplies x block r / x_bcast by expert
 * rhs[r] of the stacked [E, N, K/8] weights, with quantized_matmul's
 * numerics for each route (M <= 8 rows: the GEMV group decomposition).
 * Expert ids >= E are clamped to E - 1, as the HIP library does. */
int orc_gather_qmm(const uint16_t *x, const uint32_t *wq, const uint16_t *s,
                   const uint16_t *b, const uint32_t *rhs, uint16_t *y,
                   int64_t R, int64_t x_bcast, int64_t E, int64_t M, int64_t N,
                   int64_t K, int gs, int bits) {
  if (bits != 4) return ORC_E_UNSUPPORTED;
  if (gs != 64 || K % 64 || E <= 0 || x_bcast <= 0 || M <= 0 || M > 8) return ORC_E_SHAPE;
  const int64_t G = K / 64;
  for (int64_t r = 0; r < R; r++) {
    const int64_t e = rhs[r] < (uint32_t)E ? (int64_t)rhs[r] : E - 1;
    int rc = orc_qmatmul(x + (r / x_bcast) * M * K, wq + e * N * (K / 8), s + e * N * G, b + e * N * G,
                         y + r * M * N, M, N, K, gs, bits);
    if (rc) return rc;
  }
  return ORC_OK;
}

/* Same product evaluated in float64 on the dequantized weights
 * (s*q + b exact in double); the high-precision yardstick for tests. */
int orc_qmatmul_f64(const uint16_t *x, const uint32_t *wq, const uint16_t *s,
                    const uint16_t *b, double *y, int64_t M, int64_t N,
                    int64_t K, int gs, int bits) {
  if (bits != 4) return ORC_E_UNSUPPORTED;
  if (gs <= 0 || gs % 8 || K % gs) return ORC_E_SHAPE;
  const int64_t G = K / gs;
#pragma omp parallel for schedule(dynamic, 16)
  for (int64_t n = 0; n < N; n++) {
    const uint32_t *row = wq + n * (K / 8);
    for (int64_t m = 0; m < M; m++) {
      double acc = 0.0;
      for (int64_t k = 0; k < K; k++) {
        uint32_t q = (row[k >> 3] >> (4 * (k & 7))) & 0xfu;
        double wv = (double)bf2f(s[n * G + k / gs]) * (double)q +
                    (double)bf2f(b[n * G + k / gs]);
        acc += wv * (double)bf2f(x[m * K + k]);
      }
      y[m * N + n] = acc;
    }
  }
  return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* fast::rms_norm (qwen3.rs:44-55; kernels.rs:41, 68) [MLX upstream]:  */
/*   y = w * bf16(x * rsqrt(mean(x^2) + eps)), fp32 internally.        */
/* ------------------------------------------------------------------ */
void orc_rms_norm(const uint16_t *x, const uint16_t *w, uint16_t *y,
                  int64_t rows, int64_t dim, float eps) {
#pragma omp parallel for schedule(static) if (rows > 64)
  for (int64_t r = 0; r < rows; r++) {
    const uint16_t *xr = x + r * dim;
    float ss = 0.0f;
    for (int64_t ii = 0; ii < dim; ii++) {
      const int64_t i = g_reverse ? dim - 1 - ii : ii;
      float v = bf2f(xr[i]);
      ss += v * v;
    }
    float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int64_t i = 0; i < dim; i++) {
      float nrm = bf2f(f2bf(bf2f(xr[i]) * inv));
      y[r * dim + i] = f2bf(bf2f(w[i]) * nrm);
    }
  }
}

/* ------------------------------------------------------------------ */
/* fast::rope(x, dims=D, traditional=false, base=theta, scale=1, off)   */
/* (qwen3.rs:407-413) [MLX upstream]: rotate-half over the last axis;  */
/* for i < D/2, angle = (off + t) * theta^(-i/(D/2)),                   */
/*   y_i = x_i cos - x_{i+D/2} sin,  y_{i+D/2} = x_i sin + x_{i+D/2} cos */
/* x is [H, T, D] (heads, sequence, head_dim).                          */
/* The inverse frequencies are evaluated in double and rounded to       */
/* float once; the GPU kernel uses the same table.                      */
/* ------------------------------------------------------------------ */
void orc_rope(const uint16_t *x, uint16_t *y, int64_t H, int64_t T, int64_t D,
              float theta, int64_t offset) {
  int64_t half = D / 2;
  float *invf = (float *)malloc(sizeof(float) * (size_t)half);
  for (int64_t i = 0; i < half; i++)
    invf[i] = (float)pow((double)theta, -(double)i / (double)half);
  for (int64_t h = 0; h < H; h++)
    for (int64_t t = 0; t < T; t++) {
      const uint16_t *xr = x + (h * T + t) * D;
      uint16_t *yr = y + (h * T + t) * D;
      float pos = (float)(offset + t);
      for (int64_t i = 0; i < half; i++) {
        float ang = pos * invf[i];
        float c = cosf(ang), sn = sinf(ang);
        float a = bf2f(xr[i]), bb = bf2f(xr[i + half]);
        float o1 = a * c - bb * sn;
        float o2 = a * sn + bb * c;
        yr[i] = f2bf(o1);
        yr[i + half] = f2bf(o2);
      }
    }
  free(invf);
}

/* ------------------------------------------------------------------ */
/* mlx_ext::slice_update (mlx_ext.rs:21-64): numpy semantics           */
/*   src[start_0:stop_0:stride_0, ...] = update   (in place)           */
/* update must have the slice's shape; positive strides only.          */
/* ------------------------------------------------------------------ */
int orc_slice_update(uint16_t *src, int ndim, const int64_t *shape,
                     const uint16_t *update, const int64_t *start,
                     const int64_t *stop, const int64_t *strides) {
  if (ndim <= 0 || ndim > 8) return ORC_E_ARG;
  int64_t ext[8], sstride[8], total = 1;
  for (int d = 0; d < ndim; d++) {
    if (strides[d] <= 0 || start[d] < 0 || stop[d] > shape[d]) return ORC_E_SHAPE;
    ext[d] = stop[d] > start[d] ? (stop[d] - start[d] + strides[d] - 1) / strides[d] : 0;
    total *= ext[d];
  }
  sstride[ndim - 1] = 1;
  for (int d = ndim - 2; d >= 0; d--) sstride[d] = sstride[d + 1] * shape[d + 1];
  for (int64_t i = 0; i < total; i++) {
    int64_t rem = i, off = 0;
    for (int d = ndim - 1; d >= 0; d--) {
      int64_t c = rem % ext[d];
      rem /= ext[d];
      off += (start[d] + c * strides[d]) * sstride[d];
    }
    src[off] = update[i];
  }
  return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* fast::scaled_dot_product_attention with GQA (qwen3.rs:491-518)      */
/* [MLX upstream]: softmax(scale * q k^T + mask) v in fp32, bf16 out.  */
/* q: [Hq, M, D]; k, v: [Hkv, kv_stride, D] (first L rows used);        */
/* query head h reads kv head h / (Hq / Hkv).  causal: the additive     */
/* -1e9 mask of causal_mask_offset (qwen3.rs:629-653) -- query t may   */
/* attend keys j <= offset + t; masked keys contribute exactly 0.      */
/* out: [M, Hq * D] (the reference's transpose + reshape).             */
/* ------------------------------------------------------------------ */
void orc_sdpa(const uint16_t *q, const uint16_t *k, const uint16_t *v,
              uint16_t *out, int64_t Hq, int64_t Hkv, int64_t M, int64_t L,
              int64_t D, int64_t kv_stride, int64_t offset, int causal,
              float scale) {
  int64_t rep = Hq / Hkv;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int64_t h = 0; h < Hq; h++)
    for (int64_t t = 0; t < M; t++) {
      const uint16_t *qr = q + (h * M + t) * D;
      const uint16_t *kh = k + (h / rep) * kv_stride * D;
      const uint16_t *vh = v + (h / rep) * kv_stride * D;
      int64_t nk = causal ? offset + t + 1 : L;
      if (nk > L) nk = L;
      float *sc = (float *)malloc(sizeof(float) * (size_t)(nk > 0 ? nk : 1));
      float *acc = (float *)calloc((size_t)D, sizeof(float));
      float qs[512];
      for (int64_t d = 0; d < D; d++) qs[d] = bf2f(qr[d]) * scale;
      float mx = -INFINITY;
      for (int64_t j = 0; j < nk; j++) {
        float a = 0.0f;
        for (int64_t d = 0; d < D; d++) a += qs[d] * bf2f(kh[j * D + d]);
        sc[j] = a;
        mx = a > mx ? a : mx;
      }
      float l = 0.0f;
      for (int64_t ji = 0; ji < nk; ji++) {
        const int64_t j = g_reverse ? nk - 1 - ji : ji;
        float p = expf(sc[j] - mx);
        l += p;
        for (int64_t d = 0; d < D; d++) acc[d] += p * bf2f(vh[j * D + d]);
      }
      for (int64_t d = 0; d < D; d++) out[t * Hq * D + h * D + d] = f2bf(acc[d] / l);
      free(sc);
      free(acc);
    }
}

/* mlp_block activation (kernels.rs:73-74): silu(g) = g * sigmoid(g),
 * each MLX op rounding to bf16, then * up. */
void orc_silu_mul(const uint16_t *g, const uint16_t *u, uint16_t *y, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    float gv = bf2f(g[i]);
    float sg = bf2f(f2bf(1.0f / (1.0f + expf(-gv))));
    float act = bf2f(f2bf(gv * sg));
    y[i] = f2bf(act * bf2f(u[i]));
  }
}

/* residual add `&x + &attn` (qwen3.rs:521, 541) in bf16 */
void orc_add(const uint16_t *a, const uint16_t *b, uint16_t *y, int64_t n) {
  for (int64_t i = 0; i < n; i++) y[i] = f2bf(bf2f(a[i]) + bf2f(b[i]));
}

/* argmax / argmax_axis (engine.rs:198, speculative.rs:168, 289-293):
 * index of the largest value; the first such index on ties. */
void orc_argmax_rows(const uint16_t *x, int64_t rows, int64_t n, uint32_t *out) {
  for (int64_t r = 0; r < rows; r++) {
    const uint16_t *xr = x + r * n;
    int64_t best = 0;
    float bv = bf2f(xr[0]);
    for (int64_t i = 1; i < n; i++) {
      float v = bf2f(xr[i]);
      if (v > bv) {
        bv = v;
        best = i;
      }
    }
    out[r] = (uint32_t)best;
  }
}

/* ------------------------------------------------------------------ */
/* Qwen3 model (qwen3.rs:94-107, 164-295).  Weights are seeded random  */
/* init: projections quantized from approx N(0, sigma), norms 1.       */
/* ------------------------------------------------------------------ */
typedef struct {
  uint32_t *w;
  uint16_t *s, *b;
  int N, K;
} qlin;

enum { SLOT_Q, SLOT_K, SLOT_V, SLOT_O, SLOT_GATE, SLOT_UP, SLOT_DOWN, NSLOT };

typedef struct {
  qlin p[NSLOT];
  uint16_t *in_norm, *post_norm, *q_norm, *k_norm;
} layer_t;

struct orc_qwen3 {
  orc_qwen3_config cfg;
  qlin embed, lm_head;
  uint16_t *final_norm;
  layer_t *layers;
};

struct orc_kv {
  int layers, nkv, hd, cap, seq_len;
  uint16_t *data; /* [layers, 2, nkv, cap, hd] */
};

static int qlin_alloc(qlin *q, int N, int K) {
  q->N = N;
  q->K = K;
  q->w = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)N * (size_t)(K / 8));
  q->s = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)N * (size_t)(K / 64));
  q->b = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)N * (size_t)(K / 64));
  return q->w && q->s && q->b;
}
static void qlin_free(qlin *q) {
  free(q->w);
  free(q->s);
  free(q->b);
}
static uint16_t *ones_bf16(int n) {
  uint16_t *p = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)n);
  if (p)
    for (int i = 0; i < n; i++) p[i] = 0x3f80;
  return p;
}

orc_qwen3 *orc_qwen3_create_random(const orc_qwen3_config *cfg, uint64_t seed,
                                   double sigma) {
  if (cfg->bits != 4 || cfg->group_size != 64) return NULL;
  orc_qwen3 *m = (orc_qwen3 *)calloc(1, sizeof(orc_qwen3));
  if (!m) return NULL;
  m->cfg = *cfg;
  float c = orc_sigma_to_c(sigma);
  int H = cfg->hidden, I = cfg->inter, qd = cfg->n_heads * cfg->head_dim,
      kvd = cfg->n_kv_heads * cfg->head_dim;
  int ok = qlin_alloc(&m->embed, cfg->vocab, H);
  if (ok) orc_init_qlinear(orc_tensor_seed(seed, -1, 0), cfg->vocab, H, c, m->embed.w, m->embed.s, m->embed.b);
  if (ok && !cfg->tied) {
    ok = qlin_alloc(&m->lm_head, cfg->vocab, H);
    if (ok) orc_init_qlinear(orc_tensor_seed(seed, -2, 0), cfg->vocab, H, c, m->lm_head.w, m->lm_head.s, m->lm_head.b);
  }
  m->final_norm = ones_bf16(H);
  m->layers = (layer_t *)calloc((size_t)cfg->layers, sizeof(layer_t));
  ok = ok && m->final_norm && m->layers;
  for (int l = 0; ok && l < cfg->layers; l++) {
    layer_t *L = &m->layers[l];
    int dims[NSLOT][2] = {{qd, H}, {kvd, H}, {kvd, H}, {H, qd}, {I, H}, {I, H}, {H, I}};
    for (int sl = 0; sl < NSLOT && ok; sl++) {
      ok = qlin_alloc(&L->p[sl], dims[sl][0], dims[sl][1]);
      if (ok)
        orc_init_qlinear(orc_tensor_seed(seed, l, sl), dims[sl][0], dims[sl][1], c,
                         L->p[sl].w, L->p[sl].s, L->p[sl].b);
    }
    L->in_norm = ones_bf16(H);
    L->post_norm = ones_bf16(H);
    L->q_norm = ones_bf16(cfg->head_dim);
    L->k_norm = ones_bf16(cfg->head_dim);
    ok = ok && L->in_norm && L->post_norm && L->q_norm && L->k_norm;
  }
  if (!ok) {
    orc_qwen3_free(m);
    return NULL;
  }
  return m;
}

void orc_qwen3_free(orc_qwen3 *m) {
  if (!m) return;
  qlin_free(&m->embed);
  qlin_free(&m->lm_head);
  free(m->final_norm);
  if (m->layers)
    for (int l = 0; l < m->cfg.layers; l++) {
      for (int sl = 0; sl < NSLOT; sl++) qlin_free(&m->layers[l].p[sl]);
      free(m->layers[l].in_norm);
      free(m->layers[l].post_norm);
      free(m->layers[l].q_norm);
      free(m->layers[l].k_norm);
    }
  free(m->layers);
  free(m);
}

int orc_qwen3_qlinear(orc_qwen3 *m, int layer, int slot, uint32_t **w,
                      uint16_t **s, uint16_t **b, int *N, int *K) {
  qlin *q;
  if (layer == -1) q = &m->embed;
  else if (layer == -2) q = m->cfg.tied ? &m->embed : &m->lm_head;
  else if (layer >= 0 && layer < m->cfg.layers && slot >= 0 && slot < NSLOT)
    q = &m->layers[layer].p[slot];
  else return ORC_E_ARG;
  *w = q->w;
  *s = q->s;
  *b = q->b;
  *N = q->N;
  *K = q->K;
  return ORC_OK;
}

uint16_t *orc_qwen3_norm(orc_qwen3 *m, int layer, int which) {
  if (layer < 0) return m->final_norm;
  if (layer >= m->cfg.layers) return NULL;
  layer_t *L = &m->layers[layer];
  switch (which) {
    case 0: return L->in_norm;
    case 1: return L->post_norm;
    case 2: return L->q_norm;
    case 3: return L->k_norm;
  }
  return NULL;
}

/* KvCache (qwen3.rs:109-162) with a caller-chosen capacity in place of
 * KV_PREALLOC (qwen3.rs:125).  truncate() rewinds seq_len and keeps the
 * preallocated buffer -- the behaviour the reference's comment at
 * qwen3.rs:146-149 describes. */
orc_kv *orc_kv_create(const orc_qwen3 *m, int capacity) {
  orc_kv *kv = (orc_kv *)calloc(1, sizeof(orc_kv));
  if (!kv) return NULL;
  kv->layers = m->cfg.layers;
  kv->nkv = m->cfg.n_kv_heads;
  kv->hd = m->cfg.head_dim;
  kv->cap = capacity;
  size_t n = (size_t)kv->layers * 2 * kv->nkv * (size_t)capacity * kv->hd;
  kv->data = (uint16_t *)calloc(n, sizeof(uint16_t));
  if (!kv->data) {
    free(kv);
    return NULL;
  }
  return kv;
}
void orc_kv_free(orc_kv *kv) {
  if (!kv) return;
  free(kv->data);
  free(kv);
}
int orc_kv_seq_len(const orc_kv *kv) { return kv->seq_len; }
int orc_kv_capacity(const orc_kv *kv) { return kv->cap; }
void orc_kv_reset(orc_kv *kv) { kv->seq_len = 0; }
void orc_kv_truncate(orc_kv *kv, int target) {
  if (target >= kv->seq_len) return;
  kv->seq_len = target < 0 ? 0 : target;
}
uint16_t *orc_kv_data(orc_kv *kv) { return kv->data; }

/* Fill positions [0, seq_len) of every layer's K and V with approx N(0,1)
 * bf16 values and set seq_len: a stand-in for a long prefill when only the
 * cost of later decode steps is wanted. */
void orc_kv_fill_synthetic(orc_kv *kv, uint64_t seed, int seq_len) {
  int64_t rows = (int64_t)kv->layers * 2 * kv->nkv;
  float c = orc_sigma_to_c(1.0);
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; r++)
    for (int64_t t = 0; t < seq_len; t++)
      for (int64_t d = 0; d < kv->hd; d++) {
        int64_t i = (r * kv->cap + t) * kv->hd + d;
        kv->data[i] = f2bf(orc_normal_at(seed, (uint64_t)i, c));
      }
  kv->seq_len = seq_len;
}

/* Qwen3::forward / forward_multi -> forward_internal (qwen3.rs:297-563),
 * op for op (Appendix: embed, per layer qkv_block, QK-norm, transpose,
 * RoPE, slice_update, SDPA, o_proj + residual, mlp_block + residual,
 * final norm, last row or all rows, tied/untied head, seq_len += M). */
int orc_qwen3_forward(orc_qwen3 *m, orc_kv *kv, const uint32_t *tokens, int M,
                      int all_logits, uint16_t *logits) {
  const orc_qwen3_config *c = &m->cfg;
  if (M <= 0) return ORC_E_ARG;
  if (kv->layers != c->layers) return ORC_E_SHAPE; /* qwen3.rs:351-358 */
  const int H = c->hidden, I = c->inter, nq = c->n_heads, nkv = c->n_kv_heads,
            hd = c->head_dim, qd = nq * hd, kvd = nkv * hd;
  const int offset = kv->seq_len, new_end = offset + M;
  if (new_end > kv->cap) return ORC_E_KV_CAPACITY; /* qwen3.rs:423-428 */
  for (int i = 0; i < M; i++)
    if ((int)tokens[i] >= c->vocab) return ORC_E_ARG;
  const float scale = 1.0f / sqrtf((float)hd); /* qwen3.rs:324 */
  size_t MH = (size_t)M * H;
  uint16_t *x = malloc(2 * MH), *h = malloc(2 * MH), *q = malloc(2 * (size_t)M * qd),
           *k = malloc(2 * (size_t)M * kvd), *v = malloc(2 * (size_t)M * kvd),
           *qt = malloc(2 * (size_t)M * qd), *kt = malloc(2 * (size_t)M * kvd),
           *vt = malloc(2 * (size_t)M * kvd), *att = malloc(2 * (size_t)M * qd),
           *o = malloc(2 * MH), *g = malloc(2 * (size_t)M * I),
           *u = malloc(2 * (size_t)M * I), *a = malloc(2 * (size_t)M * I);
  int rc = ORC_OK;
  if (!x || !h || !q || !k || !v || !qt || !kt || !vt || !att || !o || !g || !u || !a) {
    rc = ORC_E_ALLOC;
    goto done;
  }
  /* x = embed.lookup(tokens)  (qwen3.rs:328-333) */
  rc = orc_dequant_gather(tokens, M, c->vocab, m->embed.w, m->embed.s, m->embed.b, H, 64, 4, x);
  if (rc) goto done;
  for (int l = 0; l < c->layers; l++) {
    layer_t *L = &m->layers[l];
    /* qkv_block: rms_norm + q/k/v projections (kernels.rs:28-46) */
    orc_rms_norm(x, L->in_norm, h, M, H, c->eps);
    orc_qlinear(h, L->p[SLOT_Q].w, L->p[SLOT_Q].s, L->p[SLOT_Q].b, q, M, qd, H, 64, 4);
    orc_qlinear(h, L->p[SLOT_K].w, L->p[SLOT_K].s, L->p[SLOT_K].b, k, M, kvd, H, 64, 4);
    orc_qlinear(h, L->p[SLOT_V].w, L->p[SLOT_V].s, L->p[SLOT_V].b, v, M, kvd, H, 64, 4);
    /* per-head QK-norm before RoPE (qwen3.rs:392-399) */
    orc_rms_norm(q, L->q_norm, q, (int64_t)M * nq, hd, c->eps);
    orc_rms_norm(k, L->k_norm, k, (int64_t)M * nkv, hd, c->eps);
    /* [seq, heads, hd] -> [heads, seq, hd]  (qwen3.rs:401-405) */
    for (int t = 0; t < M; t++) {
      for (int hh = 0; hh < nq; hh++)
        memcpy(qt + ((size_t)hh * M + t) * hd, q + ((size_t)t * nq + hh) * hd, 2 * (size_t)hd);
      for (int hh = 0; hh < nkv; hh++) {
        memcpy(kt + ((size_t)hh * M + t) * hd, k + ((size_t)t * nkv + hh) * hd, 2 * (size_t)hd);
        memcpy(vt + ((size_t)hh * M + t) * hd, v + ((size_t)t * nkv + hh) * hd, 2 * (size_t)hd);
      }
    }
    /* RoPE at offset = cache.seq_len (qwen3.rs:407-413) */
    orc_rope(qt, qt, nq, M, hd, c->rope_theta, offset);
    orc_rope(kt, kt, nkv, M, hd, c->rope_theta, offset);
    /* slice_update of K and V at [0:nkv, offset:new_end, 0:hd]
     * (qwen3.rs:431-489) */
    uint16_t *kl = kv->data + (size_t)l * 2 * nkv * kv->cap * hd;
    uint16_t *vl = kl + (size_t)nkv * kv->cap * hd;
    int64_t shape[3] = {nkv, kv->cap, hd}, st[3] = {0, offset, 0},
            sp[3] = {nkv, new_end, hd}, sd[3] = {1, 1, 1};
    orc_slice_update(kl, 3, shape, kt, st, sp, sd);
    orc_slice_update(vl, 3, shape, vt, st, sp, sd);
    /* SDPA over the valid view [.., 0:new_end, ..]; mask only for M > 1
     * (qwen3.rs:345-349, 491-518) */
    orc_sdpa(qt, kl, vl, att, nq, nkv, M, new_end, hd, kv->cap, offset, M > 1, scale);
    /* o_proj + residual (qwen3.rs:520-521) */
    orc_qlinear(att, L->p[SLOT_O].w, L->p[SLOT_O].s, L->p[SLOT_O].b, o, M, H, qd, 64, 4);
    orc_add(x, o, x, (int64_t)MH);
    /* mlp_block + residual (kernels.rs:55-78; qwen3.rs:523-541) */
    orc_rms_norm(x, L->post_norm, h, M, H, c->eps);
    orc_qlinear(h, L->p[SLOT_GATE].w, L->p[SLOT_GATE].s, L->p[SLOT_GATE].b, g, M, I, H, 64, 4);
    orc_qlinear(h, L->p[SLOT_UP].w, L->p[SLOT_UP].s, L->p[SLOT_UP].b, u, M, I, H, 64, 4);
    orc_silu_mul(g, u, a, (int64_t)M * I);
    orc_qlinear(a, L->p[SLOT_DOWN].w, L->p[SLOT_DOWN].s, L->p[SLOT_DOWN].b, o, M, H, I, 64, 4);
    orc_add(x, o, x, (int64_t)MH);
  }
  /* final norm, last row unless all logits, tied head (qwen3.rs:545-555) */
  orc_rms_norm(x, m->final_norm, h, M, H, c->eps);
  {
    const qlin *head = c->tied ? &m->embed : &m->lm_head;
    if (all_logits)
      orc_qlinear(h, head->w, head->s, head->b, logits, M, c->vocab, H, 64, 4);
    else
      orc_qlinear(h + (size_t)(M - 1) * H, head->w, head->s, head->b, logits, 1, c->vocab, H, 64, 4);
  }
  kv->seq_len += M; /* qwen3.rs:557 */
done:
  free(x); free(h); free(q); free(k); free(v); free(qt); free(kt); free(vt);
  free(att); free(o); free(g); free(u); free(a);
  return rc;
}

static int is_eos(uint32_t t, const uint32_t *eos, int n_eos) {
  for (int i = 0; i < n_eos; i++)
    if (eos[i] == t) return 1;
  return 0;
}

/* LoadedModel::generate_text with greedy pick_next (engine.rs:100-144,
 * 146-153): prefill the whole prompt, then one token per step until EOS or
 * max_new tokens have been produced; EOS is not emitted. */
int orc_generate_greedy(orc_qwen3 *m, orc_kv *kv, const uint32_t *prompt,
                        int P, int max_new, const uint32_t *eos, int n_eos,
                        uint32_t *out, int *n_out) {
  uint16_t *logits = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)m->cfg.vocab);
  if (!logits) return ORC_E_ALLOC;
  int rc = orc_qwen3_forward(m, kv, prompt, P, 0, logits);
  int produced = 0, n = 0;
  while (rc == ORC_OK) {
    uint32_t next;
    orc_argmax_rows(logits, 1, m->cfg.vocab, &next);
    produced++;
    if (is_eos(next, eos, n_eos)) break;
    out[n++] = next;
    if (produced >= max_new) break;
    rc = orc_qwen3_forward(m, kv, &next, 1, 0, logits);
  }
  *n_out = n;
  free(logits);
  return rc;
}

/* speculative::generate, greedy (speculative.rs:57-286) with a verify width
 * of spec_k tokens (leader + spec_k-1 drafts; the reference fixes
 * SPEC_K = 4 at speculative.rs:36).  stats (optional, 3 entries):
 * iterations, proposed, accepted. */
int orc_speculative_generate(orc_qwen3 *target, orc_kv *tkv, orc_qwen3 *draft,
                             orc_kv *dkv, const uint32_t *prompt, int P,
                             int max_new, int spec_k, const uint32_t *eos,
                             int n_eos, uint32_t *out, int *n_out,
                             int64_t *stats) {
  const int V = target->cfg.vocab;
  *n_out = 0;
  if (draft->cfg.vocab != V) return ORC_E_ARG; /* check_compatible, speculative.rs:40-54 */
  if (spec_k < 2 || spec_k > 16 || P <= 0 || max_new <= 0) return ORC_E_ARG;
  /* the reference starts from fresh caches (speculative.rs:71-72); caches
   * that already hold context are rewound relative to where they start */
  const int t0 = orc_kv_seq_len(tkv), d0 = orc_kv_seq_len(dkv);
  uint16_t *tl = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)V * (size_t)spec_k);
  uint16_t *dl = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)V);
  int64_t iters = 0, proposed = 0, accepted = 0;
  int rc = ORC_OK, n = 0;
  if (!tl || !dl) {
    rc = ORC_E_ALLOC;
    goto done;
  }
  /* prefill both (speculative.rs:75-79).  Only the target's last-row
   * logits are read (:82) and the draft's are discarded, so only those
   * rows are produced; the caches end up identical. */
  rc = orc_qwen3_forward(target, tkv, prompt, P, 0, tl);
  if (rc) goto done;
  rc = orc_qwen3_forward(draft, dkv, prompt, P, 0, dl);
  if (rc) goto done;
  uint32_t leader;
  orc_argmax_rows(tl, 1, V, &leader);
  if (is_eos(leader, eos, n_eos)) goto done;
  out[n++] = leader;
  rc = orc_qwen3_forward(draft, dkv, &leader, 1, 0, dl); /* :104 */
  if (rc) goto done;
  while (n < max_new) {
    uint32_t drafts[16], vin[16], preds[16];
    int nd = 0;
    for (int i = 0; i < spec_k - 1; i++) { /* :124-137 */
      uint32_t d;
      orc_argmax_rows(dl, 1, V, &d);
      drafts[nd++] = d;
      rc = orc_qwen3_forward(draft, dkv, &d, 1, 0, dl);
      if (rc) goto done;
      if (is_eos(d, eos, n_eos)) break;
    }
    vin[0] = leader;
    for (int i = 0; i < nd; i++) vin[i + 1] = drafts[i];
    rc = orc_qwen3_forward(target, tkv, vin, nd + 1, 1, tl); /* :146-148 */
    if (rc) goto done;
    orc_argmax_rows(tl, nd + 1, V, preds); /* :168-173 */
    proposed += nd;
    iters++;
    int na = 0;
    uint32_t bonus = preds[nd];
    for (int i = 0; i < nd; i++) { /* :175-192 */
      if (preds[i] == drafts[i]) na++;
      else {
        bonus = preds[i];
        break;
      }
    }
    accepted += na;
    int stop = 0;
    for (int i = 0; i < na; i++) { /* :201-211 */
      if (n >= max_new || is_eos(drafts[i], eos, n_eos)) {
        stop = 1;
        break;
      }
      out[n++] = drafts[i];
    }
    if (stop || n >= max_new || is_eos(bonus, eos, n_eos)) break;
    out[n++] = bonus;
    /* rewind both caches to prompt + emitted - 1 (:227, :234) */
    orc_kv_truncate(tkv, t0 + P + n - 1);
    orc_kv_truncate(dkv, d0 + P + n - 1);
    leader = bonus;
    rc = orc_qwen3_forward(draft, dkv, &leader, 1, 0, dl); /* :238-239 */
    if (rc) goto done;
  }
done:
  *n_out = n;
  if (stats) {
    stats[0] = iters;
    stats[1] = proposed;
    stats[2] = accepted;
  }
  free(tl);
  free(dl);
  return rc;
}

/* ------------------------------------------------------------------ */
/* Host measurement helpers for the CPU baseline (not part of the path): */
/* the OpenMP thread count the oracle runs with, and a STREAM-style      */
/* triad a[i] = b[i] + s * c[i] over n doubles (24 n bytes moved per     */
/* pass), best of `reps` passes, in GB/s.                                */
/* ------------------------------------------------------------------ */
int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

double orc_stream_triad_gbs(int64_t n, int reps) {
  double *a = (double *)malloc(sizeof(double) * (size_t)n);
  double *b = (double *)malloc(sizeof(double) * (size_t)n);
  double *c = (double *)malloc(sizeof(double) * (size_t)n);
  if (!a || !b || !c) {
    free(a);
    free(b);
    free(c);
    return 0.0;
  }
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; i++) {
    a[i] = 0.0;
    b[i] = 1.0;
    c[i] = 2.0;
  }
  double best = 0.0;
  for (int r = 0; r < reps; r++) {
#ifdef _OPENMP
    const double t0 = omp_get_wtime();
#endif
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) a[i] = b[i] + 3.0 * c[i];
#ifdef _OPENMP
    const double dt = omp_get_wtime() - t0;
#else
    const double dt = 1.0;
#endif
    const double gbs = 24.0 * (double)n / dt / 1e9;
    if (gbs > best) best = gbs;
  }
  volatile double sink = a[n / 2];
  (void)sink;
  free(a);
  free(b);
  free(c);
  return best;
}
