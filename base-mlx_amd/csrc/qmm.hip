// qmm: MLX-format 4-bit affine quantized GEMM for M > 8 rows of x (prefill,
// long verify), gfx950 bf16 MFMA.
//
// Semantics restated: mlx_rs::ops::quantized_matmul(x, W, s, b,
// transpose=true, 64, 4) (crates/base-mlx-core/src/model/qwen3.rs:30-41):
//   y[m,n] = sum_g s[n,g] * sum_{k in g} q[n,k] x[m,k] + b[n,g] * sum_{k in g} x[m,k]
// with fp32 accumulation and a bf16 result -- the same group decomposition
// as the GEMV, so prefill and decode round alike.
//
// Tile 64 (rows of x) x 128 (rows of W) x 64 (one quantization group per
// K step).  Per step the workgroup stages in LDS (rows padded to 72
// elements so 16-byte fragment reads of 16 consecutive rows hit distinct
// banks):
//   * x (64 x 64 bf16) with each 8-value unit pair-permuted to
//     (x0,x4,x1,x5,x2,x6,x3,x7), plus the group sum Sx of every row;
//   * W as bf16 (128 + q) in the same order, made with one mask and one or
//     per pair: (w >> 4j & 0x000F000F) | 0x43004300 = (128+q_j, 128+q_{j+4}),
//     plus s and b - 128 s of every row.
// Each of the 4 waves computes a 32 x 64 sub-tile as 2 x 4
// v_mfma_f32_16x16x32_bf16 over the group's two K halves (products of bf16
// integers and bf16 x are exact in fp32), then folds the group into its
// accumulators: acc += s[n] * D + (b[n] - 128 s[n]) * Sx[m].
#include "bmx_device.h"

namespace bmx {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

constexpr int BM = 64, BN = 128, PAD = 72;  // K step = one 64-wide group

__device__ __forceinline__ uint4 nibbles_bf16(uint32_t w) {
  const uint32_t magic = 0x43004300u;
  return make_uint4((w & 0x000f000fu) | magic, ((w >> 4) & 0x000f000fu) | magic, ((w >> 8) & 0x000f000fu) | magic,
                    ((w >> 12) & 0x000f000fu) | magic);
}

__global__ void __launch_bounds__(256)
    qmm_kernel(const uint16_t* __restrict__ x, const uint32_t* __restrict__ w, const uint16_t* __restrict__ s,
               const uint16_t* __restrict__ b, uint16_t* __restrict__ y, int M, int N, int K) {
  __shared__ __align__(16) uint16_t xs[BM * PAD];
  __shared__ __align__(16) uint16_t ws[BN * PAD];
  __shared__ float sxs[BM];
  __shared__ float svs[BN], bbs[BN];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;  // wave sub-tile: rows wm*32, cols wn*64
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int G = K / 64;
  const int li = lane & 15, q = lane >> 4;

  f32x4_t acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  for (int g = 0; g < G; g++) {
    // ---- load: x (2 units of 8 bf16 per thread), W (4 words per thread) ----
    uint4 xr[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int e = tid + 256 * i;  // 512 units: row e/8, unit e%8
      const int r = e >> 3, c = (e & 7) * 8;
      xr[i] = (m0 + r < M) ? *reinterpret_cast<const uint4*>(x + static_cast<int64_t>(m0 + r) * K + g * 64 + c)
                           : make_uint4(0, 0, 0, 0);
    }
    uint32_t wr[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int e = tid + 256 * i;  // 1024 words: row e/8, word e%8
      const int r = min(n0 + (e >> 3), N - 1);
      wr[i] = w[static_cast<int64_t>(r) * (K / 8) + g * 8 + (e & 7)];
    }
    float sv = 0.0f, bv = 0.0f;
    if (tid < BN) {
      const int r = min(n0 + tid, N - 1);
      sv = bf2f(s[static_cast<int64_t>(r) * G + g]);
      bv = bf2f(b[static_cast<int64_t>(r) * G + g]);
    }
    // row sums of x: the 8 units of a row are 8 consecutive threads
    float part[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const uint32_t d[4] = {xr[i].x, xr[i].y, xr[i].z, xr[i].w};
      float p = 0.0f;
#pragma unroll
      for (int e = 0; e < 4; e++) p += bf2f(d[e] & 0xffffu) + bf2f(d[e] >> 16);
      p += __shfl_xor(p, 1, 64);
      p += __shfl_xor(p, 2, 64);
      p += __shfl_xor(p, 4, 64);
      part[i] = p;
    }
    __syncthreads();  // previous step finished reading LDS
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int e = tid + 256 * i;
      *reinterpret_cast<uint4*>(xs + (e >> 3) * PAD + (e & 7) * 8) = permute_pairs(xr[i]);
      if ((e & 7) == 0) sxs[e >> 3] = part[i];
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int e = tid + 256 * i;
      *reinterpret_cast<uint4*>(ws + (e >> 3) * PAD + (e & 7) * 8) = nibbles_bf16(wr[i]);
    }
    if (tid < BN) {
      svs[tid] = sv;
      bbs[tid] = bv - 128.0f * sv;
    }
    __syncthreads();
    // ---- MFMA over the group's two K halves, then fold with s, b, Sx ----
    f32x4_t d[2][4];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) d[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < 2; t++) {
      bf16x8_t af[2], bf[4];
#pragma unroll
      for (int i = 0; i < 2; i++)
        af[i] = *reinterpret_cast<const bf16x8_t*>(xs + (wm * 32 + i * 16 + li) * PAD + t * 32 + q * 8);
#pragma unroll
      for (int j = 0; j < 4; j++)
        bf[j] = *reinterpret_cast<const bf16x8_t*>(ws + (wn * 64 + j * 16 + li) * PAD + t * 32 + q * 8);
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) d[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bf[j], d[i][j], 0, 0, 0);
    }
    float sc[4], bb[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      sc[j] = svs[wn * 64 + j * 16 + li];
      bb[j] = bbs[wn * 64 + j * 16 + li];
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const f32x4_t sx = *reinterpret_cast<const f32x4_t*>(sxs + wm * 32 + i * 16 + 4 * q);
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          acc[i][j][r] += sc[j] * d[i][j][r];
          acc[i][j][r] += bb[j] * sx[r];
        }
    }
  }
  // ---- epilogue: lane holds column li, rows 4q + r of each 16x16 tile ----
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int n = n0 + wn * 64 + j * 16 + li;
      if (n >= N) continue;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = m0 + wm * 32 + i * 16 + 4 * q + r;
        if (m < M) y[static_cast<int64_t>(m) * N + n] = f2bf(acc[i][j][r]);
      }
    }
}

}  // namespace

int launch_qmm(const uint16_t* x, const uint32_t* w, const uint16_t* s, const uint16_t* b, uint16_t* y, int M, int N,
               int K, hipStream_t stream) {
  if (M <= 0) return BMX_OK;
  if (K % 64 || N <= 0) return set_error(BMX_E_SHAPE, "qmm: N=%d K=%d", N, K);
  if (!aligned(x, 16)) return set_error(BMX_E_ALIGN, "qmm: x not 16-byte aligned");
  const dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
  if (grid.y > 65535) return set_error(BMX_E_SHAPE, "qmm: M=%d too large", M);
  hipLaunchKernelGGL(qmm_kernel, grid, dim3(256), 0, stream, x, w, s, b, y, M, N, K);
  return check_launch("qmm");
}

}  // namespace bmx
