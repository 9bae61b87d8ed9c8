// qmm: MLX-format 4-bit affine quantized GEMM for M > 8 rows of x (prefill,
// long verify), gfx950 bf16 MFMA.
//
// Semantics restated: mlx_rs::ops::quantized_matmul(x, W, s, b,
// transpose=true, 64, 4) (crates/base-mlx-core/src/model/qwen3.rs:30-41):
//   y[m,n] = sum_g s[n,g] * D_g[m,n] + sum_g b[n,g] * Sx_g[m],
//   D_g = sum_{k in g} q[n,k] x[m,k],  Sx_g = sum_{k in g} x[m,k],
// with fp32 accumulation and a bf16 result -- the group decomposition of
// the GEMV, so prefill and decode round alike.
//
// Workgroup tile: 128 rows of x by 128 rows of W, 4 waves (2 x 2), each
// 64 x 64 = 4 x 4 tiles of v_mfma_f32_16x16x32_bf16; three workgroups share
// a CU.  Per K step (one 64-wide group) the workgroup stages in LDS:
//   * x (128 x 64 bf16) and its row sums Sx_g, the latter as bf16 hi + lo
//     (hi + lo = Sx to about 2^-17) in a window of 32 groups;
//   * W as exact bf16 integers q = 0..15 (bytes of the packed word through
//     v_cvt_f32_ubyte; a small integer's bf16 is the top half of its float);
//   * s of the 128 W rows (fp32).
// Each wave runs D = x W^T over the group's two K halves and folds
// acc += s[n] * D: one fp32 FMA per output and group.  The b * Sx term runs
// on the matrix cores once per 32-group window: acc += Sx_hi b + Sx_lo b
// with A = Sx from LDS and B = 8 consecutive biases of a W row (exact bf16)
// read straight from global.  The next group's global loads are issued
// before this group's products and land in LDS after them.  When the tile
// grid is small, K is split over workgroups: fp32 partial tiles go to a
// workspace and a reduction kernel writes y.
#include <stdlib.h>

#include <algorithm>
#include <mutex>

#include "bmx_device.h"

namespace bmx {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

constexpr int QBM = 128, QBN = 128, QT = 256;  // tile rows of x, of W; threads
constexpr int XP = 72, WP = 72;                // LDS row strides (elements)
constexpr int SXW = 32;                        // groups per b * Sx window
constexpr size_t kXsElems = 1ull * QBM * XP, kWsElems = 1ull * QBN * WP, kSxElems = 2ull * QBM * SXW;
constexpr size_t kQmmLds = (kXsElems + kWsElems + kSxElems) * 2 + 1ull * QBN * 4;

struct QmmParams {
  const uint16_t* x;  // [M, K]
  const uint32_t* w;  // [N, K/8]
  const uint16_t* s;  // [N, K/64]
  const uint16_t* b;  // [N, K/64]
  uint16_t* y;        // [M, N] bf16 (one split)
  float* part;        // [splits, M, N] fp32 partials (several splits)
  int M, N, K;
  int gps;  // groups per split
};

// bf16 bits of the small integer in byte `i` of v (exact)
__device__ __forceinline__ uint32_t byte_bf16(uint32_t v, int i) {
  return __float_as_uint(static_cast<float>((v >> (8 * i)) & 0xffu)) >> 16;
}

__global__ void __launch_bounds__(QT, 2) qmm_kernel(const QmmParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);      // [QBM][XP]
  uint16_t* ws = xs + kXsElems;                          // [QBN][WP]
  uint16_t* sxs = ws + kWsElems;                         // [hi, lo][QBM][SXW]
  float* ss = reinterpret_cast<float*>(sxs + kSxElems);  // [QBN]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;  // wave sub-tile: x rows 64 wm, W rows 64 wn
  const int li = lane & 15, q = lane >> 4;
  const int M = p.M, N = p.N, K = p.K, G = K / 64;
  const int m0 = blockIdx.y * QBM, n0 = blockIdx.x * QBN;
  const int gb = blockIdx.z * p.gps, ge = min(G, gb + p.gps);

  // ---- global -> registers for one group (rows clamped: their results are
  // never stored) ----
  const int xe0 = tid, xe1 = tid + QT, xe2 = tid + 2 * QT, xe3 = tid + 3 * QT;
  auto xrow = [&](int e) { return p.x + static_cast<int64_t>(min(m0 + (e >> 3), M - 1)) * K + (e & 7) * 8; };
  const uint16_t* xp0 = xrow(xe0);
  const uint16_t* xp1 = xrow(xe1);
  const uint16_t* xp2 = xrow(xe2);
  const uint16_t* xp3 = xrow(xe3);
  auto wrow = [&](int e) { return p.w + static_cast<int64_t>(min(n0 + (e >> 1), N - 1)) * (K / 8) + (e & 1) * 4; };
  const uint32_t* wp0 = wrow(tid);
  const uint16_t* sp = p.s + static_cast<int64_t>(min(n0 + (tid & (QBN - 1)), N - 1)) * G;
  uint4 xr0, xr1, xr2, xr3, wr0;
  uint16_t sr;
  auto load = [&](int g) {
    xr0 = *reinterpret_cast<const uint4*>(xp0 + g * 64);
    xr1 = *reinterpret_cast<const uint4*>(xp1 + g * 64);
    xr2 = *reinterpret_cast<const uint4*>(xp2 + g * 64);
    xr3 = *reinterpret_cast<const uint4*>(xp3 + g * 64);
    wr0 = *reinterpret_cast<const uint4*>(wp0 + g * 8);
    sr = sp[g];
  };
  // ---- registers -> LDS: x, Sx (window slot), W as exact q, s ----
  auto store = [&](int g) {
    uint16_t* xb = xs;
    const int slot = (g - gb) % SXW;
    auto put_x = [&](int e, const uint4& v) {
      const int r = e >> 3, u = e & 7;
      *reinterpret_cast<uint4*>(xb + r * XP + u * 8) = v;
      float t = bf2f(v.x & 0xffffu) + bf2f(v.x >> 16) + bf2f(v.y & 0xffffu) + bf2f(v.y >> 16) +
                bf2f(v.z & 0xffffu) + bf2f(v.z >> 16) + bf2f(v.w & 0xffffu) + bf2f(v.w >> 16);
      t = lanes_sum(t, 8);  // the 8 units of a row are 8 consecutive lanes
      if (u == 0) {
        const uint16_t hi = f2bf(t);
        const uint16_t lo = f2bf(t - bf2f(hi));
        sxs[r * SXW + slot] = hi;
        sxs[QBM * SXW + r * SXW + slot] = lo;
        if (g == ge - 1)  // last group: the rest of the window holds zeros
          for (int z = slot + 1; z < SXW; z++) sxs[r * SXW + z] = sxs[QBM * SXW + r * SXW + z] = 0;
      }
    };
    put_x(xe0, xr0);
    put_x(xe1, xr1);
    put_x(xe2, xr2);
    put_x(xe3, xr3);
    uint16_t* wb = ws;
    auto put_word = [&](uint16_t* dst, uint32_t word) {
      // nibble k of the word is value k: even k in the low nibble of byte
      // k/2, odd k in the high nibble
      const uint32_t lo = word & 0x0f0f0f0fu, hi = (word >> 4) & 0x0f0f0f0fu;
      uint4 o;
      o.x = byte_bf16(lo, 0) | (byte_bf16(hi, 0) << 16);
      o.y = byte_bf16(lo, 1) | (byte_bf16(hi, 1) << 16);
      o.z = byte_bf16(lo, 2) | (byte_bf16(hi, 2) << 16);
      o.w = byte_bf16(lo, 3) | (byte_bf16(hi, 3) << 16);
      *reinterpret_cast<uint4*>(dst) = o;
    };
    auto put_w = [&](int e, const uint4& v) {
      uint16_t* dst = wb + (e >> 1) * WP + (e & 1) * 32;
      put_word(dst, v.x);
      put_word(dst + 8, v.y);
      put_word(dst + 16, v.z);
      put_word(dst + 24, v.w);
    };
    put_w(tid, wr0);
    if (tid < QBN) ss[tid] = bf2f(sr);
  };

  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // b * Sx over the window of groups [w0, w0 + SXW): acc += (Sx_hi + Sx_lo) b.
  // Window slots past the split's last group hold zero Sx; their biases are
  // read clamped to the row.
  const bool b_vec = (G % 8) == 0 && (gb % 8) == 0;  // 16-byte bias reads
  auto window = [&](int w0) {
    bf16x8_t sh[4], sl[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int r = wm * 64 + i * 16 + li;
      sh[i] = *reinterpret_cast<const bf16x8_t*>(sxs + r * SXW + 8 * q);
      sl[i] = *reinterpret_cast<const bf16x8_t*>(sxs + QBM * SXW + r * SXW + 8 * q);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int n = min(n0 + wn * 64 + j * 16 + li, N - 1);
      const uint16_t* brow = p.b + static_cast<int64_t>(n) * G;
      uint4 bw;
      if (b_vec) {
        bw = *reinterpret_cast<const uint4*>(brow + min(w0 + 8 * q, G - 8));
      } else {
        uint32_t h[8];
#pragma unroll
        for (int k = 0; k < 8; k++) h[k] = brow[min(w0 + 8 * q + k, G - 1)];
        bw = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
      }
      const bf16x8_t bv = __builtin_bit_cast(bf16x8_t, bw);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sh[i], bv, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sl[i], bv, acc[i][j], 0, 0, 0);
      }
    }
  };

  load(gb);
  store(gb);
  __syncthreads();
  for (int g = gb; g < ge; g++) {
    const bool more = g + 1 < ge;
    if (more) load(g + 1);
    const uint16_t* xb = xs;
    const uint16_t* wb = ws;
    bf16x8_t af[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int t = 0; t < 2; t++)
        af[i][t] = *reinterpret_cast<const bf16x8_t*>(xb + (wm * 64 + i * 16 + li) * XP + t * 32 + q * 8);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int c = wn * 64 + j * 16 + li;
      const bf16x8_t b0 = *reinterpret_cast<const bf16x8_t*>(wb + c * WP + q * 8);
      const bf16x8_t b1 = *reinterpret_cast<const bf16x8_t*>(wb + c * WP + 32 + q * 8);
      const float sv = ss[c];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        f32x4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i][0], b0, d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i][1], b1, d, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; r++) acc[i][j][r] += sv * d[r];
      }
    }
    if (((g - gb) % SXW) == SXW - 1 || !more) window(g - (g - gb) % SXW);
    if (!more) break;
    __syncthreads();  // every read of this group's tiles (and window) is done
    store(g + 1);
    __syncthreads();
  }

  // ---- epilogue: lane holds W row 16 j + li, x rows 4 q + r of each tile ----
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int n = n0 + wn * 64 + j * 16 + li;
      if (n >= N) continue;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = m0 + wm * 64 + i * 16 + 4 * q + r;
        if (m >= M) continue;
        if (p.part)
          p.part[(static_cast<int64_t>(blockIdx.z) * M + m) * N + n] = acc[i][j][r];
        else
          p.y[static_cast<int64_t>(m) * N + n] = f2bf(acc[i][j][r]);
      }
    }
}

// y = bf16(sum over splits of the fp32 partials), 4 outputs per thread
__global__ void __launch_bounds__(256) qmm_reduce_kernel(const float* part, uint16_t* y, int64_t mn, int splits) {
  const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i0 >= mn) return;
  for (int64_t i = i0; i < min(i0 + 4, mn); i++) {
    float t = 0.0f;
    for (int s = 0; s < splits; s++) t += part[s * mn + i];
    y[i] = f2bf(t);
  }
}

// Split-K partials: one device buffer per process, grown on demand (the
// GEMM path is never inside a captured graph).
std::mutex g_part_mu;
float* g_part = nullptr;
size_t g_part_floats = 0;

int part_buffer(size_t floats, float** out) {
  std::lock_guard<std::mutex> lock(g_part_mu);
  if (floats > g_part_floats) {
    if (g_part) {
      // earlier launches may still read the old buffer
      if (hipDeviceSynchronize() != hipSuccess) return set_error(BMX_E_ALLOC, "qmm: device sync failed");
      (void)hipFree(g_part);
    }
    g_part = nullptr;
    g_part_floats = 0;
    if (hipMalloc(&g_part, floats * sizeof(float)) != hipSuccess)
      return set_error(BMX_E_ALLOC, "qmm: no memory for %zu split-K partials", floats);
    g_part_floats = floats;
  }
  *out = g_part;
  return BMX_OK;
}

}  // namespace

int launch_qmm(const uint16_t* x, const uint32_t* w, const uint16_t* s, const uint16_t* b, uint16_t* y, int M, int N,
               int K, hipStream_t stream) {
  if (M <= 0) return BMX_OK;
  if (K % 64 || N <= 0) return set_error(BMX_E_SHAPE, "qmm: N=%d K=%d", N, K);
  if (!aligned(x, 16) || !aligned(w, 16)) return set_error(BMX_E_ALIGN, "qmm: x and W must be 16-byte aligned");
  if ((M + QBM - 1) / QBM > 65535) return set_error(BMX_E_SHAPE, "qmm: M=%d too large", M);
  const int G = K / 64;
  const int tiles = ((N + QBN - 1) / QBN) * ((M + QBM - 1) / QBM);
  // split K while the tiles leave most of the device idle (splits of at
  // least 8 groups, a multiple of 8 groups each)
  int splits = 1;
  while (tiles * splits * 2 <= 512 && G / (splits * 2) >= 8) splits *= 2;
  int gps = (G + splits - 1) / splits;
  if (splits > 1) gps = (gps + 7) / 8 * 8;
  splits = (G + gps - 1) / gps;
  QmmParams p{x, w, s, b, y, nullptr, M, N, K, gps};
  if (splits > 1)
    if (int rc = part_buffer(static_cast<size_t>(splits) * M * N, &p.part)) return rc;
  if (int rc = allow_lds_ptr(reinterpret_cast<const void*>(qmm_kernel), kQmmLds)) return rc;
  const dim3 grid((N + QBN - 1) / QBN, (M + QBM - 1) / QBM, splits);
  hipLaunchKernelGGL(qmm_kernel, grid, dim3(QT), kQmmLds, stream, p);
  if (int rc = check_launch("qmm")) return rc;
  if (splits > 1) {
    const int64_t mn = static_cast<int64_t>(M) * N;
    hipLaunchKernelGGL(qmm_reduce_kernel, dim3(static_cast<unsigned>((mn + 1023) / 1024)), dim3(256), 0, stream,
                       p.part, y, mn, splits);
    return check_launch("qmm_reduce");
  }
  return BMX_OK;
}

}  // namespace bmx
