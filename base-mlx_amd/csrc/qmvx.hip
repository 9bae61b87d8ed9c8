// qmvx: MLX-format 4-bit affine quantized matmul for 2..8 rows of x on the
// matrix cores (speculative verify M = 5, small batches), gfx950.
//
// Semantics restated: mlx_rs::ops::quantized_matmul(x, W, s, b,
// transpose=true, group_size=64, bits=4) (crates/base-mlx-core/src/model/
// qwen3.rs:30-41, model/kernels.rs:42-44, 69-75):
//   y[m,n] = sum_g s[n,g] * sum_{k in g} q[n,k] x[m,k] + b[n,g] * sum_{k in g} x[m,k]
// fp32 accumulation, bf16 result -- the group decomposition of the GEMV and
// of qmm, so all paths round alike.
//
// With several rows of x the dot2 GEMV runs out of VALU: every nibble pair
// is multiplied M times.  Here the nibbles are unpacked once and the
// products run on v_mfma_f32_16x16x32_bf16:
//   A = x (16 rows, rows >= M read as zeros): lane l holds x row l%16 and k
//       slice l/16 of the 32-wide step, from LDS;
//   B = W^T: lane l holds W row n = l%16 of a 16-row tile; in step t of a
//       64-wide group the lane's k slice is packed word 2(l/16) + t of the
//       group, unpacked with one mask and one or per bf16 pair
//         (w >> 4j & 0x000F000F) | 0x43004300 == (128 + q_j, 128 + q_{j+4})
//       so x sits in LDS pair-permuted (x_j, x_{j+4});
//   D (per group) -> acc += s * D + (b - 128 s) * Sx, Sx the group sum of x.
// The output tile puts W row l%16 and x rows 4(l/16) + r in lane l.
//
// A workgroup of 8 waves owns TB tiles of 16 rows and splits the K groups
// SK ways (TB * SK = 8), so small projections still put thousands of waves
// on the chip.  x (all rows, all K) and the workgroup's s|b are staged in
// LDS once; each wave issues all of its W loads (8 bytes per lane per group)
// up front and unconditionally, so every wait is for one specific group.
// The SK partial tiles are added in LDS; store / residual / SwiGLU epilogue.
#include <stdlib.h>

#include <algorithm>

#include "bmx_device.h"

namespace bmx {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kXU = 8;  // x staging units (8 values) per thread per batch

__device__ __forceinline__ uint4 permute_pairs(uint4 d) {
  uint4 r;
  r.x = (d.x & 0xffffu) | (d.z << 16);
  r.y = (d.x >> 16) | (d.z & 0xffff0000u);
  r.z = (d.y & 0xffffu) | (d.w << 16);
  r.w = (d.y >> 16) | (d.w & 0xffff0000u);
  return r;
}

// 8 nibbles of a packed word -> bf16 (128 + q), pair-permuted order
__device__ __forceinline__ bf16x8_t nibbles_bf16(uint32_t w) {
  const uint32_t magic = 0x43004300u;
  uint4 p;
  p.x = (w & 0x000f000fu) | magic;
  p.y = ((w >> 4) & 0x000f000fu) | magic;
  p.z = ((w >> 8) & 0x000f000fu) | magic;
  p.w = ((w >> 12) & 0x000f000fu) | magic;
  return __builtin_bit_cast(bf16x8_t, p);
}

template <int MT, int NI, int EPI>
__global__ void __launch_bounds__(kThreads) qmvx_kernel(const QmvParams p, const int TB) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int NH = (EPI == QMV_SWIGLU) ? 2 : 1;
  const int SK = kWaves / TB;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tile = wave % TB, slice = wave / TB;
  const int n_l = lane & 15, q = lane >> 4;
  const int M = p.m, K = p.K, G = K / 64, U = G * 8;  // U: 16-byte x units per row
  const int RW = 16 * TB;                              // W rows per workgroup
  const int XS = U + 1;                                // LDS row stride in units (bank skew)
  uint4* xs = reinterpret_cast<uint4*>(smem);                             // [MT][XS]
  float* sxs = reinterpret_cast<float*>(xs + MT * XS);                    // [G][16]
  uint32_t* sbs = reinterpret_cast<uint32_t*>(sxs + G * 16);              // [NH][RW][G]
  float* red = reinterpret_cast<float*>(sbs + NH * RW * G);               // [kWaves][MT] (norm)
  float* part = red + kWaves * MT;                                        // [kWaves][NH][4][64]

  int seg = 0;
  if constexpr (EPI != QMV_SWIGLU) {
    if (p.nseg > 1 && static_cast<int>(blockIdx.x) >= p.seg[1].blk0) seg = 1;
    if (p.nseg > 2 && static_cast<int>(blockIdx.x) >= p.seg[2].blk0) seg = 2;
  }
  const int rows = p.seg[seg].rows;
  const int wrow0 = (static_cast<int>(blockIdx.x) - p.seg[seg].blk0) * RW;  // first row of the workgroup
  const int trow = wrow0 + tile * 16 + n_l;                                 // this lane's W row
  // groups of this wave: slice, slice + SK, ...
  const int n_g = (G - slice + SK - 1) / SK;

  // ---- 1. every W load of the wave (8 bytes per lane per group) ----
  u32x2 wv[NI][NH];
  {
    const int64_t rr = min(trow, rows - 1);
#pragma unroll
    for (int h = 0; h < NH; h++) {
      const uint32_t* wrow = p.seg[EPI == QMV_SWIGLU ? h : seg].w + rr * (K / 8) + 2 * q;
#pragma unroll
      for (int i = 0; i < NI; i++) {
        const int g = min(slice + SK * i, G - 1);
        wv[i][h] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(wrow + g * 8));
      }
    }
  }
  // ---- 2. optional RMSNorm of each x row: sums of squares ----
  const bool has_norm = p.norm_w != nullptr;
  if (has_norm) {
#pragma unroll
    for (int m = 0; m < MT; m++) {
      float t = 0.0f;
      if (m < M) {
        for (int j = threadIdx.x; j < U; j += kThreads) {
          const uint4 d = *reinterpret_cast<const uint4*>(p.x + m * p.ldx + j * 8);
          const uint32_t v[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
          for (int k = 0; k < 4; k++) {
            const float lo = bf2f(v[k] & 0xffffu), hi = bf2f(v[k] >> 16);
            t += lo * lo + hi * hi;
          }
        }
      }
      t = wave_sum_xor(t, 64);
      if (lane == 0) red[wave * MT + m] = t;
    }
    __syncthreads();
  }
  // ---- 3. x into LDS: pair-permuted units, group sums; s|b of the workgroup ----
  for (int b0 = 0; b0 < MT * U; b0 += kThreads * kXU) {
    uint4 xr[kXU], nr[kXU];
#pragma unroll
    for (int i = 0; i < kXU; i++) {
      const int e = min(b0 + i * kThreads + static_cast<int>(threadIdx.x), MT * U - 1);
      const int m = e / U, j = e - (e / U) * U;
      xr[i] = *reinterpret_cast<const uint4*>(p.x + min(m, M - 1) * p.ldx + j * 8);
      nr[i] = *reinterpret_cast<const uint4*>((has_norm ? p.norm_w : p.x) + j * 8);
    }
#pragma unroll
    for (int i = 0; i < kXU; i++) {
      const int e = b0 + i * kThreads + static_cast<int>(threadIdx.x);
      if (e >= MT * U) break;
      const int m = e / U, j = e - (e / U) * U;
      uint4 d = xr[i];
      if (m >= M) d = make_uint4(0, 0, 0, 0);  // rows beyond M: zeros
      if (has_norm && m < M) {
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; w++) t += red[w * MT + m];
        const float inv = 1.0f / sqrtf(t / static_cast<float>(K) + p.eps);
        uint32_t dv[4] = {d.x, d.y, d.z, d.w};
        const uint32_t wq[4] = {nr[i].x, nr[i].y, nr[i].z, nr[i].w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const float lo = bf2f(wq[k] & 0xffffu) * round_bf(bf2f(dv[k] & 0xffffu) * inv);
          const float hi = bf2f(wq[k] >> 16) * round_bf(bf2f(dv[k] >> 16) * inv);
          dv[k] = static_cast<uint32_t>(f2bf(lo)) | (static_cast<uint32_t>(f2bf(hi)) << 16);
        }
        d = make_uint4(dv[0], dv[1], dv[2], dv[3]);
      }
      xs[m * XS + j] = permute_pairs(d);
    }
  }
  // s|b of the workgroup's rows (4-byte words s | b << 16)
  for (int e = threadIdx.x; e < NH * RW * G; e += kThreads) {
    const int h = e / (RW * G);
    const int rem = e - h * (RW * G);
    const int r = rem / G, g = rem - (rem / G) * G;
    const QmvSegment& sg = p.seg[EPI == QMV_SWIGLU ? h : seg];
    const int64_t off = static_cast<int64_t>(min(wrow0 + r, rows - 1)) * G + g;
    sbs[e] = static_cast<uint32_t>(sg.s[off]) | (static_cast<uint32_t>(sg.b[off]) << 16);
  }
  __syncthreads();
  // group sums Sx[g][m] (rows >= M are zero) from the staged units
  for (int e = threadIdx.x; e < G * 16; e += kThreads) {
    const int g = e >> 4, m = e & 15;
    float t = 0.0f;
    if (m < MT) {
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const uint4 d = xs[m * XS + g * 8 + u];
        const uint32_t v[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
        for (int k = 0; k < 4; k++) t += bf2f(v[k] & 0xffffu) + bf2f(v[k] >> 16);
      }
    }
    sxs[e] = t;
  }
  __syncthreads();

  // ---- 4. MFMA over the wave's groups ----
  f32x4_t acc[NH];
#pragma unroll
  for (int h = 0; h < NH; h++) acc[h] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const int xm = n_l < MT ? n_l : 0;
  const bool xrow_live = n_l < MT;
#pragma unroll
  for (int i = 0; i < NI; i++) {
    if (i < n_g) {
      const int g = slice + SK * i;
      // rows >= MT of A are zero: select the values, not the address
      const uint4 v0 = xs[xm * XS + g * 8 + 2 * q];
      const uint4 v1 = xs[xm * XS + g * 8 + 2 * q + 1];
      const uint32_t keep = xrow_live ? 0xffffffffu : 0u;
      const uint4 a0u = make_uint4(v0.x & keep, v0.y & keep, v0.z & keep, v0.w & keep);
      const uint4 a1u = make_uint4(v1.x & keep, v1.y & keep, v1.z & keep, v1.w & keep);
      const bf16x8_t a0 = __builtin_bit_cast(bf16x8_t, a0u), a1 = __builtin_bit_cast(bf16x8_t, a1u);
      const f32x4_t sx = *reinterpret_cast<const f32x4_t*>(sxs + g * 16 + 4 * q);
#pragma unroll
      for (int h = 0; h < NH; h++) {
        f32x4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, nibbles_bf16(wv[i][h].x), d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, nibbles_bf16(wv[i][h].y), d, 0, 0, 0);
        const uint32_t sb = sbs[(h * RW + tile * 16 + n_l) * G + g];
        const float sv = bf2f(sb & 0xffffu);
        const float bb = bf2f(sb >> 16) - 128.0f * sv;
#pragma unroll
        for (int r = 0; r < 4; r++) {
          acc[h][r] += sv * d[r];
          acc[h][r] += bb * sx[r];
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  // ---- 5. add the SK partial tiles, epilogue ----
  if (SK > 1) {
#pragma unroll
    for (int h = 0; h < NH; h++)
#pragma unroll
      for (int r = 0; r < 4; r++) part[((wave * NH + h) * 4 + r) * 64 + lane] = acc[h][r];
    __syncthreads();
    if (slice == 0) {
      for (int s = 1; s < SK; s++) {
        const int w = s * TB + tile;
#pragma unroll
        for (int h = 0; h < NH; h++)
#pragma unroll
          for (int r = 0; r < 4; r++) acc[h][r] += part[((w * NH + h) * 4 + r) * 64 + lane];
      }
    }
  }
  if (slice == 0 && trow < rows) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int m = 4 * q + r;
      if (m >= M) break;
      if constexpr (EPI == QMV_STORE) {
        p.seg[seg].y[static_cast<int64_t>(m) * rows + trow] = f2bf(acc[0][r]);
      } else if constexpr (EPI == QMV_RESIDUAL) {
        // x = x + o_proj(attn) in bf16 (qwen3.rs:520-521, 541)
        const int64_t o = static_cast<int64_t>(m) * p.N + trow;
        p.seg[0].y[o] = f2bf(bf2f(p.res[o]) + round_bf(acc[0][r]));
      } else {
        // silu(gate) * up, each MLX op rounding to bf16 (kernels.rs:73-74)
        const float g = round_bf(acc[0][r]);
        const float u = round_bf(acc[NH - 1][r]);
        const float sg = round_bf(1.0f / (1.0f + expf(-g)));
        p.seg[0].y[static_cast<int64_t>(m) * p.N + trow] = f2bf(round_bf(g * sg) * u);
      }
    }
  }
}

template <int MT, int NI>
int launch_ni(QmvEpilogue epi, const QmvParams& p, int TB, int blocks, size_t lds, hipStream_t st) {
  switch (epi) {
    case QMV_STORE:
      if (int rc = allow_lds(qmvx_kernel<MT, NI, QMV_STORE>, lds)) return rc;
      hipLaunchKernelGGL((qmvx_kernel<MT, NI, QMV_STORE>), dim3(blocks), dim3(kThreads), lds, st, p, TB);
      break;
    case QMV_RESIDUAL:
      if (int rc = allow_lds(qmvx_kernel<MT, NI, QMV_RESIDUAL>, lds)) return rc;
      hipLaunchKernelGGL((qmvx_kernel<MT, NI, QMV_RESIDUAL>), dim3(blocks), dim3(kThreads), lds, st, p, TB);
      break;
    default:
      if (int rc = allow_lds(qmvx_kernel<MT, NI, QMV_SWIGLU>, lds)) return rc;
      hipLaunchKernelGGL((qmvx_kernel<MT, NI, QMV_SWIGLU>), dim3(blocks), dim3(kThreads), lds, st, p, TB);
  }
  return check_launch("qmvx");
}

template <int MT>
int launch_mt(int ni, QmvEpilogue epi, const QmvParams& p, int TB, int blocks, size_t lds, hipStream_t st) {
  if (ni <= 4) return launch_ni<MT, 4>(epi, p, TB, blocks, lds, st);
  if (ni <= 8) return launch_ni<MT, 8>(epi, p, TB, blocks, lds, st);
  if (ni <= 16) return launch_ni<MT, 16>(epi, p, TB, blocks, lds, st);
  if (ni <= 24 && epi != QMV_SWIGLU) return launch_ni<MT, 24>(epi, p, TB, blocks, lds, st);
  return -1;
}

}  // namespace

int try_launch_qmvx(QmvParams p, QmvEpilogue epi, hipStream_t stream) {
  if (p.m < 2 || p.m > 8) return -1;
  const int mt = p.m <= 2 ? 2 : p.m <= 4 ? 4 : p.m <= 5 ? 5 : 8;
  const int G = p.K / 64;
  const int nh = epi == QMV_SWIGLU ? 2 : 1;
  // tiles per workgroup: as many as keep >= ~1024 workgroups' worth of
  // waves on the chip, the rest of the 8 waves split K
  int rows_total = 0;
  if (epi == QMV_SWIGLU) rows_total = p.N;
  else
    for (int i = 0; i < p.nseg; i++) rows_total += p.seg[i].rows;
  int TB = 8;
  while (TB > 1 && (rows_total + 16 * TB - 1) / (16 * TB) < 256) TB >>= 1;
  static const int env_tb = getenv("BMX_QMVX_TB") ? atoi(getenv("BMX_QMVX_TB")) : 0;
  if (env_tb == 1 || env_tb == 2 || env_tb == 4 || env_tb == 8) TB = env_tb;
  // groups per wave within what is instantiated (16 for SwiGLU, 24 else)
  const int max_ni = nh == 2 ? 16 : 24;
  while (TB > 1 && (G + kWaves / TB - 1) / (kWaves / TB) > max_ni) TB >>= 1;
  const int SK = kWaves / TB;
  const int ni = (G + SK - 1) / SK;
  if (ni > max_ni) return -1;
  const int RW = 16 * TB;
  const size_t lds = static_cast<size_t>(mt) * (G * 8 + 1) * 16 + static_cast<size_t>(G) * 16 * 4 +
                     static_cast<size_t>(nh) * RW * G * 4 + kWaves * mt * 4 +
                     (SK > 1 ? static_cast<size_t>(kWaves) * nh * 4 * 64 * 4 : 0);
  if (lds > 160 * 1024) return -1;
  // segments start on workgroup boundaries
  int blocks = 0;
  if (epi == QMV_SWIGLU) {
    blocks = (p.N + RW - 1) / RW;
    for (int i = 0; i < p.nseg; i++) p.seg[i].blk0 = 0;
  } else {
    for (int i = 0; i < p.nseg; i++) {
      p.seg[i].blk0 = blocks;
      blocks += (p.seg[i].rows + RW - 1) / RW;
    }
  }
  switch (mt) {
    case 2: return launch_mt<2>(ni, epi, p, TB, blocks, lds, stream);
    case 4: return launch_mt<4>(ni, epi, p, TB, blocks, lds, stream);
    case 5: return launch_mt<5>(ni, epi, p, TB, blocks, lds, stream);
    default: return launch_mt<8>(ni, epi, p, TB, blocks, lds, stream);
  }
}

}  // namespace bmx
