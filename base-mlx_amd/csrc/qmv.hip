// qmv: MLX-format 4-bit affine quantized GEMV for M <= 8 rows of x
// (decode M=1, speculative verify M=5), gfx950.
//
// Semantics restated: mlx_rs::ops::quantized_matmul(x, W, s, b,
// transpose=true, group_size=64, bits=4) as called from QLinear::forward
// (crates/base-mlx-core/src/model/qwen3.rs:30-41), the tied lm_head
// (qwen3.rs:80-91) and the fused blocks (model/kernels.rs:42-44, 69-75):
//   y[m,n] = sum_g s[n,g] * sum_{k in g} q[n,k] x[m,k] + b[n,g] * sum_{k in g} x[m,k]
// with fp32 accumulation and a bf16 result.
//
// Work decomposition.  A workgroup owns RB = 4 * 64/S consecutive output
// rows; each row is served by S lanes of one wave that stride over the
// row's 16-byte chunks of packed W (32 nibbles, half a 64-wide group), so
// S consecutive lanes read S*16 contiguous bytes of a row per load.  The
// main loop issues exactly one vector-memory instruction per 16 bytes of W:
// everything else it needs comes from LDS, staged once per workgroup with
// 16-byte loads --
//   * x, pair-permuted so that the nibble pairs (q_e, q_{e+4}) of a packed
//     word line up with (x_e, x_{e+4}):
//       (w & 0x000F000F) | 0x43004300 == bf16 pair (128 + q0, 128 + q4)
//     which feeds v_dot2c_f32_bf16 directly;
//   * per-chunk sums Sx, which remove the +128 offset:
//       sum_k q x = D - 128 Sx,  so  y += s * D + (b - 128 s) * Sx;
//   * the workgroup's rows of s and b, interleaved as (s | b << 16).
// W loads run U chunks ahead in a register ring; the first U are issued
// before the staging so HBM latency overlaps it.  Each 64-byte x chunk
// occupies 80 bytes of LDS so the 16-byte reads of 8 consecutive lanes
// land in distinct banks.  Lanes of a row are reduced with xor shuffles.
#include <stdlib.h>

#include <algorithm>
#include <type_traits>

#include "bmx_device.h"

namespace bmx {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kChunkBytes = 80;  // 64 data bytes + 16 pad per 32 x values
constexpr int kLdsBudget = 40 * 1024;

// The epilogue of output (m, row): y, y = res + y (o / down projections,
// qwen3.rs:520-521, 541) or SwiGLU silu(gate) * up (kernels.rs:73-74), each
// MLX op rounding to bf16.  g / u are the fp32 sums of the (first, second)
// weight matrix.
template <int EPI>
__device__ __forceinline__ void gemv_store(const QmvParams& p, int seg, int m, int rows, int row, float g, float u) {
  if constexpr (EPI == QMV_STORE) {
    p.seg[seg].y[static_cast<int64_t>(m) * rows + row] = f2bf(g);
  } else if constexpr (EPI == QMV_RESIDUAL) {
    const int64_t o = static_cast<int64_t>(m) * p.N + row;
    p.seg[0].y[o] = f2bf(bf2f(p.res[o]) + round_bf(g));
  } else {
    const float gr = round_bf(g);
    const float ur = round_bf(u);
    const float sg = round_bf(1.0f / (1.0f + expf(-gr)));
    p.seg[0].y[static_cast<int64_t>(m) * p.N + row] = f2bf(round_bf(gr * sg) * ur);
  }
}

// Phased GEMV: any K, s / b in 16-byte units or one group at a time.  x and
// the workgroup's s|b are staged in LDS one phase of p.kp columns at a time
// (p.kp a multiple of 32 S, so lane sl still meets its chunks c = sl mod S
// in increasing order, as in the single-phase kernels).  W streams U chunks
// ahead in a register ring that runs across phase boundaries (W does not
// wait for x): lane chunk i sits in slot i mod U.  S (lanes per row) is a
// launch parameter.
template <int MT, int EPI, int U>
__global__ void __launch_bounds__(kThreads) qmv_kernel(const QmvParams p, const int S) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int NH = (EPI == QMV_SWIGLU) ? 2 : 1;  // weight rows per lane
  const int lshift = __builtin_ctz(S);
  const int SLOTS = 64 >> lshift;
  const int RB = 4 * SLOTS;  // rows per workgroup
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int slot = lane >> lshift;
  const int sl = lane & (S - 1);
  const int M = p.m;
  const int K = p.K;
  const int G = K / 64;
  const int CP = p.kp / 32;  // x chunks per phase
  const int GP = p.kp / 64;  // groups per phase
  unsigned char* xs = smem;                                                 // [MT][CP] x 80 B
  float* sxs = reinterpret_cast<float*>(smem + MT * CP * kChunkBytes);      // [MT][CP]
  uint32_t* sbs = reinterpret_cast<uint32_t*>(sxs + MT * CP);               // [NH][RB][GP]
  float* red = reinterpret_cast<float*>(sbs + NH * RB * GP);                // [4][MT]
  float* amv = red + 4 * MT;                                                 // [MT][RB] (argmax partials)
  uint32_t* ami = reinterpret_cast<uint32_t*>(amv + MT * RB);                // [MT][RB]

  // Segments start on workgroup boundaries, so the segment (and every
  // kernel-argument field read through it) is uniform across the workgroup
  // and is read with scalar loads.
  int seg = 0;
  if constexpr (EPI != QMV_SWIGLU) {
    if (p.nseg > 1 && static_cast<int>(blockIdx.x) >= p.seg[1].blk0) seg = 1;
    if (p.nseg > 2 && static_cast<int>(blockIdx.x) >= p.seg[2].blk0) seg = 2;
  }
  const int rows = p.seg[seg].rows;
  const int row0 = (static_cast<int>(blockIdx.x) - p.seg[seg].blk0) * RB;  // first row of the workgroup
  const int rl = wave * SLOTS + slot;  // row within the workgroup
  const int row = row0 + rl;           // row within the segment
  const bool valid = row < rows;

  const uint32_t* wrow[NH];
  {
    const int64_t rr = min(row, rows - 1);
#pragma unroll
    for (int h = 0; h < NH; h++) wrow[h] = p.seg[EPI == QMV_SWIGLU ? h : seg].w + rr * (K / 8);
  }

  constexpr int XU = 4;  // x words per thread per staging batch
  constexpr int SU = 2;  // s|b units per thread per staging batch
  uint4 wv[U][NH];
  auto load_chunk = [&](int u, int c) {
#pragma unroll
    for (int h = 0; h < NH; h++) {
      // W is streamed exactly once: nontemporal loads keep it out of the way
      const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[h] + c * 4));
      wv[u][h] = make_uint4(t.x, t.y, t.z, t.w);
    }
  };
  // the lane's chunks over all of K: c = sl + S i, i < n_all; the first U
  // go out before anything else
  const int C = K / 32;
  const int n_all = sl < C ? (C - sl + S - 1) / S : 0;
#pragma unroll
  for (int u = 0; u < U; u++)
    if (u < n_all) load_chunk(u, sl + S * u);

  // Optional fused RMSNorm of each x row (fast::rms_norm, qwen3.rs:50-55):
  //   h = w * bf16(x * rsqrt(mean(x^2) + eps)); thread t sums units t,
  //   t + 256, ... of the row (the single-phase kernels' assignment)
  float inv[MT];
#pragma unroll
  for (int m = 0; m < MT; m++) inv[m] = 1.0f;
  if (p.norm_w != nullptr) {
#pragma unroll
    for (int m = 0; m < MT; m++) {
      float ss = 0.0f;
      if (m < M) {
        const uint16_t* xr = p.x + m * p.ldx;
        for (int k = threadIdx.x * 8; k < K; k += kThreads * 8)
          ss = gemv_ss_unit(*reinterpret_cast<const uint4*>(xr + k), ss);
      }
      ss = lanes_sum(ss, 64);
      if (lane == 0) red[wave * MT + m] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < MT; m++) inv[m] = gemv_norm_inv(red[m], red[MT + m], red[2 * MT + m], red[3 * MT + m], K, p.eps);
  }

  float acc[NH][MT];
#pragma unroll
  for (int h = 0; h < NH; h++)
#pragma unroll
    for (int m = 0; m < MT; m++) acc[h][m] = 0.0f;

  for (int k0 = 0, i0 = 0; k0 < K; k0 += p.kp) {
    const int kpp = min(p.kp, K - k0);
    const int words = kpp / 8;  // multiple of 8
    const int total = MT * words;
    const int ncp = kpp / 32;   // chunks in this phase
    const int gpp = kpp / 64;   // groups in this phase
    const int cbase = k0 / 32;  // a multiple of S
    const int gbase = k0 / 64;
    // this lane's chunks of the phase: i in [i0, i1)
    const int i1 = sl < cbase + ncp ? (cbase + ncp - sl + S - 1) / S : 0;
    __syncthreads();  // previous phase finished reading LDS
    // ---- stage x[:, k0:k0+kpp] (pair-permuted, chunk sums) and the
    //      workgroup's s|b words.  Each batch issues all of its loads before
    //      consuming any, so their latencies overlap (and overlap W). ----
    const int gunits = gpp / 8;  // 16-byte s/b units per row
    const int sb_units = p.sb_vec ? RB * gunits : RB * gpp;  // per weight matrix
    const float rcp_words = 1.0f / static_cast<float>(words);
    const float rcp_gu = 1.0f / static_cast<float>(p.sb_vec ? gunits : gpp);
    for (int b0x = 0, b0s = 0; b0x < total || b0s < sb_units; b0x += kThreads * XU, b0s += kThreads * SU) {
      uint4 xr[XU];
      uint4 sr[NH][SU], br[NH][SU];
#pragma unroll
      for (int i = 0; i < XU; i++) {
        const int idx = b0x + i * kThreads + threadIdx.x;
        xr[i] = make_uint4(0, 0, 0, 0);
        if (idx < total) {
          const int m = (MT == 1) ? 0 : udiv_small(idx, rcp_words);
          if (m < M) xr[i] = *reinterpret_cast<const uint4*>(p.x + m * p.ldx + k0 + (idx - m * words) * 8);
        }
      }
      if (p.sb_vec) {
#pragma unroll
        for (int h = 0; h < NH; h++) {
          const QmvSegment& sgm = p.seg[EPI == QMV_SWIGLU ? h : seg];
#pragma unroll
          for (int i = 0; i < SU; i++) {
            const int e = b0s + i * kThreads + threadIdx.x;
            const int r = udiv_small(e, rcp_gu);
            if (e < sb_units && row0 + r < rows) {
              const int64_t off = static_cast<int64_t>(row0 + r) * G + gbase + (e - r * gunits) * 8;
              sr[h][i] = *reinterpret_cast<const uint4*>(sgm.s + off);
              br[h][i] = *reinterpret_cast<const uint4*>(sgm.b + off);
            }
          }
        }
      }
      // consume x
#pragma unroll
      for (int i = 0; i < XU; i++) {
        const int idx = b0x + i * kThreads + threadIdx.x;
        const bool act = idx < total;
        const int m = (MT == 1 || !act) ? 0 : udiv_small(idx, rcp_words);
        const int j = act ? idx - m * words : 0;
        uint4 d = xr[i];
        float part = 0.0f;
        if (act && m < M) {
          if (p.norm_w != nullptr)
            d = gemv_norm_unit(d, *reinterpret_cast<const uint4*>(p.norm_w + k0 + j * 8), inv[m]);
          part = gemv_unit_sum(d);
        }
        // a chunk of 32 values = 4 consecutive words = 4 consecutive lanes
        // (words is a multiple of 8, so j and threadIdx.x agree mod 4)
        part += dpp_f32<0xB1>(part);
        part += dpp_f32<0x4E>(part);
        if (act) {
          *reinterpret_cast<uint4*>(xs + (m * CP + (j >> 2)) * kChunkBytes + (j & 3) * 16) = permute_pairs(d);
          if ((j & 3) == 0) sxs[m * CP + (j >> 2)] = part;
        }
      }
      // consume s|b
#pragma unroll
      for (int h = 0; h < NH; h++) {
        const QmvSegment& sgm = p.seg[EPI == QMV_SWIGLU ? h : seg];
#pragma unroll
        for (int i = 0; i < SU; i++) {
          const int e = b0s + i * kThreads + threadIdx.x;
          const int r = udiv_small(e, rcp_gu);
          if (e >= sb_units || row0 + r >= rows) continue;
          if (p.sb_vec) {
            const uint32_t s4[4] = {sr[h][i].x, sr[h][i].y, sr[h][i].z, sr[h][i].w};
            const uint32_t b4[4] = {br[h][i].x, br[h][i].y, br[h][i].z, br[h][i].w};
            uint32_t* dst = sbs + (h * RB + r) * GP + (e - r * gunits) * 8;
#pragma unroll
            for (int q = 0; q < 4; q++) {
              dst[2 * q] = (s4[q] & 0xffffu) | (b4[q] << 16);
              dst[2 * q + 1] = (s4[q] >> 16) | (b4[q] & 0xffff0000u);
            }
          } else {
            const int g = e - r * gpp;
            const int64_t off = static_cast<int64_t>(row0 + r) * G + gbase + g;
            sbs[(h * RB + r) * GP + g] = static_cast<uint32_t>(sgm.s[off]) | (static_cast<uint32_t>(sgm.b[off]) << 16);
          }
        }
      }
    }
    __syncthreads();

    // ---- stream W over this phase's chunks (slot u = i mod U; the
    // unrolled rounds start at the ring-aligned chunk at or below i0) ----
    const NibbleK nk = nibble_consts();
    for (int ib = (i0 / U) * U; ib < i1; ib += U) {
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int i = ib + u;
        if (i >= i0 && i < i1) {
          const int c = sl + S * i - cbase;  // chunk within the phase
          float sv[NH], bb[NH];
#pragma unroll
          for (int h = 0; h < NH; h++) gemv_sb(sbs[(h * RB + rl) * GP + (c >> 1)], sv[h], bb[h]);
#pragma unroll
          for (int m = 0; m < MT; m++) {
            if (m < M) {
              const uint4* xp = reinterpret_cast<const uint4*>(xs + (m * CP + c) * kChunkBytes);
              const uint4 x0 = xp[0], x1 = xp[1], x2 = xp[2], x3 = xp[3];
              const float sx = sxs[m * CP + c];
#pragma unroll
              for (int h = 0; h < NH; h++) acc[h][m] = gemv_chunk(wv[u][h], x0, x1, x2, x3, sv[h], bb[h], sx, acc[h][m], nk);
            }
          }
          if (i + U < n_all) load_chunk(u, sl + S * (i + U));
        }
      }
    }
    i0 = i1;
  }

  // ---- reduce the S lanes of each row and write ----
#pragma unroll
  for (int h = 0; h < NH; h++)
#pragma unroll
    for (int m = 0; m < MT; m++) acc[h][m] = lanes_sum(acc[h][m], S);

  if (sl == 0 && valid) {
#pragma unroll
    for (int m = 0; m < MT; m++) {
      if (m >= M) break;
      gemv_store<EPI>(p, seg, m, rows, row, acc[0][m], acc[NH - 1][m]);
    }
  }
  if constexpr (EPI == QMV_STORE) {
    if (p.amax != nullptr) {
      // argmax partial of the workgroup's rows (first index on ties)
      if (sl == 0) {
#pragma unroll
        for (int m = 0; m < MT; m++) {
          const bool ok = valid && m < M;
          amv[m * RB + rl] = ok ? bf2f(f2bf(acc[0][m])) : -INFINITY;
          ami[m * RB + rl] = ok ? static_cast<uint32_t>(row) : 0xffffffffu;
        }
      }
      __syncthreads();
      if (static_cast<int>(threadIdx.x) < M) {
        const int m = threadIdx.x;
        float bv = -INFINITY;
        uint32_t bi = 0xffffffffu;
        for (int r = 0; r < RB; r++) {
          const float v = amv[m * RB + r];
          const uint32_t i = ami[m * RB + r];
          if (v > bv || (v == bv && i < bi)) {
            bv = v;
            bi = i;
          }
        }
        p.amax[static_cast<int64_t>(m) * gridDim.x + blockIdx.x] = make_uint2(__float_as_uint(bv), bi);
      }
    }
  }
}

// Single-phase GEMV, the decode shapes: 1..8 rows of x (MT) with the whole K
// in one LDS phase.  Every load of the workgroup is unconditional (indices
// are clamped; duplicate addresses coalesce inside an instruction): first
// x, the norm weight, s|b and the lane's first 16-byte W chunk; then, once x
// and s|b are staged in LDS, the remaining NI - 1 chunks.  With the count of
// loads in flight fixed, the compiler waits for each W chunk on its own, so
// the dot products of chunk u overlap the arrival of the later ones.
// S (lanes per row) is a launch parameter; NI = ceil(K/32 / S) rounded up to
// an instantiated value.
constexpr int kXU1 = 5;  // x units (8 values) per thread: K <= 256 * 8 * 5

// XU: x units per thread and row the launch needs (2 up to K = 4096, else
// kXU1), so that no thread issues loads of clamped duplicates; NORM: the
// RMSNorm prologue (p.norm_w set), whose weight loads are issued only then
template <int NI, int EPI, int XU, bool NORM, int MT>
__global__ void __launch_bounds__(kThreads) qmv1_kernel(const QmvParams p, const int S) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int NH = (EPI == QMV_SWIGLU) ? 2 : 1;
  const int lshift = __builtin_ctz(S);
  const int SLOTS = 64 >> lshift;
  const int RB = 4 * SLOTS;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int slot = lane >> lshift;
  const int sl = lane & (S - 1);
  const int M = p.m;
  const int K = p.K;
  const int G = K / 64, C = K / 32, W8 = K / 8, GU = G / 8;
  unsigned char* xs = smem;                                             // [MT][C] x 80 B
  float* sxs = reinterpret_cast<float*>(smem + MT * C * kChunkBytes);   // [MT][C]
  uint32_t* sbs = reinterpret_cast<uint32_t*>(sxs + MT * C);            // [NH][RB][G]
  float* red = reinterpret_cast<float*>(sbs + NH * RB * G);             // [4][MT]
  float* amv = red + 4 * MT;                                            // [RB]
  uint32_t* ami = reinterpret_cast<uint32_t*>(amv + RB);                // [RB]

  int seg = 0;
  if constexpr (EPI != QMV_SWIGLU) {
    if (p.nseg > 1 && static_cast<int>(blockIdx.x) >= p.seg[1].blk0) seg = 1;
    if (p.nseg > 2 && static_cast<int>(blockIdx.x) >= p.seg[2].blk0) seg = 2;
  }
  const int rows = p.seg[seg].rows;
  const int row0 = (static_cast<int>(blockIdx.x) - p.seg[seg].blk0) * RB;
  const int rl = wave * SLOTS + slot;
  const int row = row0 + rl;
  const bool valid = row < rows;
  const uint16_t* nw = p.norm_w;

  // ---- 1. staging loads (unconditional, clamped) ----
  uint4 xr[MT][XU], nr[XU];
#pragma unroll
  for (int i = 0; i < XU; i++) {
    const int idx = min(i * kThreads + static_cast<int>(threadIdx.x), W8 - 1);
#pragma unroll
    for (int m = 0; m < MT; m++) xr[m][i] = *reinterpret_cast<const uint4*>(p.x + min(m, M - 1) * p.ldx + idx * 8);
    if constexpr (NORM) nr[i] = *reinterpret_cast<const uint4*>(nw + idx * 8);
  }
  uint4 sr[NH], br[NH];
  const int sb_units = RB * GU;
  const float rcp_gu = 1.0f / static_cast<float>(GU);
  const int e_sb = min(static_cast<int>(threadIdx.x), sb_units - 1);
  const int r_sb = udiv_small(e_sb, rcp_gu);
#pragma unroll
  for (int h = 0; h < NH; h++) {
    const QmvSegment& sgm = p.seg[EPI == QMV_SWIGLU ? h : seg];
    const int64_t off = static_cast<int64_t>(min(row0 + r_sb, rows - 1)) * G + (e_sb - r_sb * GU) * 8;
    sr[h] = *reinterpret_cast<const uint4*>(sgm.s + off);
    br[h] = *reinterpret_cast<const uint4*>(sgm.b + off);
  }
  // keep the staging loads ahead of the W stream in issue order
  __builtin_amdgcn_sched_barrier(0);
  // ---- 2. the lane's W chunks, in the order they are consumed: chunk by
  // chunk, both matrices of a chunk together.  Only chunk 0 goes out here;
  // the others after x and s|b are staged (step 4): the issuing wave stalls
  // while the load queue drains, so staging between the two batches overlaps
  // the W stream instead of waiting behind the whole issue loop ----
  uint4 wv[NI][NH];
  const uint32_t* wrow[NH];
  {
    const int64_t rr = min(row, rows - 1);
#pragma unroll
    for (int h = 0; h < NH; h++) wrow[h] = p.seg[EPI == QMV_SWIGLU ? h : seg].w + rr * (K / 8);
  }
  auto issue_w = [&](int u) {
    const int c = min(sl + (u << lshift), C - 1);
#pragma unroll
    for (int h = 0; h < NH; h++) {
      const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[h] + c * 4));
      wv[u][h] = make_uint4(t.x, t.y, t.z, t.w);
    }
  };
  issue_w(0);
  // ---- 3. fused RMSNorm (fast::rms_norm, qwen3.rs:50-55) of each x row
  //      from the staged x: h = w * bf16(x * rsqrt(mean(x^2) + eps)) ----
  float inv[MT];
#pragma unroll
  for (int m = 0; m < MT; m++) inv[m] = 1.0f;
  if constexpr (NORM) {
#pragma unroll
    for (int m = 0; m < MT; m++) {
      float ss = 0.0f;
      if (m < M) {
#pragma unroll
        for (int i = 0; i < XU; i++) {
          if (i * kThreads >= W8) break;  // uniform: the remaining units are clamped copies
          if (i * kThreads + static_cast<int>(threadIdx.x) < W8) ss = gemv_ss_unit(xr[m][i], ss);
        }
      }
      ss = lanes_sum(ss, 64);
      if (lane == 0) red[wave * MT + m] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < MT; m++) inv[m] = gemv_norm_inv(red[m], red[MT + m], red[2 * MT + m], red[3 * MT + m], K, p.eps);
  }
  // ---- 4. x (pair-permuted, chunk sums) and s|b into LDS ----
#pragma unroll
  for (int m = 0; m < MT; m++) {
    if (m >= M) break;
#pragma unroll
    for (int i = 0; i < XU; i++) {
      if (i * kThreads >= W8) break;  // uniform: the remaining units are clamped copies
      const int idx = i * kThreads + static_cast<int>(threadIdx.x);
      const bool act = idx < W8;
      uint4 d = xr[m][i];
      float part = 0.0f;
      if (act) {
        if constexpr (NORM) d = gemv_norm_unit(d, nr[i], inv[m]);
        part = gemv_unit_sum(d);
      }
      // a chunk of 32 values = 4 consecutive words = 4 consecutive lanes
      part += dpp_f32<0xB1>(part);
      part += dpp_f32<0x4E>(part);
      if (act) {
        *reinterpret_cast<uint4*>(xs + (m * C + (idx >> 2)) * kChunkBytes + (idx & 3) * 16) = permute_pairs(d);
        if ((idx & 3) == 0) sxs[m * C + (idx >> 2)] = part;
      }
    }
  }
  if (static_cast<int>(threadIdx.x) < sb_units && row0 + r_sb < rows) {
#pragma unroll
    for (int h = 0; h < NH; h++) {
      const uint32_t s4[4] = {sr[h].x, sr[h].y, sr[h].z, sr[h].w};
      const uint32_t b4[4] = {br[h].x, br[h].y, br[h].z, br[h].w};
      uint32_t* dst = sbs + (h * RB + r_sb) * G + (e_sb - r_sb * GU) * 8;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        dst[2 * q] = (s4[q] & 0xffffu) | (b4[q] << 16);
        dst[2 * q + 1] = (s4[q] >> 16) | (b4[q] & 0xffff0000u);
      }
    }
  }
  // the rest of the W stream (step 2)
#pragma unroll
  for (int u = 1; u < NI; u++) issue_w(u);
  __syncthreads();
  // ---- 5. dot products, chunk by chunk as the W stream arrives ----
  const NibbleK nk = nibble_consts();
  float acc[NH][MT];
#pragma unroll
  for (int h = 0; h < NH; h++)
#pragma unroll
    for (int m = 0; m < MT; m++) acc[h][m] = 0.0f;
#pragma unroll
  for (int u = 0; u < NI; u++) {
    const int c = sl + (u << lshift);
    if (c < C) {
      float sv[NH], bb[NH];
#pragma unroll
      for (int h = 0; h < NH; h++) gemv_sb(sbs[(h * RB + rl) * G + (c >> 1)], sv[h], bb[h]);
#pragma unroll
      for (int m = 0; m < MT; m++) {
        if (m >= M) break;
        const uint4* xp = reinterpret_cast<const uint4*>(xs + (m * C + c) * kChunkBytes);
        const uint4 x0 = xp[0], x1 = xp[1], x2 = xp[2], x3 = xp[3];
        const float sx = sxs[m * C + c];
#pragma unroll
        for (int h = 0; h < NH; h++) acc[h][m] = gemv_chunk(wv[u][h], x0, x1, x2, x3, sv[h], bb[h], sx, acc[h][m], nk);
      }
    }
    // consume the chunks in issue order (each waits only for its own loads)
    __builtin_amdgcn_sched_barrier(0);
  }
  // ---- 6. reduce the S lanes of each row, epilogue ----
#pragma unroll
  for (int h = 0; h < NH; h++)
#pragma unroll
    for (int m = 0; m < MT; m++) acc[h][m] = lanes_sum(acc[h][m], S);
  if (sl == 0 && valid) {
#pragma unroll
    for (int m = 0; m < MT; m++) {
      if (m >= M) break;
      gemv_store<EPI>(p, seg, m, rows, row, acc[0][m], acc[NH - 1][m]);
    }
  }
  if constexpr (EPI == QMV_STORE && MT == 1) {
    if (p.amax != nullptr) {
      // argmax partial of the workgroup's rows (first index on ties): across
      // the row slots of each wave with shuffles, then the 4 waves in LDS
      float bv = valid ? bf2f(f2bf(acc[0][0])) : -INFINITY;
      uint32_t bi = valid ? static_cast<uint32_t>(row) : 0xffffffffu;
      for (int off = S; off < 64; off <<= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const uint32_t oi = __shfl_xor(bi, off, 64);
        if (ov > bv || (ov == bv && oi < bi)) {
          bv = ov;
          bi = oi;
        }
      }
      if (lane == 0) {
        amv[wave] = bv;
        ami[wave] = bi;
      }
      __syncthreads();
      if (threadIdx.x == 0) {
#pragma unroll
        for (int w = 1; w < 4; w++)
          if (amv[w] > bv || (amv[w] == bv && ami[w] < bi)) {
            bv = amv[w];
            bi = ami[w];
          }
        p.amax[blockIdx.x] = make_uint2(__float_as_uint(bv), bi);
      }
    }
  }
}

template <int NI, int XU, int MT>
int launch_qmv1_xu(QmvEpilogue epi, int S, const QmvParams& p, int blocks, size_t lds, hipStream_t st) {
  const bool norm = p.norm_w != nullptr;
  auto go = [&](auto kern) {
    if (int rc = allow_lds(kern, lds)) return rc;
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(kThreads), lds, st, p, S);
    return check_launch("qmv1");
  };
  // the combinations the library uses: store with or without the fused
  // norm (q|k|v, lm_head; plain projections), residual without it (o,
  // down), SwiGLU with it (gate|up); others go to the phased kernel
  switch (epi) {
    case QMV_STORE:
      return norm ? go(qmv1_kernel<NI, QMV_STORE, XU, true, MT>) : go(qmv1_kernel<NI, QMV_STORE, XU, false, MT>);
    case QMV_RESIDUAL:
      return norm ? kNoFit : go(qmv1_kernel<NI, QMV_RESIDUAL, XU, false, MT>);
    default:
      return norm ? go(qmv1_kernel<NI, QMV_SWIGLU, XU, true, MT>) : kNoFit;
  }
}

// x units per thread and row: 2 up to K = 4096, else kXU1; several rows stay
// within 12 units per thread in all
constexpr int qmv1_xu(int K) { return K / 8 <= 2 * kThreads ? 2 : kXU1; }
constexpr bool qmv1_fits(int mt, int xu) { return mt == 1 || mt * xu <= 12; }

template <int NI, int MT>
int launch_qmv1_ni(QmvEpilogue epi, int S, const QmvParams& p, int blocks, size_t lds, hipStream_t st) {
  if (qmv1_xu(p.K) == 2) {
    if constexpr (qmv1_fits(MT, 2)) return launch_qmv1_xu<NI, 2, MT>(epi, S, p, blocks, lds, st);
  } else {
    if constexpr (qmv1_fits(MT, kXU1)) return launch_qmv1_xu<NI, kXU1, MT>(epi, S, p, blocks, lds, st);
  }
  return kNoFit;
}

template <int MT>
int launch_qmv1_mt(int ni, int nh, QmvEpilogue epi, int S, const QmvParams& p, int blocks, size_t lds,
                   hipStream_t st) {
  if (ni <= 2) return launch_qmv1_ni<2, MT>(epi, S, p, blocks, lds, st);
  if (ni <= 3) return launch_qmv1_ni<3, MT>(epi, S, p, blocks, lds, st);
  if (ni <= 5) return launch_qmv1_ni<5, MT>(epi, S, p, blocks, lds, st);
  if (ni <= 8) return launch_qmv1_ni<8, MT>(epi, S, p, blocks, lds, st);
  if (nh == 1 && ni <= 10) return launch_qmv1_ni<10, MT>(epi, S, p, blocks, lds, st);
  if (nh == 1 && ni <= 16) return launch_qmv1_ni<16, MT>(epi, S, p, blocks, lds, st);
  return kNoFit;
}

// Launches the single-phase GEMV when it applies (one phase, 16-byte s|b
// staging, x within kXU1 units per thread and row -- with several rows at
// most 12 units per thread in all, so the staging stays in registers -- and
// the workgroup's s|b within one unit per thread); returns kNoFit otherwise.
int try_launch_qmv1(QmvEpilogue epi, int mt, int S, const QmvParams& p, int blocks, hipStream_t st) {
  if (!p.sb_vec || p.K / 8 > kThreads * kXU1) return kNoFit;
  if (!qmv1_fits(mt, qmv1_xu(p.K))) return kNoFit;
  const int C = p.K / 32, G = p.K / 64;
  const int RB = 4 * (64 / S);
  if (RB * (G / 8) > kThreads) return kNoFit;
  const int ni = (C + S - 1) / S;
  const int nh = epi == QMV_SWIGLU ? 2 : 1;
  const size_t lds = static_cast<size_t>(mt) * C * (kChunkBytes + 4) + static_cast<size_t>(nh) * RB * G * 4 +
                     16ull * mt + static_cast<size_t>(RB) * 8;
  if (lds > 160 * 1024) return kNoFit;
  switch (mt) {
    case 1: return launch_qmv1_mt<1>(ni, nh, epi, S, p, blocks, lds, st);
    case 2: return launch_qmv1_mt<2>(ni, nh, epi, S, p, blocks, lds, st);
    case 4: return launch_qmv1_mt<4>(ni, nh, epi, S, p, blocks, lds, st);
    case 5: return launch_qmv1_mt<5>(ni, nh, epi, S, p, blocks, lds, st);
    default: return kNoFit;  // 8 rows exceed the staging registers
  }
}

// One-workgroup-per-CU GEMV for one row of x (the decode step's q|k|v, o,
// gate|up and down projections).  A launch of one workgroup per CU (up to
// 16 waves, a block of consecutive weight rows each) removes the load
// ordering that holds the single-workgroup kernels back: every wave first
// issues its staging loads (x, the norm weight, its rows' s|b), the
// workgroup meets at a barrier -- so on each CU all of them are queued ahead
// of any W load -- and then every lane issues its whole W stream at once;
// the RMSNorm and the LDS staging run while W is on its way.  Each row is
// computed with the operations of qmv1_kernel in the same order (the same S
// lanes per row and chunk -> lane assignment, the norm's sums of squares
// from the first 256 threads as qmv1 assigns them, the same chunk sums and
// reductions), so its bits equal qmv1's for the same row.  Rows of a
// workgroup may span q|k|v segments: a lane's segment follows its row.
constexpr int kQmvcMaxThreads = 1024;
constexpr int kQmvcMinLanes = 16;  // lanes per row from which it is used
constexpr int kQmvcPreLoads = 40;   // W loads per CU all issued ahead of the staging
constexpr int kQmvcPipeLoads = 32;  // else about this many, the rest pipelined

__device__ __forceinline__ int qmvc_seg_of(const QmvParams& p, int r) {
  return (p.nseg > 2 && r >= p.seg[2].row0) ? 2 : (p.nseg > 1 && r >= p.seg[1].row0) ? 1 : 0;
}
// a field of segment sg (0..2) by selects, so that a per-lane segment does
// not index the kernel-argument struct
#define BMX_SEG_FIELD(p, sg, f) ((sg) == 0 ? (p).seg[0].f : (sg) == 1 ? (p).seg[1].f : (p).seg[2].f)

template <int NI, int EPI, int XU, bool NORM, int NPRE>
__global__ void __launch_bounds__(kQmvcMaxThreads) qmvc_kernel(const QmvParams p, const int S, const int rows_wg) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int NH = (EPI == QMV_SWIGLU) ? 2 : 1;
  const int lshift = __builtin_ctz(S);
  const int SLOTS = 64 >> lshift;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int tid = threadIdx.x;
  const int t256 = tid & (kThreads - 1);  // staging thread as qmv1 numbers it
  const int slot = lane >> lshift;
  const int sl = lane & (S - 1);
  const int K = p.K;
  const int G = K / 64, C = K / 32, W8 = K / 8, GU = G / 8;
  // output rows: all segments in one numbering (SWIGLU: rows of one matrix)
  const int n_rows = (EPI == QMV_SWIGLU) ? p.N : p.seg[p.nseg - 1].row0 + p.seg[p.nseg - 1].rows;
  unsigned char* xs = smem;                                            // [C] x 80 B
  float* sxs = reinterpret_cast<float*>(smem + C * kChunkBytes);       // [C]
  uint32_t* sbs = reinterpret_cast<uint32_t*>(sxs + C);                // [NH][rows_wg][G]
  float* red = reinterpret_cast<float*>(sbs + NH * rows_wg * G);       // [4]
  const int wg_row0 = blockIdx.x * rows_wg;

  // ---- 1. staging loads: x and the norm weight (units as qmv1's 256
  // threads take them; waves past the fourth load copies they do not use),
  // the workgroup's s|b units ----
  uint4 xr[XU], nr[XU];
#pragma unroll
  for (int i = 0; i < XU; i++) {
    const int idx = min(i * kThreads + t256, W8 - 1);
    xr[i] = *reinterpret_cast<const uint4*>(p.x + idx * 8);
    if constexpr (NORM) nr[i] = *reinterpret_cast<const uint4*>(p.norm_w + idx * 8);
  }
  const int sb_units = rows_wg * GU;
  const float rcp_gu = 1.0f / static_cast<float>(GU);
  const int e_sb = min(tid, sb_units - 1);
  const int r_sb = udiv_small(e_sb, rcp_gu);  // row within the workgroup
  const int gr_sb = min(wg_row0 + r_sb, n_rows - 1);
  const int sg_sb = qmvc_seg_of(p, gr_sb);
  uint4 sr[NH], br[NH];
#pragma unroll
  for (int h = 0; h < NH; h++) {
    const int sg = EPI == QMV_SWIGLU ? h : sg_sb;
    const int lr = EPI == QMV_SWIGLU ? gr_sb : gr_sb - BMX_SEG_FIELD(p, sg, row0);
    const int64_t off = static_cast<int64_t>(lr) * G + (e_sb - r_sb * GU) * 8;
    sr[h] = *reinterpret_cast<const uint4*>(BMX_SEG_FIELD(p, sg, s) + off);
    br[h] = *reinterpret_cast<const uint4*>(BMX_SEG_FIELD(p, sg, b) + off);
  }
  // every staging load of the CU is issued before any W load
  __syncthreads();

  // ---- 2. the whole W stream of the lane, chunk by chunk ----
  const int rl = wave * SLOTS + slot;  // row within the workgroup
  const int grow = wg_row0 + rl;
  const bool valid = grow < n_rows;
  const int gr = min(grow, n_rows - 1);
  const int sg_w = EPI == QMV_SWIGLU ? 0 : qmvc_seg_of(p, gr);
  const int lrow = EPI == QMV_SWIGLU ? gr : gr - BMX_SEG_FIELD(p, sg_w, row0);
  const uint32_t* wrow[NH];
#pragma unroll
  for (int h = 0; h < NH; h++) {
    const int sg = EPI == QMV_SWIGLU ? h : sg_w;
    wrow[h] = BMX_SEG_FIELD(p, sg, w) + static_cast<int64_t>(lrow) * (K / 8);
  }
  uint4 wv[NI][NH];
  auto issue_w = [&](int u) {
    const int c = min(sl + (u << lshift), C - 1);
#pragma unroll
    for (int h = 0; h < NH; h++) {
      const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[h] + c * 4));
      wv[u][h] = make_uint4(t.x, t.y, t.z, t.w);
    }
  };
  // the first NPRE chunks now, the rest behind the dot products: a wave with
  // more loads than the CU's load queue takes stalls at issue, which would
  // hold the staging barrier below
#pragma unroll
  for (int u = 0; u < NPRE; u++) issue_w(u);
  __builtin_amdgcn_sched_barrier(0);

  // ---- 3. fused RMSNorm (fast::rms_norm, qwen3.rs:50-55): the sums of
  // squares of the first four waves, as in qmv1 ----
  float inv = 1.0f;
  if constexpr (NORM) {
    if (wave < 4) {
      float ss = 0.0f;
#pragma unroll
      for (int i = 0; i < XU; i++) {
        if (i * kThreads >= W8) break;
        if (i * kThreads + t256 < W8) ss = gemv_ss_unit(xr[i], ss);
      }
      ss = lanes_sum(ss, 64);
      if (lane == 0) red[wave] = ss;
    }
    __syncthreads();
    inv = gemv_norm_inv(red[0], red[1], red[2], red[3], K, p.eps);
  }
  // ---- 4. x (pair-permuted, chunk sums) and s|b into LDS ----
  if (wave < 4) {
#pragma unroll
    for (int i = 0; i < XU; i++) {
      if (i * kThreads >= W8) break;
      const int idx = i * kThreads + t256;
      const bool act = idx < W8;
      uint4 d = xr[i];
      float part = 0.0f;
      if (act) {
        if constexpr (NORM) d = gemv_norm_unit(d, nr[i], inv);
        part = gemv_unit_sum(d);
      }
      part += dpp_f32<0xB1>(part);
      part += dpp_f32<0x4E>(part);
      if (act) {
        *reinterpret_cast<uint4*>(xs + (idx >> 2) * kChunkBytes + (idx & 3) * 16) = permute_pairs(d);
        if ((idx & 3) == 0) sxs[idx >> 2] = part;
      }
    }
  }
  if (tid < sb_units && wg_row0 + r_sb < n_rows) {
#pragma unroll
    for (int h = 0; h < NH; h++) {
      const uint32_t s4[4] = {sr[h].x, sr[h].y, sr[h].z, sr[h].w};
      const uint32_t b4[4] = {br[h].x, br[h].y, br[h].z, br[h].w};
      uint32_t* dst = sbs + (h * rows_wg + r_sb) * G + (e_sb - r_sb * GU) * 8;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        dst[2 * q] = (s4[q] & 0xffffu) | (b4[q] << 16);
        dst[2 * q + 1] = (s4[q] >> 16) | (b4[q] & 0xffff0000u);
      }
    }
  }
  __syncthreads();
  // ---- 5. dot products, chunk by chunk as the W stream arrives; the
  // chunks not yet issued go out one by one behind the products (after
  // chunk u, chunk u + NPRE), so no wave waits at a barrier while its loads
  // queue ----
  const NibbleK nk = nibble_consts();
  float acc[NH];
#pragma unroll
  for (int h = 0; h < NH; h++) acc[h] = 0.0f;
#pragma unroll
  for (int u = 0; u < NI; u++) {
    const int c = sl + (u << lshift);
    if (c < C) {
      float sv[NH], bb[NH];
#pragma unroll
      for (int h = 0; h < NH; h++) gemv_sb(sbs[(h * rows_wg + rl) * G + (c >> 1)], sv[h], bb[h]);
      const uint4* xp = reinterpret_cast<const uint4*>(xs + c * kChunkBytes);
      const uint4 x0 = xp[0], x1 = xp[1], x2 = xp[2], x3 = xp[3];
      const float sx = sxs[c];
#pragma unroll
      for (int h = 0; h < NH; h++) acc[h] = gemv_chunk(wv[u][h], x0, x1, x2, x3, sv[h], bb[h], sx, acc[h], nk);
    }
    if (u + NPRE < NI) issue_w(u + NPRE);
    __builtin_amdgcn_sched_barrier(0);
  }
  // ---- 6. reduce the S lanes of each row, epilogue ----
#pragma unroll
  for (int h = 0; h < NH; h++) acc[h] = lanes_sum(acc[h], S);
  if (sl == 0 && valid) {
    if constexpr (EPI == QMV_STORE)
      BMX_SEG_FIELD(p, sg_w, y)[lrow] = f2bf(acc[0]);  // a lane's segment, by selects
    else
      gemv_store<EPI>(p, 0, 0, p.N, lrow, acc[0], acc[NH - 1]);
  }
}
#undef BMX_SEG_FIELD

template <int NI, int XU, int NPRE>
int launch_qmvc_xu(QmvEpilogue epi, int S, const QmvParams& p, int blocks, int threads, int rows_wg, size_t lds,
                   hipStream_t st) {
  const bool norm = p.norm_w != nullptr;
  auto go = [&](auto kern) {
    if (int rc = allow_lds(kern, lds)) return rc;
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(threads), lds, st, p, S, rows_wg);
    return check_launch("qmvc");
  };
  switch (epi) {
    case QMV_STORE:
      return norm ? go(qmvc_kernel<NI, QMV_STORE, XU, true, NPRE>) : go(qmvc_kernel<NI, QMV_STORE, XU, false, NPRE>);
    case QMV_RESIDUAL:
      return norm ? kNoFit : go(qmvc_kernel<NI, QMV_RESIDUAL, XU, false, NPRE>);
    default:
      return norm ? go(qmvc_kernel<NI, QMV_SWIGLU, XU, true, NPRE>) : kNoFit;
  }
}

// Launches the one-workgroup-per-CU GEMV when it applies: one row of x, no
// argmax partials, K within the single-phase limits, a workgroup of at most
// 16 waves whose s|b units fit one per thread.  kNoFit otherwise.
int try_launch_qmvc(QmvEpilogue epi, int S, const QmvParams& p, hipStream_t st) {
  if (p.m != 1 || p.amax || !p.sb_vec || p.K / 8 > kThreads * kXU1) return kNoFit;
  if (S < kQmvcMinLanes) return kNoFit;
  const int C = p.K / 32, G = p.K / 64;
  const int slots = 64 / S;
  const int n_rows = epi == QMV_SWIGLU ? p.N : p.seg[p.nseg - 1].row0 + p.seg[p.nseg - 1].rows;
  static int cus = 0;
  if (cus == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
  }
  const int per_cu = (n_rows + cus - 1) / cus;
  const int waves = (per_cu + slots - 1) / slots;
  if (waves < 4 || waves > kQmvcMaxThreads / 64) return kNoFit;
  const int rows_wg = waves * slots;
  if (rows_wg * (G / 8) > waves * 64) return kNoFit;
  const int blocks = (n_rows + rows_wg - 1) / rows_wg;
  const int nh = epi == QMV_SWIGLU ? 2 : 1;
  const size_t lds = static_cast<size_t>(C) * (kChunkBytes + 4) + static_cast<size_t>(nh) * rows_wg * G * 4 + 16;
  if (lds > 64 * 1024) return kNoFit;
  const int ni = (C + S - 1) / S;
  const int xu = qmv1_xu(p.K);
  // W chunks issued ahead of the staging (the rest go out behind the
  // products): all of them while the CU's waves have at most kQmvcPreLoads
  // loads in all, else about kQmvcPipeLoads, at least two chunks per lane.
  // Probe timings per launch (eager, weights rotated over 1 GiB), chunks
  // ahead 1 / 2 / 3 / all: gate|up SwiGLU 9728 x 2560 8.63 / 7.79 / 8.64 /
  // 9.71 us; 9728 x 2560 store 6.44 / 5.51 / 5.46 / 5.61; down 2560 x 9728
  // - / 6.34 / 6.07 / 6.11; q|k|v 5.84 / 5.26 / 5.10 (all).
  const int per_lane = waves * nh;
  const int npre = per_lane * ni <= kQmvcPreLoads ? ni : std::min(ni, std::max(2, kQmvcPipeLoads / per_lane));
  auto by_ni = [&](auto xu_c) {
    constexpr int XU = decltype(xu_c)::value;
    if (ni <= 2) return launch_qmvc_xu<2, XU, 2>(epi, S, p, blocks, waves * 64, rows_wg, lds, st);
    if (ni <= 3)
      return npre == 3 ? launch_qmvc_xu<3, XU, 3>(epi, S, p, blocks, waves * 64, rows_wg, lds, st)
                       : launch_qmvc_xu<3, XU, 2>(epi, S, p, blocks, waves * 64, rows_wg, lds, st);
    if (ni <= 5)
      return npre == 5   ? launch_qmvc_xu<5, XU, 5>(epi, S, p, blocks, waves * 64, rows_wg, lds, st)
             : npre >= 3 ? launch_qmvc_xu<5, XU, 3>(epi, S, p, blocks, waves * 64, rows_wg, lds, st)
                         : launch_qmvc_xu<5, XU, 2>(epi, S, p, blocks, waves * 64, rows_wg, lds, st);
    return kNoFit;
  };
  return xu == 2 ? by_ni(std::integral_constant<int, 2>{}) : by_ni(std::integral_constant<int, kXU1>{});
}

// Persistent GEMV for M <= 8 rows of x with the whole K in LDS.  About two
// workgroups per CU stage x once (with the fused RMSNorm for M = 1) and then
// stream their share of row tiles (RB rows each; a tile is what one
// workgroup of qmv1 handles): while a tile's dot products run, the next
// tile's W and s|b are already in flight in a second register buffer.  All
// loads are unconditional (clamped), so every wait is for one specific load.
template <int MT, int NI, int NH>
struct QmvTileRegs {
  uint4 w[NI][NH];
  uint4 s[NH];
  uint4 b[NH];
};

template <int MT, int NI, int EPI>
__global__ void __launch_bounds__(kThreads) qmvp_kernel(const QmvParams p, const int S, const int ntiles) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int NH = (EPI == QMV_SWIGLU) ? 2 : 1;
  constexpr int XU = (MT == 1) ? 5 : 8;  // x units (8 values) per thread per staging batch
  const int lshift = __builtin_ctz(S);
  const int SLOTS = 64 >> lshift;
  const int RB = 4 * SLOTS;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int slot = lane >> lshift;
  const int sl = lane & (S - 1);
  const int rl = wave * SLOTS + slot;
  const int M = p.m;
  const int K = p.K;
  const int G = K / 64, C = K / 32, W8 = K / 8, GU = G / 8;
  unsigned char* xs = smem;                                            // [MT][C] x 80 B
  float* sxs = reinterpret_cast<float*>(smem + MT * C * kChunkBytes);  // [MT][C]
  uint32_t* sbs = reinterpret_cast<uint32_t*>(sxs + MT * C);           // [2][NH][RB][G]
  float* red = reinterpret_cast<float*>(sbs + 2 * NH * RB * G);        // [4][MT]
  float* amv = red + 4 * MT;                                           // [4]
  uint32_t* ami = reinterpret_cast<uint32_t*>(amv + 4);                // [4]
  const bool has_norm = p.norm_w != nullptr;
  const int sb_units = RB * GU;
  const float rcp_gu = 1.0f / static_cast<float>(GU);
  const int e_sb = min(static_cast<int>(threadIdx.x), sb_units - 1);
  const int r_sb = udiv_small(e_sb, rcp_gu);

  auto seg_of = [&](int t) {
    int sg = 0;
    if constexpr (EPI != QMV_SWIGLU) {
      if (p.nseg > 1 && t >= p.seg[1].blk0) sg = 1;
      if (p.nseg > 2 && t >= p.seg[2].blk0) sg = 2;
    }
    return sg;
  };
  // loads of tile t (clamped to the last tile: the prefetch past the end is
  // never consumed): s|b units of the workgroup's rows, then W
  auto issue_tile = [&](int t, QmvTileRegs<MT, NI, NH>& R) {
    t = min(t, ntiles - 1);
    const int sg = seg_of(t);
    const int rows = p.seg[sg].rows;
    const int row0 = (t - p.seg[sg].blk0) * RB;
    const int64_t rs = min(row0 + r_sb, rows - 1);
    const int64_t rr = min(row0 + rl, rows - 1);
#pragma unroll
    for (int h = 0; h < NH; h++) {
      const QmvSegment& sgm = p.seg[EPI == QMV_SWIGLU ? h : sg];
      const int64_t off = rs * G + (e_sb - r_sb * GU) * 8;
      R.s[h] = *reinterpret_cast<const uint4*>(sgm.s + off);
      R.b[h] = *reinterpret_cast<const uint4*>(sgm.b + off);
    }
    const uint32_t* wrow[NH];
#pragma unroll
    for (int h = 0; h < NH; h++) wrow[h] = p.seg[EPI == QMV_SWIGLU ? h : sg].w + rr * (K / 8);
#pragma unroll
    for (int u = 0; u < NI; u++) {
      const int c = min(sl + (u << lshift), C - 1);
#pragma unroll
      for (int h = 0; h < NH; h++) {
        const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[h] + c * 4));
        R.w[u][h] = make_uint4(v.x, v.y, v.z, v.w);
      }
    }
  };

  QmvTileRegs<MT, NI, NH> A, B;
  int t = blockIdx.x;

  // ---- x into LDS once: pair-permuted, chunk sums; RMSNorm fused for M = 1 ----
  // 1 / rms of x row m from the per-wave sums of squares in red [4][MT]
  auto inv_of = [&](int m) { return gemv_norm_inv(red[m], red[MT + m], red[2 * MT + m], red[3 * MT + m], K, p.eps); };
  auto stage_unit = [&](int idx, uint4 d, const uint4& wn, float inv) {
    const bool act = idx < MT * W8;
    float part = 0.0f;
    int m = 0, j = 0;
    if (act) {
      m = (MT == 1) ? 0 : idx / W8;
      j = idx - m * W8;
      if (MT > 1 && has_norm) inv = inv_of(m);
      if (has_norm) d = gemv_norm_unit(d, wn, inv);
      part = gemv_unit_sum(d);
    }
    // a chunk of 32 values = 4 consecutive words = 4 consecutive lanes
    part += dpp_f32<0xB1>(part);
    part += dpp_f32<0x4E>(part);
    if (act) {
      *reinterpret_cast<uint4*>(xs + (m * C + (j >> 2)) * kChunkBytes + (j & 3) * 16) = permute_pairs(d);
      if ((j & 3) == 0) sxs[m * C + (j >> 2)] = part;
    }
  };
  if constexpr (MT == 1) {
    const uint16_t* nw = has_norm ? p.norm_w : p.x;  // a readable address either way
    uint4 xr[XU], nr[XU];
#pragma unroll
    for (int i = 0; i < XU; i++) {
      const int idx = min(i * kThreads + static_cast<int>(threadIdx.x), W8 - 1);
      xr[i] = *reinterpret_cast<const uint4*>(p.x + idx * 8);
      nr[i] = *reinterpret_cast<const uint4*>(nw + idx * 8);
    }
    __builtin_amdgcn_sched_barrier(0);
    issue_tile(t, A);  // the first tile's loads stream in behind x
    __builtin_amdgcn_sched_barrier(0);
    float inv = 1.0f;
    if (has_norm) {
      // fast::rms_norm (qwen3.rs:50-55): h = w * bf16(x * rsqrt(mean(x^2) + eps))
      float ss = 0.0f;
#pragma unroll
      for (int i = 0; i < XU; i++) {
        if (i * kThreads >= W8) break;
        if (i * kThreads + static_cast<int>(threadIdx.x) < W8) ss = gemv_ss_unit(xr[i], ss);
      }
      ss = lanes_sum(ss, 64);
      if (lane == 0) red[wave] = ss;
      __syncthreads();
      inv = inv_of(0);
    }
#pragma unroll
    for (int i = 0; i < XU; i++) {
      if (i * kThreads >= W8) break;
      stage_unit(i * kThreads + static_cast<int>(threadIdx.x), xr[i], nr[i], inv);
    }
  } else {
    if (has_norm) {
      // fast::rms_norm (qwen3.rs:50-55) of each x row: a first pass for the
      // sums of squares (thread t sums units t, t + 256, ... of the row, as
      // for one row), then the staging pass normalises
#pragma unroll
      for (int m = 0; m < MT; m++) {
        float ss = 0.0f;
        if (m < M) {
          for (int j = threadIdx.x; j < W8; j += kThreads)
            ss = gemv_ss_unit(*reinterpret_cast<const uint4*>(p.x + m * p.ldx + j * 8), ss);
        }
        ss = lanes_sum(ss, 64);
        if (lane == 0) red[wave * MT + m] = ss;
      }
      __syncthreads();
    }
    for (int b0 = 0; b0 < MT * W8; b0 += kThreads * XU) {
      uint4 xr[XU], nr[XU];
#pragma unroll
      for (int i = 0; i < XU; i++) {
        const int idx = min(b0 + i * kThreads + static_cast<int>(threadIdx.x), MT * W8 - 1);
        const int m = idx / W8;
        const int j = idx - m * W8;
        xr[i] = *reinterpret_cast<const uint4*>(p.x + min(m, M - 1) * p.ldx + j * 8);
        nr[i] = *reinterpret_cast<const uint4*>((has_norm ? p.norm_w : p.x) + j * 8);
      }
#pragma unroll
      for (int i = 0; i < XU; i++) stage_unit(b0 + i * kThreads + static_cast<int>(threadIdx.x), xr[i], nr[i], 1.0f);
    }
    issue_tile(t, A);
  }
  __syncthreads();

  // ---- one tile: s|b to LDS, prefetch the next tile, dot products, epilogue ----
  // pf: whether a next tile exists (its loads are issued before the dot
  // products of this one); the last tile of the workgroup issues none
  auto step = [&](auto pf, int tt, QmvTileRegs<MT, NI, NH>& cur, QmvTileRegs<MT, NI, NH>& nxt, int par) {
    const int sg = seg_of(tt);
    const int rows = p.seg[sg].rows;
    const int row0 = (tt - p.seg[sg].blk0) * RB;
    uint32_t* sb = sbs + par * NH * RB * G;
    if (static_cast<int>(threadIdx.x) < sb_units && row0 + r_sb < rows) {
#pragma unroll
      for (int h = 0; h < NH; h++) {
        const uint32_t s4[4] = {cur.s[h].x, cur.s[h].y, cur.s[h].z, cur.s[h].w};
        const uint32_t b4[4] = {cur.b[h].x, cur.b[h].y, cur.b[h].z, cur.b[h].w};
        uint32_t* dst = sb + (h * RB + r_sb) * G + (e_sb - r_sb * GU) * 8;
#pragma unroll
        for (int q = 0; q < 4; q++) {
          dst[2 * q] = (s4[q] & 0xffffu) | (b4[q] << 16);
          dst[2 * q + 1] = (s4[q] >> 16) | (b4[q] & 0xffff0000u);
        }
      }
    }
    __syncthreads();
    if constexpr (decltype(pf)::value) issue_tile(tt + static_cast<int>(gridDim.x), nxt);
    __builtin_amdgcn_sched_barrier(0);
    const NibbleK nk = nibble_consts();
    float acc[NH][MT];
#pragma unroll
    for (int h = 0; h < NH; h++)
#pragma unroll
      for (int m = 0; m < MT; m++) acc[h][m] = 0.0f;
#pragma unroll
    for (int u = 0; u < NI; u++) {
      const int c = sl + (u << lshift);
      if (c < C) {
        float sv[NH], bb[NH];
#pragma unroll
        for (int h = 0; h < NH; h++) gemv_sb(sb[(h * RB + rl) * G + (c >> 1)], sv[h], bb[h]);
#pragma unroll
        for (int m = 0; m < MT; m++) {
          if (m >= M) break;
          const uint4* xp = reinterpret_cast<const uint4*>(xs + (m * C + c) * kChunkBytes);
          const uint4 x0 = xp[0], x1 = xp[1], x2 = xp[2], x3 = xp[3];
          const float sx = sxs[m * C + c];
#pragma unroll
          for (int h = 0; h < NH; h++)
            acc[h][m] = gemv_chunk(cur.w[u][h], x0, x1, x2, x3, sv[h], bb[h], sx, acc[h][m], nk);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    const int row = row0 + rl;
    const bool valid = row < rows;
#pragma unroll
    for (int h = 0; h < NH; h++)
#pragma unroll
      for (int m = 0; m < MT; m++) acc[h][m] = lanes_sum(acc[h][m], S);
    if (sl == 0 && valid) {
#pragma unroll
      for (int m = 0; m < MT; m++) {
        if (m >= M) break;
        gemv_store<EPI>(p, sg, m, rows, row, acc[0][m], acc[NH - 1][m]);
      }
    }
    if constexpr (EPI == QMV_STORE && MT == 1) {
      if (p.amax != nullptr) {
        // argmax partial of the tile (first index on ties): across row slots
        // with shuffles, then the 4 waves in LDS
        float bv = valid ? bf2f(f2bf(acc[0][0])) : -INFINITY;
        uint32_t bi = valid ? static_cast<uint32_t>(row) : 0xffffffffu;
        for (int off = S; off < 64; off <<= 1) {
          const float ov = __shfl_xor(bv, off, 64);
          const uint32_t oi = __shfl_xor(bi, off, 64);
          if (ov > bv || (ov == bv && oi < bi)) {
            bv = ov;
            bi = oi;
          }
        }
        if (lane == 0) {
          amv[wave] = bv;
          ami[wave] = bi;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
#pragma unroll
          for (int w = 1; w < 4; w++)
            if (amv[w] > bv || (amv[w] == bv && ami[w] < bi)) {
              bv = amv[w];
              bi = ami[w];
            }
          p.amax[tt] = make_uint2(__float_as_uint(bv), bi);
        }
      }
    }
  };
  using more = std::integral_constant<bool, true>;
  using last = std::integral_constant<bool, false>;
  const int g = static_cast<int>(gridDim.x);
  for (;;) {
    if (t + g >= ntiles) {
      step(last{}, t, A, B, 0);
      break;
    }
    step(more{}, t, A, B, 0);
    t += g;
    if (t + g >= ntiles) {
      step(last{}, t, B, A, 1);
      break;
    }
    step(more{}, t, B, A, 1);
    t += g;
  }
}

template <int MT, int NI>
int launch_qmvp_epi(QmvEpilogue epi, int S, const QmvParams& p, int ntiles, int grid, size_t lds, hipStream_t st) {
  // the vocabulary-sized projections are plain stores (the lm_head)
  if (epi != QMV_STORE) return kNoFit;
  if (int rc = allow_lds(qmvp_kernel<MT, NI, QMV_STORE>, lds)) return rc;
  hipLaunchKernelGGL((qmvp_kernel<MT, NI, QMV_STORE>), dim3(grid), dim3(kThreads), lds, st, p, S, ntiles);
  return check_launch("qmvp");
}

template <int MT>
int launch_qmvp_ni(int ni, int nh, QmvEpilogue epi, int S, const QmvParams& p, int ntiles, int grid, size_t lds,
                   hipStream_t st) {
  if (ni <= 2) return launch_qmvp_epi<MT, 2>(epi, S, p, ntiles, grid, lds, st);
  if (ni <= 3) return launch_qmvp_epi<MT, 3>(epi, S, p, ntiles, grid, lds, st);
  if (ni <= 5) return launch_qmvp_epi<MT, 5>(epi, S, p, ntiles, grid, lds, st);
  if (nh == 1 && ni <= 10) return launch_qmvp_epi<MT, 10>(epi, S, p, ntiles, grid, lds, st);
  return kNoFit;
}

// Launches the persistent GEMV when it applies (whole K in LDS, 16-byte s|b
// staging, the workgroup's s|b in one unit per thread); returns kNoFit
// otherwise.  GEMVs with at least this many weight rows (the vocabulary
// projection) go to the persistent kernel.
constexpr int kPersistentRows = 65536;

int try_launch_qmvp(QmvEpilogue epi, int mt, int S, const QmvParams& p, int ntiles, hipStream_t st) {
  if (!p.sb_vec) return kNoFit;
  if (mt == 1 && p.K / 8 > kThreads * 5) return kNoFit;
  const int C = p.K / 32, G = p.K / 64;
  const int RB = 4 * (64 / S);
  if (RB * (G / 8) > kThreads) return kNoFit;
  const int ni = (C + S - 1) / S;
  const int nh = epi == QMV_SWIGLU ? 2 : 1;
  const size_t lds = static_cast<size_t>(mt) * C * (kChunkBytes + 4) + 2ull * nh * RB * G * 4 +
                     4ull * mt * 4 + 32;
  if (lds > 150 * 1024) return kNoFit;
  int grid = mt == 1 ? 512 : 256;
  grid = std::min(grid, ntiles);
  switch (mt) {
    case 1: return launch_qmvp_ni<1>(ni, nh, epi, S, p, ntiles, grid, lds, st);
    case 2: return launch_qmvp_ni<2>(ni, nh, epi, S, p, ntiles, grid, lds, st);
    case 4: return launch_qmvp_ni<4>(ni, nh, epi, S, p, ntiles, grid, lds, st);
    case 5: return launch_qmvp_ni<5>(ni, nh, epi, S, p, ntiles, grid, lds, st);
    default: return launch_qmvp_ni<8>(ni, nh, epi, S, p, ntiles, grid, lds, st);
  }
}

// W chunks in flight per lane in the phased kernel (its register ring)
constexpr int kRing = 8;

template <int MT>
int launch_epi(QmvEpilogue epi, int S, const QmvParams& p, int blocks, size_t lds, hipStream_t st) {
  auto go = [&](auto kern) {
    if (int rc = allow_lds(kern, lds)) return rc;
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(kThreads), lds, st, p, S);
    return check_launch("qmv");
  };
  switch (epi) {
    case QMV_STORE: return go(qmv_kernel<MT, QMV_STORE, kRing>);
    case QMV_RESIDUAL: return go(qmv_kernel<MT, QMV_RESIDUAL, kRing>);
    default: return go(qmv_kernel<MT, QMV_SWIGLU, kRing>);
  }
}

// Lanes per row: balance lane utilisation (groups per row vs S) against
// the number of waves the launch puts on the 256 CUs.
int pick_lanes_per_row(int N, int K) {
  const int C = K / 32;  // 16-byte chunks per row
  int best = 64;
  double best_score = -1.0;
  for (int S = 8; S <= 64; S *= 2) {
    const int iters = (C + S - 1) / S;
    const double util = static_cast<double>(C) / (static_cast<double>(S) * iters);
    const double waves = static_cast<double>(N) * S / 64.0;
    const double fill = std::min(1.0, waves / 2048.0);
    const double score = util * fill;
    if (score > best_score + 1e-9) {
      best_score = score;
      best = S;
    }
  }
  return best;
}

struct QmvGrid {
  int mt, S, rows_per_block, blocks;
  int blk0[3];
};

// Tile shape and grid of one launch: lanes per row S (a function of N and K
// only, so that every row count shares one chunk -> lane assignment), rows
// per workgroup, and the first workgroup of each segment (segments start on
// workgroup boundaries; SWIGLU's two matrices share every workgroup).
QmvGrid qmv_grid(const QmvParams& p, QmvEpilogue epi) {
  QmvGrid g{};
  g.mt = p.m <= 1 ? 1 : p.m <= 2 ? 2 : p.m <= 4 ? 4 : p.m <= 5 ? 5 : 8;
  g.S = pick_lanes_per_row(p.N, p.K);
  g.rows_per_block = (kThreads / 64) * (64 / g.S);
  if (epi == QMV_SWIGLU) {
    g.blocks = (p.N + g.rows_per_block - 1) / g.rows_per_block;
  } else {
    for (int i = 0; i < p.nseg && i < 3; i++) {
      g.blk0[i] = g.blocks;
      g.blocks += (p.seg[i].rows + g.rows_per_block - 1) / g.rows_per_block;
    }
  }
  return g;
}

}  // namespace

int qmv_blocks(const QmvParams& p, QmvEpilogue epi) { return qmv_grid(p, epi).blocks; }

int launch_qmv(QmvParams p, QmvEpilogue epi, hipStream_t stream) {
  if (p.m < 1 || p.m > 8) return set_error(BMX_E_SHAPE, "qmv: M=%d outside 1..8", p.m);
  if (p.K <= 0 || p.K % 64) return set_error(BMX_E_SHAPE, "qmv: K=%d not a positive multiple of 64", p.K);
  if (p.N <= 0) return set_error(BMX_E_SHAPE, "qmv: N=%d", p.N);
  if (!aligned(p.x, 16) || p.ldx % 8)
    return set_error(BMX_E_ALIGN, "qmv: x must be 16-byte aligned with a row stride multiple of 8");
  if (p.norm_w && !aligned(p.norm_w, 16)) return set_error(BMX_E_ALIGN, "qmv: norm weight not 16-byte aligned");
  for (int i = 0; i < p.nseg; i++) {
    if (!p.seg[i].w || !p.seg[i].s || !p.seg[i].b || !p.seg[i].y)
      return set_error(BMX_E_ARG, "qmv: null pointer in segment %d", i);
    if (!aligned(p.seg[i].w, 16)) return set_error(BMX_E_ALIGN, "qmv: W must be 16-byte aligned");
  }
  if (p.amax && (epi != QMV_STORE || p.nseg != 1))
    return set_error(BMX_E_ARG, "qmv: argmax partials need the store epilogue and one segment");
  const QmvGrid gr = qmv_grid(p, epi);
  const int mt = gr.mt, S = gr.S;
  const int nh = epi == QMV_SWIGLU ? 2 : 1;
  const int rows_per_block = gr.rows_per_block;
  // every segment starts on a workgroup boundary (the kernel reads its
  // segment's fields with scalar loads)
  const int blocks = gr.blocks;
  for (int i = 0; i < p.nseg; i++) p.seg[i].blk0 = gr.blk0[i];
  // 16-byte staging of s/b needs whole 8-group units at 16-byte alignment
  p.sb_vec = (p.K % 512) == 0;
  for (int i = 0; i < p.nseg; i++)
    p.sb_vec = p.sb_vec && aligned(p.seg[i].s, 16) && aligned(p.seg[i].b, 16);
  // The large matrices take the matrix-core GEMV for every row count (a
  // function of the shape only, like every choice below).
  if (qmv_mfma_family(p.N, p.K)) {
    if (p.amax)
      return set_error(BMX_E_ARG, "qmv: no argmax partials from the matrix-core GEMV (%d x %d)", p.N, p.K);
    const int rc = try_launch_qmvx(p, epi, stream);
    if (rc != kNoFit) return rc;
  }
  // Kernel choice: the persistent kernel on vocabulary-sized projections,
  // the single-phase kernel where x and s|b fit it, the phased kernel
  // otherwise.  All three compute every row with the same operations in the
  // same order (bmx_device.h, gemv_*), so which one runs -- and how many
  // rows of x share the launch -- never changes a row's bits.  Argmax
  // partials of several rows come from the phased kernel.
  int rows_total = 0;
  for (int i = 0; i < p.nseg; i++) rows_total += p.seg[i].rows;
  const bool amax_multi = p.amax != nullptr && mt > 1;
  if (rows_total >= kPersistentRows && !amax_multi) {
    const int rc = try_launch_qmvp(epi, mt, S, p, blocks, stream);
    if (rc != kNoFit) return rc;
  }
  if (mt == 1) {
    const int rc = try_launch_qmvc(epi, S, p, stream);
    if (rc != kNoFit) return rc;
  }
  if (!amax_multi) {
    const int rc = try_launch_qmv1(epi, mt, S, p, blocks, stream);
    if (rc != kNoFit) return rc;
  }
  // the phased kernel.  LDS per phase: x chunks (80 B + 4 B sum per 32
  // columns per x row) and the workgroup's s|b words (4 B per 64 columns per
  // weight row).  A phase is a multiple of 32 S columns (whole rounds of the
  // S lanes over the chunks), so the phase split never changes which lane
  // adds which chunk.
  const double per_col = mt * (kChunkBytes + 4) / 32.0 + nh * rows_per_block * 4 / 64.0;
  const int unit = std::max(512, 32 * S);
  int kp = static_cast<int>(kLdsBudget / per_col);
  kp = std::max(unit, (kp / unit) * unit);
  p.kp = std::min(kp, p.K);
  const int CP = p.kp / 32, GP = p.kp / 64;
  const size_t lds = static_cast<size_t>(mt) * CP * (kChunkBytes + 4) +
                     static_cast<size_t>(nh) * rows_per_block * GP * 4 + 4 * static_cast<size_t>(mt) * 4 +
                     (p.amax ? static_cast<size_t>(mt) * rows_per_block * 8 : 0);
  switch (mt) {
    case 1: return launch_epi<1>(epi, S, p, blocks, lds, stream);
    case 2: return launch_epi<2>(epi, S, p, blocks, lds, stream);
    case 4: return launch_epi<4>(epi, S, p, blocks, lds, stream);
    case 5: return launch_epi<5>(epi, S, p, blocks, lds, stream);
    default: return launch_epi<8>(epi, S, p, blocks, lds, stream);
  }
}

}  // namespace bmx
