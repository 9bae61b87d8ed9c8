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
// Work decomposition.  A wave owns 64/S output rows; each row is served by
// S lanes that stride over the row's 64-wide groups.  Per group a lane
// issues two 16-byte loads of packed W (64 nibbles) and one bf16 load each
// of s and b.  x is staged once per workgroup in LDS, pair-permuted so that
// the nibble pairs (q_e, q_{e+4}) of a packed word line up with
// (x_e, x_{e+4}):
//   (w & 0x000F000F) | 0x43004300  ==  bf16 pair (128 + q0, 128 + q4)
// which feeds v_dot2c_f32_bf16 directly.  The +128 offset is removed per
// group with the precomputed group sum Sx:
//   sum_k q x = D - 128 Sx,  so  y += s * D + (b - 128 s) * Sx.
// Each x chunk of 64 bytes occupies 80 bytes of LDS so that the 16-byte
// reads of 8 consecutive lanes land in distinct banks.  Lanes of a row are
// reduced with cross-lane xor shuffles.
#include <stdlib.h>

#include <algorithm>

#include "bmx_device.h"

namespace bmx {
namespace {

constexpr int kThreads = 256;
constexpr int kChunkBytes = 80;  // 64 data bytes + 16 pad per 32 x values
constexpr int kLdsBudget = 40 * 1024;

__device__ __forceinline__ uint4 permute_pairs(uint4 d) {
  // bf16 e0..e7 in d.x=(e0,e1) d.y=(e2,e3) d.z=(e4,e5) d.w=(e6,e7)
  // -> (e0,e4) (e1,e5) (e2,e6) (e3,e7)
  uint4 r;
  r.x = (d.x & 0xffffu) | (d.z << 16);
  r.y = (d.x >> 16) | (d.z & 0xffff0000u);
  r.z = (d.y & 0xffffu) | (d.w << 16);
  r.w = (d.y >> 16) | (d.w & 0xffff0000u);
  return r;
}

// Dot of one packed word (8 nibbles) with its permuted x pairs, +128 bias.
__device__ __forceinline__ float word_dot(uint32_t w, uint4 xp, float acc) {
  const uint32_t magic = 0x43004300u;
  acc = dot2_bf16((w & 0x000f000fu) | magic, xp.x, acc);
  acc = dot2_bf16(((w >> 4) & 0x000f000fu) | magic, xp.y, acc);
  acc = dot2_bf16(((w >> 8) & 0x000f000fu) | magic, xp.z, acc);
  acc = dot2_bf16(((w >> 12) & 0x000f000fu) | magic, xp.w, acc);
  return acc;
}

template <int MT, int S, int EPI>
__global__ void __launch_bounds__(kThreads) qmv_kernel(const QmvParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int NH = (EPI == QMV_SWIGLU) ? 2 : 1;  // weight rows per lane
  constexpr int SLOTS = 64 / S;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int slot = lane / S;
  const int sl = lane % S;
  const int M = p.m;
  const int K = p.K;
  const int CP = p.kp / 32;  // x chunks per phase
  const int GP = p.kp / 64;  // groups per phase
  unsigned char* xs = smem;
  float* sxs = reinterpret_cast<float*>(smem + MT * CP * kChunkBytes);
  float* red = sxs + MT * GP;  // [4 waves][MT] for the RMSNorm prologue

  const int row = (blockIdx.x * (kThreads / 64) + wave) * SLOTS + slot;
  const bool valid = row < p.N;
  const int rr = valid ? row : 0;

  const uint32_t* wrow[NH];
  const uint16_t* srow[NH];
  const uint16_t* brow[NH];
  int seg = 0;
  if (EPI == QMV_SWIGLU) {
#pragma unroll
    for (int h = 0; h < NH; h++) {
      wrow[h] = p.seg[h].w + static_cast<int64_t>(rr) * (K / 8);
      srow[h] = p.seg[h].s + static_cast<int64_t>(rr) * (K / 64);
      brow[h] = p.seg[h].b + static_cast<int64_t>(rr) * (K / 64);
    }
  } else {
    if (p.nseg > 1 && rr >= p.seg[1].row0) seg = 1;
    if (p.nseg > 2 && rr >= p.seg[2].row0) seg = 2;
    const int lr = rr - p.seg[seg].row0;
    wrow[0] = p.seg[seg].w + static_cast<int64_t>(lr) * (K / 8);
    srow[0] = p.seg[seg].s + static_cast<int64_t>(lr) * (K / 64);
    brow[0] = p.seg[seg].b + static_cast<int64_t>(lr) * (K / 64);
  }

  // Optional fused RMSNorm of x (fast::rms_norm, qwen3.rs:50-55):
  //   h = w * bf16(x * rsqrt(mean(x^2) + eps))
  float inv[MT];
#pragma unroll
  for (int m = 0; m < MT; m++) inv[m] = 1.0f;
  if (p.norm_w != nullptr) {
    float ss[MT];
#pragma unroll
    for (int m = 0; m < MT; m++) {
      ss[m] = 0.0f;
      if (m < M) {
        const uint16_t* xr = p.x + m * p.ldx;
        for (int k = threadIdx.x * 8; k < K; k += kThreads * 8) {
          uint4 d = *reinterpret_cast<const uint4*>(xr + k);
          uint32_t v[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
          for (int i = 0; i < 4; i++) {
            float lo = bf2f(v[i] & 0xffffu), hi = bf2f(v[i] >> 16);
            ss[m] += lo * lo + hi * hi;
          }
        }
      }
      ss[m] = wave_sum_xor(ss[m], 64);
      if (lane == 0) red[wave * MT + m] = ss[m];
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < MT; m++) {
      float t = red[m] + red[MT + m] + red[2 * MT + m] + red[3 * MT + m];
      inv[m] = 1.0f / sqrtf(t / static_cast<float>(K) + p.eps);
    }
  }

  float acc[NH][MT];
#pragma unroll
  for (int h = 0; h < NH; h++)
#pragma unroll
    for (int m = 0; m < MT; m++) acc[h][m] = 0.0f;

  // Register ring of U groups: loads for the first U groups of a phase are
  // issued before x is staged, so HBM latency overlaps the staging.
  constexpr int U = (NH == 1 && MT == 1) ? 4 : 2;
  uint4 wv[U][NH][2];
  float sv[U][NH], bv[U][NH];
  auto load_group = [&](int u, int gk) {
#pragma unroll
    for (int h = 0; h < NH; h++) {
      const uint4* wp = reinterpret_cast<const uint4*>(wrow[h] + gk * 8);
      wv[u][h][0] = wp[0];
      wv[u][h][1] = wp[1];
      sv[u][h] = bf2f(srow[h][gk]);
      bv[u][h] = bf2f(brow[h][gk]);
    }
  };

  for (int k0 = 0; k0 < K; k0 += p.kp) {
    const int kpp = min(p.kp, K - k0);
    const int words = kpp / 8;  // multiple of 8
    const int total = MT * words;
    const int gpp = kpp / 64;
    const int gbase = k0 / 64;
    const int n_i = sl < gpp ? (gpp - sl + S - 1) / S : 0;  // groups of this lane
#pragma unroll
    for (int u = 0; u < U; u++)
      if (u < n_i) load_group(u, gbase + sl + S * u);
    __syncthreads();  // previous phase finished reading LDS
    // ---- stage x[:, k0:k0+kpp] pair-permuted, plus group sums ----
    for (int base = 0; base < total; base += kThreads) {
      const int idx = base + threadIdx.x;
      const bool act = idx < total;
      const int m = act ? idx / words : 0;
      const int j = act ? idx - m * words : 0;
      uint4 d = make_uint4(0, 0, 0, 0);
      float part = 0.0f;
      if (act && m < M) {
        const int k = k0 + j * 8;
        d = *reinterpret_cast<const uint4*>(p.x + m * p.ldx + k);
        if (p.norm_w != nullptr) {
          uint4 wn = *reinterpret_cast<const uint4*>(p.norm_w + k);
          uint32_t dv[4] = {d.x, d.y, d.z, d.w}, wq[4] = {wn.x, wn.y, wn.z, wn.w};
#pragma unroll
          for (int i = 0; i < 4; i++) {
            float lo = bf2f(wq[i] & 0xffffu) * round_bf(bf2f(dv[i] & 0xffffu) * inv[m]);
            float hi = bf2f(wq[i] >> 16) * round_bf(bf2f(dv[i] >> 16) * inv[m]);
            dv[i] = static_cast<uint32_t>(f2bf(lo)) | (static_cast<uint32_t>(f2bf(hi)) << 16);
          }
          d = make_uint4(dv[0], dv[1], dv[2], dv[3]);
        }
        uint32_t dv[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
        for (int i = 0; i < 4; i++) part += bf2f(dv[i] & 0xffffu) + bf2f(dv[i] >> 16);
      }
      // group of 64 values = 8 consecutive words = 8 consecutive lanes
      part += __shfl_xor(part, 1, 64);
      part += __shfl_xor(part, 2, 64);
      part += __shfl_xor(part, 4, 64);
      if (act) {
        *reinterpret_cast<uint4*>(xs + (m * CP + (j >> 2)) * kChunkBytes + (j & 3) * 16) =
            permute_pairs(d);
        if ((j & 7) == 0) sxs[m * GP + (j >> 3)] = part;
      }
    }
    __syncthreads();

    // ---- stream W over this phase's groups ----
    for (int i0 = 0; i0 < n_i; i0 += U) {
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int i = i0 + u;
        if (i < n_i) {
          const int g = sl + S * i;
          float bb[NH];
#pragma unroll
          for (int h = 0; h < NH; h++) bb[h] = bv[u][h] - 128.0f * sv[u][h];
#pragma unroll
          for (int m = 0; m < MT; m++) {
            if (m < M) {
              const unsigned char* c0 = xs + (m * CP + 2 * g) * kChunkBytes;
              const uint4* x0 = reinterpret_cast<const uint4*>(c0);
              const uint4* x1 = reinterpret_cast<const uint4*>(c0 + kChunkBytes);
              uint4 xv[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
              const float sx = sxs[m * GP + g];
#pragma unroll
              for (int h = 0; h < NH; h++) {
                float d = 0.0f;
                d = word_dot(wv[u][h][0].x, xv[0], d);
                d = word_dot(wv[u][h][0].y, xv[1], d);
                d = word_dot(wv[u][h][0].z, xv[2], d);
                d = word_dot(wv[u][h][0].w, xv[3], d);
                d = word_dot(wv[u][h][1].x, xv[4], d);
                d = word_dot(wv[u][h][1].y, xv[5], d);
                d = word_dot(wv[u][h][1].z, xv[6], d);
                d = word_dot(wv[u][h][1].w, xv[7], d);
                acc[h][m] += sv[u][h] * d;
                acc[h][m] += bb[h] * sx;
              }
            }
          }
          if (i + U < n_i) load_group(u, gbase + g + S * U);
        }
      }
    }
  }

  // ---- reduce the S lanes of each row and write ----
#pragma unroll
  for (int h = 0; h < NH; h++)
#pragma unroll
    for (int m = 0; m < MT; m++) acc[h][m] = wave_sum_xor(acc[h][m], S);

  if (sl == 0 && valid) {
#pragma unroll
    for (int m = 0; m < MT; m++) {
      if (m >= M) break;
      if (EPI == QMV_STORE) {
        const QmvSegment& sg = p.seg[seg];
        sg.y[static_cast<int64_t>(m) * sg.rows + (row - sg.row0)] = f2bf(acc[0][m]);
      } else if (EPI == QMV_RESIDUAL) {
        // x = x + o_proj(attn) in bf16 (qwen3.rs:520-521, 541)
        const int64_t o = static_cast<int64_t>(m) * p.N + row;
        const float r = bf2f(p.res[o]);
        p.seg[0].y[o] = f2bf(r + round_bf(acc[0][m]));
      } else {
        // silu(gate) * up, each MLX op rounding to bf16 (kernels.rs:73-74)
        const float g = round_bf(acc[0][m]);
        const float u = round_bf(acc[1][m]);
        const float sg = round_bf(1.0f / (1.0f + expf(-g)));
        const float a = round_bf(g * sg);
        p.seg[0].y[static_cast<int64_t>(m) * p.N + row] = f2bf(a * u);
      }
    }
  }
}

template <int MT, int EPI>
int launch_s(int S, const QmvParams& p, int blocks, size_t lds, hipStream_t st) {
  if constexpr (MT == 1) {
    if (S == 8) {
      hipLaunchKernelGGL((qmv_kernel<MT, 8, EPI>), dim3(blocks), dim3(kThreads), lds, st, p);
      return check_launch("qmv");
    }
    if (S == 32) {
      hipLaunchKernelGGL((qmv_kernel<MT, 32, EPI>), dim3(blocks), dim3(kThreads), lds, st, p);
      return check_launch("qmv");
    }
  }
  if (S == 16) {
    hipLaunchKernelGGL((qmv_kernel<MT, 16, EPI>), dim3(blocks), dim3(kThreads), lds, st, p);
  } else {
    hipLaunchKernelGGL((qmv_kernel<MT, 64, EPI>), dim3(blocks), dim3(kThreads), lds, st, p);
  }
  return check_launch("qmv");
}

template <int MT>
int launch_epi(QmvEpilogue epi, int S, const QmvParams& p, int blocks, size_t lds,
               hipStream_t st) {
  switch (epi) {
    case QMV_STORE: return launch_s<MT, QMV_STORE>(S, p, blocks, lds, st);
    case QMV_RESIDUAL: return launch_s<MT, QMV_RESIDUAL>(S, p, blocks, lds, st);
    default: return launch_s<MT, QMV_SWIGLU>(S, p, blocks, lds, st);
  }
}

// Lanes per row: balance lane utilisation (groups per row vs S) against
// the number of waves the launch puts on the 256 CUs.
int pick_lanes_per_row(int N, int K) {
  const int G = K / 64;
  int best = 64;
  double best_score = -1.0;
  for (int S = 8; S <= 64; S *= 2) {
    const int iters = (G + S - 1) / S;
    const double util = static_cast<double>(G) / (static_cast<double>(S) * iters);
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

}  // namespace

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
  int mt = p.m <= 1 ? 1 : p.m <= 2 ? 2 : p.m <= 4 ? 4 : p.m <= 5 ? 5 : 8;
  // LDS per phase: MT * kp * (80/32 + 4/64) bytes
  int kp = static_cast<int>(kLdsBudget / (mt * 2.5625));
  kp = std::max(64, (kp / 64) * 64);
  p.kp = std::min(kp, p.K);
  const int CP = p.kp / 32, GP = p.kp / 64;
  const size_t lds = static_cast<size_t>(mt) * CP * kChunkBytes + static_cast<size_t>(mt) * GP * 4 +
                     4 * static_cast<size_t>(mt) * 4;
  int S = (mt == 1) ? pick_lanes_per_row(p.N, p.K) : (p.K / 64 >= 64 ? 64 : 16);
  // Tuning override: BMX_QMV_LANES = lanes per output row (8/16/32/64).
  if (const char* e = getenv("BMX_QMV_LANES")) {
    const int v = atoi(e);
    if (v == 16 || v == 64 || (mt == 1 && (v == 8 || v == 32))) S = v;
  }
  const int rows_per_block = (kThreads / 64) * (64 / S);
  const int blocks = (p.N + rows_per_block - 1) / rows_per_block;
  switch (mt) {
    case 1: return launch_epi<1>(epi, S, p, blocks, lds, stream);
    case 2: return launch_epi<2>(epi, S, p, blocks, lds, stream);
    case 4: return launch_epi<4>(epi, S, p, blocks, lds, stream);
    case 5: return launch_epi<5>(epi, S, p, blocks, lds, stream);
    default: return launch_epi<8>(epi, S, p, blocks, lds, stream);
  }
}

}  // namespace bmx
