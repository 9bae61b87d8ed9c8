#pragma once
// qmvx_kernel.h: MLX-format 4-bit affine quantized matmul for 1..8 rows of x on the
// matrix cores (the large matrices: decode and speculative verify M = 5), gfx950.
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
// products run on v_mfma_f32_16x16x32_bf16 -- for every row count, so that
// one row's arithmetic never depends on how many rows share the launch:
//   A = x (16 rows; rows >= M are never stored): lane l holds x row l%16 and k
//       slice l/16 of the 32-wide step, from LDS;
//   B = W^T: lane l holds W row n = l%16 of a 16-row tile.  W is read 16
//       bytes per lane, a pair of groups per load: lane quarter q = l/16
//       gets words 4q..4q+3 of the pair (64 contiguous bytes per row and
//       load).  One v_permlane32_swap per two registers trades words
//       between the lane halves so that every lane then holds words
//       2 pi(q) + t (t = 0, 1) of both groups, pi = (0, 2, 1, 3); in step t
//       of a group the lane's k slice is that word, unpacked with one mask
//       and one or per bf16 pair
//         (w >> 4j & 0x000F000F) | 0x43004300 == (128 + q_j, 128 + q_{j+4})
//       so x sits in LDS pair-permuted (x_j, x_{j+4});
//   D (per group) -> acc = fma(b - 128 s, Sx, fma(s, D, acc)), Sx the group
//   sum of x (explicit FMAs: the same operations in every instantiation).
// The output tile puts W row l%16 and x rows 4(l/16) + r in lane l.
//
// Work layout.  Weight rows are cut into tiles of 16 and a tile-set is TB
// consecutive tiles; K is cut into NKC chunks of KC groups (one chunk when
// x fits in LDS, which RMSNorm fusion requires).  A step is one (tile-set,
// chunk) pair.  The workgroup (8 waves = TB tiles x SK K-slices) is
// persistent: it walks steps tile-set-major over tile-sets b, b + grid, ...
// x of the current chunk (normalised, pair-permuted, with its group sums)
// and the step's s|b sit in LDS; W sits in registers.  Each step first
// issues the loads of the NEXT step -- s|b and, with several chunks, the
// next x chunk, then W -- and only then computes the current one, so the
// weight stream never stops and every wait is for one specific load.  After
// a tile-set's last chunk the SK partial tiles are added in LDS and the
// store / residual / SwiGLU epilogue runs.
//
// Split mode (long K, no fused norm): restaging x for every step would move
// as many bytes as the weights, so workgroup b instead owns chunk b mod nkc
// only -- its x chunk is staged once -- and walks every (grid / nkc)-th
// tile-set, writing fp32 partial tiles; a second launch adds the nkc
// partials of each output in chunk order and runs the epilogue.
#include <stdlib.h>

#include <algorithm>
#include <type_traits>

#include "bmx_device.h"

namespace bmx {
namespace qmvx {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kXU = 12;      // x units (8 values) per thread per chunk: chunk <= 6144 units (96 KB)
constexpr int kMaxKC = 128;      // groups in a single chunk
constexpr int kMaxChunkKC = 64;  // groups per chunk when K needs several

struct Shape {
  int TB, SK;  // tiles per tile-set, K slices (TB * SK = 8)
  int KC;      // groups per chunk, a multiple of 8
  int nkc;     // chunks
  int npc;     // group pairs per wave per step (<= NP)
  int nts;     // tile-sets
};

// LDS row stride (floats) of the s and b - 128 s tiles of a step, [RW rows]
// [KC groups]: 16-byte aligned rows whose stride in 16-byte units is odd, so
// that the 16 rows of a tile, read at one group, fall in 16 different banks
// (KC = 64 unpadded put all of them in one bank)
__host__ __device__ inline int sb_stride(int KC) { return KC + ((KC / 4) % 2 == 0 ? 4 : 0); }

// Modes: the whole K in one chunk; several chunks walked by each workgroup
// per tile-set (x restaged per step); K split over workgroups, one chunk
// each, fp32 partial tiles reduced by a second launch.
constexpr int kOneChunk = 0, kChunked = 1, kSplit = 2;

// One launcher per x-row tile (1, 2, 4, 5, 8 rows), each in its own
// translation unit (qmvx_m*.hip) so the kernel variants compile in parallel.
int launch_m1(int mode, QmvEpilogue epi, const QmvParams& p, const Shape& sh, size_t lds, hipStream_t st);
int launch_m2(int mode, QmvEpilogue epi, const QmvParams& p, const Shape& sh, size_t lds, hipStream_t st);
int launch_m4(int mode, QmvEpilogue epi, const QmvParams& p, const Shape& sh, size_t lds, hipStream_t st);
int launch_m5(int mode, QmvEpilogue epi, const QmvParams& p, const Shape& sh, size_t lds, hipStream_t st);
int launch_m8(int mode, QmvEpilogue epi, const QmvParams& p, const Shape& sh, size_t lds, hipStream_t st);

#ifdef BMX_QMVX_KERNELS
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// 8 nibbles of a packed word -> bf16 (128 + q), pair-permuted order
// (mask and magic in registers: one v_and_or_b32 per pair, see NibbleK)
__device__ __forceinline__ bf16x8_t nibbles_bf16(uint32_t w, const NibbleK& k) {
  uint4 p;
  p.x = (w & k.mask) | k.magic;
  p.y = ((w >> 4) & k.mask) | k.magic;
  p.z = ((w >> 8) & k.mask) | k.magic;
  p.w = ((w >> 12) & k.mask) | k.magic;
  return __builtin_bit_cast(bf16x8_t, p);
}

template <int NP, int NH>
struct WRegs {
  u32x4 w[NP][NH];
};

// staging registers of a step: the s and the b unit of one row and 8 groups,
// x chunk units and norm weight units
struct SbRegs {
  uint4 v0, v1;
};
struct XRegs {
  uint4 x[kXU];
  uint4 n[kXU];
};

template <int MT, int NP, int EPI, bool CHUNK, bool SPLIT>
__global__ void __launch_bounds__(kThreads) qmvx_kernel(const QmvParams p, const Shape sh) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int NH = (EPI == QMV_SWIGLU) ? 2 : 1;
  const int TB = sh.TB, SK = sh.SK, KC = sh.KC, nkc = sh.nkc, npc = sh.npc;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tile = wave % TB, slice = wave / TB;
  const int n_l = lane & 15, q = lane >> 4;
  const int M = p.m, K = p.K, G = K / 64, W8 = K / 8;
  const int RW = 16 * TB;  // W rows per tile-set
  const int UC = KC * 8;   // x units (8 values) per row of a chunk
  const int XS = UC + 1;   // LDS row stride in units (bank skew)
  uint4* xs = reinterpret_cast<uint4*>(smem);                 // [MT][XS]
  float* sxs = reinterpret_cast<float*>(xs + MT * XS);        // [KC][16]
  const int SBS = sb_stride(KC);
  float* ss = sxs + KC * 16;                                  // [NH][RW][SBS] s
  float* bs = ss + NH * RW * SBS;                             // [NH][RW][SBS] b - 128 s
  float* red = bs + NH * RW * SBS;                            // [kWaves][NH][4][64]
  float* nred = red + kWaves * NH * 4 * 64;                   // [kWaves + 1][MT]: sums of squares, 1 / rms
  const bool has_norm = p.norm_w != nullptr;
  const int grid = static_cast<int>(gridDim.x);
  // SPLIT: workgroup b owns chunk b mod nkc of every nkc-th tile-set (grid
  // is a multiple of nkc) and writes fp32 partial tiles
  const int tstride = SPLIT ? grid / nkc : grid;
  if (static_cast<int>(blockIdx.x) / (SPLIT ? nkc : 1) >= sh.nts) return;

  auto seg_of = [&](int ts) {
    int sg = 0;
    if constexpr (EPI != QMV_SWIGLU) {
      if (p.nseg > 1 && ts >= p.seg[1].blk0) sg = 1;
      if (p.nseg > 2 && ts >= p.seg[2].blk0) sg = 2;
    }
    return sg;
  };

  // ---- s|b of a step: a thread loads the s and the b unit (8 groups) of
  // one (matrix, row, unit) of [NH][RW rows][KC/8 units] and stages s and
  // b - 128 s as fp32, once per row and group instead of once per lane ----
  const int KCU = KC / 8;
  const int sb_total = NH * RW * KCU;  // at most kThreads (checked by the planner)
  int sb_u, sb_r, sb_h;
  {
    const float rcp_kcu = 1.0f / static_cast<float>(KCU), rcp_rw = 1.0f / static_cast<float>(RW);
    const int e = min(static_cast<int>(threadIdx.x), sb_total - 1);
    const int ru = udiv_small(e, rcp_kcu);
    sb_u = e - ru * KCU;
    sb_h = udiv_small(ru, rcp_rw);
    sb_r = ru - sb_h * RW;
  }
  auto issue_sb = [&](int ts, int kc, SbRegs& sbr) {
    const int sg = seg_of(ts);
    const int rows = p.seg[sg].rows;
    const int row0 = (ts - p.seg[sg].blk0) * RW;
    const int g0 = kc * KC;
    const int ku = min(KC, G - g0) / 8;  // units in this chunk
    // plain values, no array: a select between two array slots becomes an
    // indexed scratch load
    const QmvSegment& s0 = p.seg[EPI == QMV_SWIGLU ? 0 : sg];
    const QmvSegment& s1 = p.seg[EPI == QMV_SWIGLU ? 1 : sg];
    const uint16_t* s0s = s0.s;
    const uint16_t* s0b = s0.b;
    const uint16_t* s1s = s1.s;
    const uint16_t* s1b = s1.b;
    const uint16_t* sp = s0s;
    const uint16_t* bp = s0b;
    if constexpr (NH == 2) {
      sp = sb_h ? s1s : s0s;
      bp = sb_h ? s1b : s0b;
    }
    const int64_t off = min(row0 + sb_r, rows - 1) * static_cast<int64_t>(G) + g0 + min(sb_u, ku - 1) * 8;
    sbr.v0 = *reinterpret_cast<const uint4*>(sp + off);
    sbr.v1 = *reinterpret_cast<const uint4*>(bp + off);
  };
  auto store_sb = [&](const SbRegs& sbr) {
    if (static_cast<int>(threadIdx.x) < sb_total) {
      const uint32_t sw[4] = {sbr.v0.x, sbr.v0.y, sbr.v0.z, sbr.v0.w};
      const uint32_t bw[4] = {sbr.v1.x, sbr.v1.y, sbr.v1.z, sbr.v1.w};
      float sf[8], bf[8];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        sf[2 * k] = bf2f(sw[k] & 0xffffu);
        sf[2 * k + 1] = bf2f(sw[k] >> 16);
        bf[2 * k] = __builtin_fmaf(-128.0f, sf[2 * k], bf2f(bw[k] & 0xffffu));
        bf[2 * k + 1] = __builtin_fmaf(-128.0f, sf[2 * k + 1], bf2f(bw[k] >> 16));
      }
      const int o = (sb_h * RW + sb_r) * SBS + sb_u * 8;
      *reinterpret_cast<float4*>(ss + o) = make_float4(sf[0], sf[1], sf[2], sf[3]);
      *reinterpret_cast<float4*>(ss + o + 4) = make_float4(sf[4], sf[5], sf[6], sf[7]);
      *reinterpret_cast<float4*>(bs + o) = make_float4(bf[0], bf[1], bf[2], bf[3]);
      *reinterpret_cast<float4*>(bs + o + 4) = make_float4(bf[4], bf[5], bf[6], bf[7]);
    }
  };

  // ---- W of one step: NP group pairs x NH matrices, 16 bytes per lane each ----
  auto issue_w = [&](int ts, int kc, WRegs<NP, NH>& R) {
    const int sg = seg_of(ts);
    const int rows = p.seg[sg].rows;
    const int row0 = (ts - p.seg[sg].blk0) * RW;
    const int g0 = kc * KC;
    const int kl = min(KC, G - g0);
    const int64_t rr = min(row0 + tile * 16 + n_l, rows - 1);
    const uint32_t* wrow[NH];
#pragma unroll
    for (int h = 0; h < NH; h++) wrow[h] = p.seg[EPI == QMV_SWIGLU ? h : sg].w + rr * W8 + 4 * q;
#pragma unroll
    for (int i = 0; i < NP; i++) {
      const int g = g0 + 2 * min(slice * npc + i, kl / 2 - 1);
#pragma unroll
      for (int h = 0; h < NH; h++)
        R.w[i][h] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[h] + g * 8));
    }
  };

  // ---- x chunk: loads, then (optional RMSNorm) LDS staging with group sums ----
  const float rcp_uc = 1.0f / static_cast<float>(UC);
  const int xu_total = MT * UC;
  auto issue_x = [&](int kc, XRegs& xr, bool with_norm) {
    const int g0 = kc * KC;
    const int ul = min(KC, G - g0) * 8;               // units per row in this chunk
    const uint16_t* nw = with_norm ? p.norm_w : p.x;  // a readable address either way
#pragma unroll
    for (int i = 0; i < kXU; i++) {
      if (i * kThreads >= xu_total) break;
      const int e = min(i * kThreads + static_cast<int>(threadIdx.x), xu_total - 1);
      const int m = udiv_small(e, rcp_uc);
      const int j = min(e - m * UC, ul - 1);
      xr.x[i] = *reinterpret_cast<const uint4*>(p.x + min(m, M - 1) * p.ldx + (g0 * 8 + j) * 8);
      if (with_norm) xr.n[i] = *reinterpret_cast<const uint4*>(nw + (g0 * 8 + j) * 8);
    }
  };
  auto stage_x = [&](const XRegs& xr, bool with_norm) {
#pragma unroll
    for (int i = 0; i < kXU; i++) {
      if (i * kThreads >= xu_total) break;
      const int e = i * kThreads + static_cast<int>(threadIdx.x);
      const bool act = e < xu_total;
      const int m = act ? udiv_small(e, rcp_uc) : 0;
      const int j = e - m * UC;
      uint4 d = xr.x[i];
      if (m >= M) d = make_uint4(0, 0, 0, 0);  // rows beyond M: zeros
      if (with_norm) {
        // fast::rms_norm (qwen3.rs:50-55): h = w * bf16(x * rsqrt(mean(x^2) + eps))
        const float iv = nred[kWaves * MT + m];
        uint32_t dv[4] = {d.x, d.y, d.z, d.w};
        const uint32_t wq[4] = {xr.n[i].x, xr.n[i].y, xr.n[i].z, xr.n[i].w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const float lo = bf2f(wq[k] & 0xffffu) * round_bf(bf2f(dv[k] & 0xffffu) * iv);
          const float hi = bf2f(wq[k] >> 16) * round_bf(bf2f(dv[k] >> 16) * iv);
          dv[k] = static_cast<uint32_t>(f2bf(lo)) | (static_cast<uint32_t>(f2bf(hi)) << 16);
        }
        d = make_uint4(dv[0], dv[1], dv[2], dv[3]);
      }
      float part = 0.0f;
      {
        const uint32_t dv[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
        for (int k = 0; k < 4; k++) part += bf2f(dv[k] & 0xffffu) + bf2f(dv[k] >> 16);
      }
      // a group = 8 consecutive units of one row = 8 consecutive lanes
      part = lanes_sum(part, 8);
      if (act) {
        xs[m * XS + j] = permute_pairs(d);
        if ((j & 7) == 0) sxs[(j >> 3) * 16 + m] = part;
      }
    }
  };

  // ---- prologue: first x chunk, first s|b, first W ----
  for (int e = threadIdx.x; e < KC * (16 - MT); e += kThreads) {
    const int g = e / (16 - MT), m = MT + e % (16 - MT);
    sxs[g * 16 + m] = 0.0f;  // rows MT..15 of the group sums stay zero
  }
  WRegs<NP, NH> A, B;
  int ts = SPLIT ? static_cast<int>(blockIdx.x) / nkc : static_cast<int>(blockIdx.x);
  int kc = SPLIT ? static_cast<int>(blockIdx.x) % nkc : 0;
  {
  XRegs xr;
  SbRegs sbr;
  issue_x(kc, xr, has_norm);
  issue_sb(ts, kc, sbr);
  __builtin_amdgcn_sched_barrier(0);
  issue_w(ts, kc, A);
  __builtin_amdgcn_sched_barrier(0);
  if (has_norm) {
    float sq[MT];
#pragma unroll
    for (int m = 0; m < MT; m++) sq[m] = 0.0f;
#pragma unroll
    for (int i = 0; i < kXU; i++) {
      if (i * kThreads >= xu_total) break;
      const int e = i * kThreads + static_cast<int>(threadIdx.x);
      if (e < xu_total) {
        const int m = udiv_small(e, rcp_uc);
        const uint32_t v[4] = {xr.x[i].x, xr.x[i].y, xr.x[i].z, xr.x[i].w};
        float t = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const float lo = bf2f(v[k] & 0xffffu), hi = bf2f(v[k] >> 16);
          t = __builtin_fmaf(lo, lo, t);
          t = __builtin_fmaf(hi, hi, t);
        }
#pragma unroll
        for (int mm = 0; mm < MT; mm++) sq[mm] += (m == mm) ? t : 0.0f;
      }
    }
#pragma unroll
    for (int m = 0; m < MT; m++) {
      const float v = lanes_sum(sq[m], 64);
      if (lane == 0) nred[wave * MT + m] = v;
    }
    __syncthreads();
    if (threadIdx.x < MT) {
      const int m = threadIdx.x;
      float t = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; w++) t += nred[w * MT + m];
      nred[kWaves * MT + m] = 1.0f / sqrtf(t / static_cast<float>(K) + p.eps);
    }
    __syncthreads();
  }
  stage_x(xr, has_norm);
  store_sb(sbr);
  }
  __syncthreads();

  // ---- steps ----
  f32x4_t acc[NH];
#pragma unroll
  for (int h = 0; h < NH; h++) acc[h] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  // A row l%16 is x row l%16 for l%16 < MT; the lanes of rows MT..15 read
  // row 0 again: each row of the product depends on its own A row only, and
  // rows >= M are never stored, so they need not be zeros
  const int xm = n_l < MT ? n_l : 0;
  const NibbleK nk = nibble_consts();
  const int pq = ((q & 1) << 1) | (q >> 1);  // this lane's word pair in a group after the swap

  // pf: whether a next step exists (its loads are issued before this step's
  // products); the workgroup's last step issues none
  auto step = [&](auto pf, int cts, int ckc, int nts_, int nkc_, WRegs<NP, NH>& cur, WRegs<NP, NH>& nxt) {
    XRegs nx;     // next x chunk (several chunks only)
    SbRegs nsb;  // next s|b
    // The next step's W goes out pair by pair between this step's products
    // (pair i after the products of pair i): a wave that issued them all
    // first stalled ~2 us on the full memory queue before any product.
    const uint32_t* nrow[NH];
    int ng0 = 0, nkl = 2;
    if constexpr (decltype(pf)::value) {
      if constexpr (CHUNK) issue_x(nkc_, nx, false);
      issue_sb(nts_, nkc_, nsb);
      const int sg = seg_of(nts_);
      const int rows = p.seg[sg].rows;
      ng0 = nkc_ * KC;
      nkl = min(KC, G - ng0);
      const int64_t rr = min((nts_ - p.seg[sg].blk0) * RW + tile * 16 + n_l, rows - 1);
#pragma unroll
      for (int h = 0; h < NH; h++) nrow[h] = p.seg[EPI == QMV_SWIGLU ? h : sg].w + rr * W8 + 4 * q;
      __builtin_amdgcn_sched_barrier(0);
    }
    auto issue_next_pair = [&](int i) {
      const int g = ng0 + 2 * min(slice * npc + i, nkl / 2 - 1);
#pragma unroll
      for (int h = 0; h < NH; h++)
        nxt.w[i][h] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(nrow[h] + g * 8));
    };
    const int kl = min(KC, G - ckc * KC);
#pragma unroll
    for (int i = 0; i < NP; i++) {
      const int pl = slice * npc + i;
      if (i < npc && 2 * pl < kl) {
        // lanes q = 0, 1 hold words 0..7 of the first group, q = 2, 3 of the
        // second; swap words 0, 1 of the upper half with 2, 3 of the lower
        uint32_t wv[NH][4];
#pragma unroll
        for (int h = 0; h < NH; h++) {
          const auto s02 = __builtin_amdgcn_permlane32_swap(cur.w[i][h].x, cur.w[i][h].z, false, false);
          const auto s13 = __builtin_amdgcn_permlane32_swap(cur.w[i][h].y, cur.w[i][h].w, false, false);
          wv[h][0] = s02[0];  // first group, word 2 pi(q)
          wv[h][1] = s13[0];  // first group, word 2 pi(q) + 1
          wv[h][2] = s02[1];  // second group, word 2 pi(q)
          wv[h][3] = s13[1];  // second group, word 2 pi(q) + 1
        }
#pragma unroll
        for (int e = 0; e < 2; e++) {
          const int gl = 2 * pl + e;
          const uint4 v0 = xs[xm * XS + gl * 8 + 2 * pq];
          const uint4 v1 = xs[xm * XS + gl * 8 + 2 * pq + 1];
          const bf16x8_t a0 = __builtin_bit_cast(bf16x8_t, v0), a1 = __builtin_bit_cast(bf16x8_t, v1);
          const f32x4_t sx = *reinterpret_cast<const f32x4_t*>(sxs + gl * 16 + 4 * q);
#pragma unroll
          for (int h = 0; h < NH; h++) {
            f32x4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, nibbles_bf16(wv[h][2 * e], nk), d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, nibbles_bf16(wv[h][2 * e + 1], nk), d, 0, 0, 0);
            const int so = (h * RW + tile * 16 + n_l) * SBS + gl;
            const float sv = ss[so];
            const float bb = bs[so];
#pragma unroll
            for (int r = 0; r < 4; r++) {
              acc[h][r] = __builtin_fmaf(sv, d[r], acc[h][r]);
              acc[h][r] = __builtin_fmaf(bb, sx[r], acc[h][r]);
            }
          }
        }
      }
      if constexpr (decltype(pf)::value) issue_next_pair(i);
      __builtin_amdgcn_sched_barrier(0);
    }
    const bool last_chunk = SPLIT || ckc == nkc - 1;
    if (last_chunk && SK > 1) {
#pragma unroll
      for (int h = 0; h < NH; h++)
#pragma unroll
        for (int r = 0; r < 4; r++) red[((wave * NH + h) * 4 + r) * 64 + lane] = acc[h][r];
    }
    __syncthreads();  // (A) this step's LDS reads are done, partials visible
    if (last_chunk) {
      if (slice == 0) {
        for (int s = 1; s < SK; s++) {
          const int w = s * TB + tile;
#pragma unroll
          for (int h = 0; h < NH; h++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[h][r] += red[((w * NH + h) * 4 + r) * 64 + lane];
        }
        const int sg = seg_of(cts);
        const int rows = p.seg[sg].rows;
        const int trow = (cts - p.seg[sg].blk0) * RW + tile * 16 + n_l;
        if constexpr (SPLIT) {
          // fp32 partial of chunk ckc: part[ckc][m][tile-set row]
          const int64_t ntr = static_cast<int64_t>(sh.nts) * RW;
          float* dst = p.part + static_cast<int64_t>(ckc) * M * ntr + cts * RW + tile * 16 + n_l;
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const int m = 4 * q + r;
            if (m >= M) break;
            dst[m * ntr] = acc[0][r];
          }
        } else if (trow < rows) {
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const int m = 4 * q + r;
            if (m >= M) break;
            if constexpr (EPI == QMV_STORE) {
              p.seg[sg].y[static_cast<int64_t>(m) * rows + trow] = f2bf(acc[0][r]);
            } else if constexpr (EPI == QMV_RESIDUAL) {
              // x = x + o_proj(attn) in bf16 (qwen3.rs:520-521, 541)
              const int64_t o = static_cast<int64_t>(m) * p.N + trow;
              p.seg[0].y[o] = f2bf(bf2f(p.res[o]) + round_bf(acc[0][r]));
            } else {
              // silu(gate) * up, each MLX op rounding to bf16 (kernels.rs:73-74)
              const float g = round_bf(acc[0][r]);
              const float u = round_bf(acc[NH - 1][r]);
              const float sgm = round_bf(1.0f / (1.0f + expf(-g)));
              p.seg[0].y[static_cast<int64_t>(m) * p.N + trow] = f2bf(round_bf(g * sgm) * u);
            }
          }
        }
      }
#pragma unroll
      for (int h = 0; h < NH; h++) acc[h] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
    if constexpr (decltype(pf)::value) {
      if constexpr (CHUNK) stage_x(nx, false);
      store_sb(nsb);
      __syncthreads();  // (B) the next step's x / s|b are in place; red is free
    }
  };
  using more = std::integral_constant<bool, true>;
  using last = std::integral_constant<bool, false>;
  // steps of this workgroup: tile-sets blockIdx.x + i * grid, each over nkc chunks
  auto advance = [&](int& t, int& c) {
    if constexpr (SPLIT) {
      t += tstride;
      return;
    }
    if (++c == nkc) {
      c = 0;
      t += grid;
    }
  };
  for (;;) {
    int t2 = ts, c2 = kc;
    advance(t2, c2);
    if (t2 >= sh.nts) {
      step(last{}, ts, kc, t2, c2, A, B);
      break;
    }
    step(more{}, ts, kc, t2, c2, A, B);
    ts = t2;
    kc = c2;
    advance(t2, c2);
    if (t2 >= sh.nts) {
      step(last{}, ts, kc, t2, c2, B, A);
      break;
    }
    step(more{}, ts, kc, t2, c2, B, A);
    ts = t2;
    kc = c2;
  }
}

template <int MT, int NP, bool CHUNK, bool SPLIT>
int launch_epi(QmvEpilogue epi, const QmvParams& p, const Shape& sh, size_t lds, hipStream_t st) {
  const void* k = nullptr;
  switch (epi) {
    case QMV_STORE: k = reinterpret_cast<const void*>(qmvx_kernel<MT, NP, QMV_STORE, CHUNK, SPLIT>); break;
    case QMV_RESIDUAL: k = reinterpret_cast<const void*>(qmvx_kernel<MT, NP, QMV_RESIDUAL, CHUNK, SPLIT>); break;
    default:
      // SwiGLU carries the norm (one chunk) and two matrices (at most 8 pairs)
      if constexpr (CHUNK || SPLIT || NP > 8) return kNoFit;
      else k = reinterpret_cast<const void*>(qmvx_kernel<MT, NP, QMV_SWIGLU, false, false>);
  }
  if (int rc = allow_lds_ptr(k, lds)) return rc;
  const int res = resident_blocks(k, kThreads, lds);
  // SPLIT: a multiple of nkc workgroups (each owns one chunk)
  const int grid = SPLIT ? std::min(sh.nts, std::max(1, res / sh.nkc)) * sh.nkc : std::min(sh.nts, res);
  switch (epi) {
    case QMV_STORE:
      hipLaunchKernelGGL((qmvx_kernel<MT, NP, QMV_STORE, CHUNK, SPLIT>), dim3(grid), dim3(kThreads), lds, st, p, sh);
      break;
    case QMV_RESIDUAL:
      hipLaunchKernelGGL((qmvx_kernel<MT, NP, QMV_RESIDUAL, CHUNK, SPLIT>), dim3(grid), dim3(kThreads), lds, st, p,
                         sh);
      break;
    default:
      if constexpr (!CHUNK && !SPLIT && NP <= 8)
        hipLaunchKernelGGL((qmvx_kernel<MT, NP, QMV_SWIGLU, false, false>), dim3(grid), dim3(kThreads), lds, st, p,
                           sh);
  }
  return check_launch("qmvx");
}

template <int MT>
int launch_mt(int mode, QmvEpilogue epi, const QmvParams& p, const Shape& sh, size_t lds, hipStream_t st) {
  const int n = sh.npc;
  if (mode == kChunked)
    return n <= 4 ? launch_epi<MT, 4, true, false>(epi, p, sh, lds, st) : launch_epi<MT, 8, true, false>(epi, p, sh, lds, st);
  if (mode == kSplit)
    return n <= 4 ? launch_epi<MT, 4, false, true>(epi, p, sh, lds, st) : launch_epi<MT, 8, false, true>(epi, p, sh, lds, st);
  if (epi == QMV_SWIGLU) {
    if (n <= 4) return launch_epi<MT, 4, false, false>(epi, p, sh, lds, st);
    if (n <= 6) return launch_epi<MT, 6, false, false>(epi, p, sh, lds, st);
    return launch_epi<MT, 8, false, false>(epi, p, sh, lds, st);
  }
  if (n <= 4) return launch_epi<MT, 4, false, false>(epi, p, sh, lds, st);
  if (n <= 6) return launch_epi<MT, 6, false, false>(epi, p, sh, lds, st);
  if (n <= 8) return launch_epi<MT, 8, false, false>(epi, p, sh, lds, st);
  if (n <= 12) return launch_epi<MT, 12, false, false>(epi, p, sh, lds, st);
  return launch_epi<MT, 16, false, false>(epi, p, sh, lds, st);
}

}  // namespace
#endif  // BMX_QMVX_KERNELS

}  // namespace qmvx
}  // namespace bmx
