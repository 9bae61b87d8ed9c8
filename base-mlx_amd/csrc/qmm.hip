// qmm: MLX-format 4-bit affine quantized GEMM for M > 8 rows of x (prefill,
// long verify), gfx950 bf16 MFMA.
//
// Semantics restated: mlx_rs::ops::quantized_matmul(x, W, s, b,
// transpose=true, 64, 4) (crates/base-mlx-core/src/model/qwen3.rs:30-41) on
// the GEMM path: the weight tile is dequantized to bf16, w = bf16(s q + b)
// (the value mlx_rs::ops::dequantize produces, one rounding), and
//   y[m,n] = sum_k x[m,k] w[n,k]
// runs with fp32 accumulation and a bf16 result.  (The GEMV path, M <= 8,
// keeps the group decomposition s * sum q x + b * sum x instead.)
//
// Workgroup tile: 128 rows of x by 128 rows of W, 4 waves (2 x 2), each
// 64 x 64 = 4 x 4 tiles of v_mfma_f32_16x16x32_bf16, 3 workgroups per CU;
// on large grids 128 x 256 (waves of 64 x 128, 2 workgroups per CU); from
// M = 2048 on, where their grid fills the chip, 256 rows of x on 8 waves,
// one workgroup per CU, with two W tiles so that dequantizing the next
// group's W overlaps the other waves' products.  Per K
// step (one 64-wide group) the workgroup has x (128 x 64 bf16) and the
// dequantized W tile (128 or 256 x 64 bf16: nibble bytes through
// v_cvt_f32_ubyte, one FMA, v_cvt_pk_bf16_f32 per pair) in LDS: x comes
// straight from memory into one of two LDS tiles (global_load_lds_dwordx4)
// a group ahead, W through registers.  When the tile grid is small, K is
// split over workgroups: fp32 partial tiles go to a workspace and a
// reduction kernel writes y.
//
// Epilogues (the prefill's MLX op sequence fused, with the same bf16
// roundings): store; residual, y = res + bf16(x W^T) (qwen3.rs:520-521, 541);
// SwiGLU of the gate and up weights (kernels.rs:73-74): each wave's half of
// the W tile holds gate rows and the up rows of the same output columns, so
// both products of an output end in one lane.
#include <stdlib.h>

#include <algorithm>
#include <map>
#include <mutex>

#include "bmx_device.h"

namespace bmx {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(2))) float f32x2_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

constexpr int QBM = 128, QBN = 128, QT = 256;  // tile rows of x, of W; threads
// LDS tiles: 64 bf16 (128 bytes, 8 chunks of 16 bytes) per row, unpadded;
// chunk c of row r sits at chunk c ^ (r & 7).  The swizzle keeps the MFMA
// operand reads (16 rows x one chunk per ds_read_b128) and both tile stores
// free of bank conflicts on gfx950; the padded strides tried (144 and 160
// bytes) left the operand reads or the W stores 4-8 cycles per instruction
// in conflicts.
constexpr int RS = 64;  // LDS row stride (elements)
// LDS of a workgroup with a BN-row W tile: two x tiles and the W tile
// (48, 52 or 64 KB for BN 128, 160, 256); with 256-row x tiles (one
// workgroup per CU) two W tiles (104 KB for BN 160, 128 KB for BN 256)
constexpr int qmm_wbufs(int qm) { return qm == QBM ? 1 : 2; }
constexpr size_t qmm_lds(int bn, int qm = QBM) {
  return (2ull * qm * RS + 1ull * qmm_wbufs(qm) * bn * RS) * 2;
}
// 256-row W tiles where the grid of them still spans two or more rounds of
// the 512 resident workgroups they allow (2 per CU): at M = 4096 on
// 12288 x 4096 / 9728 x 2560 / 19456 x 2560, 10-17% faster than 128-row
// tiles; on smaller grids tile quantization eats the gain
bool qmm_wide(int M, int cols_wide_n) {
  return static_cast<int64_t>((M + QBM - 1) / QBM) * cols_wide_n >= 1024;
}
// 160-row W tiles (not SwiGLU) where N is a multiple of 160 and they fill
// the 512 resident workgroups they allow (2 per CU) better than 128-row
// tiles fill theirs: N = 2560 at M = 4096 is 640 tiles of 128 (half the
// CUs run 3) or 512 of 160 (every CU runs 2): 289 -> 271 us at K = 9728.
// (With one 160-row tile per CU, M = 2048, the K split of 128-row tiles
// measured faster: 169 against 233 us.)
bool qmm_tile160(int M, int N) {
  if (N % 160) return false;
  const int64_t mt = (M + QBM - 1) / QBM, t128 = mt * ((N + 127) / 128), t160 = mt * (N / 160);
  return t160 > 384 && t160 <= 512 && (t128 + 255) / 256 * 128 > (t160 + 255) / 256 * 160;
}
__device__ __forceinline__ int swz(int row, int chunk) { return row * RS + ((chunk ^ (row & 7)) << 3); }

struct QmmParams {
  const uint16_t* x;   // [M, K]
  const uint32_t* w;   // [N, K/8] (SwiGLU: gate)
  const uint16_t* s;   // [N, K/64]
  const uint16_t* b;   // [N, K/64]
  const uint32_t* w2;  // SwiGLU: up weight, scales and biases
  const uint16_t* s2;
  const uint16_t* b2;
  const uint16_t* res;  // residual: [M, N] (may alias y)
  uint16_t* y;          // [M, N] bf16 (one split)
  float* part;          // [splits, M, N] fp32 partials (several splits)
  int M, N, K;
  int gps;     // groups per split
  int mtiles;  // row tiles of x (the grid's x dimension enumerates mtiles x column tiles)
  int xcd;     // tile order: 0 row-major; XCD-grouped 1 column-major, 2 row-major
  // Store epilogue over up to 3 column segments (q | k | v of one layer in
  // one launch): segment i covers output columns [seg_n0[i], seg_n0[i+1])
  // of the launch (multiples of the tile width) with its own W, s, b and y
  // (y row stride = the segment's width).  nseg = 0: the plain product.
  int nseg;
  int seg_n0[4];
  const uint32_t* seg_w[3];
  const uint16_t* seg_s[3];
  const uint16_t* seg_b[3];
  uint16_t* seg_y[3];
  // Group-major weights (the model's prefill copy): w, w2 and seg_w hold
  // [K/64][N][8] words (each row's 64 nibbles of one group, rows of a group
  // consecutive), and sb, sb2 and seg_sb [K/64][N] words s | b << 16, so a
  // tile's W and s|b of one group are contiguous
  const uint32_t* sb;
  const uint32_t* sb2;
  const uint32_t* seg_sb[3];
  // QMM_QKV_ROPE: where the normed / rotated rows go
  QkvRopeOut rope;
};

// two floats -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}

// BN: W rows per tile, 128 (waves of 64 x 64) or 256 (waves of 64 x 128:
// the x tile serves twice the W rows, for large grids).  GM: weights in the
// group-major layout (QmmParams), else MLX's row-major one.
template <int EPI, int BN, bool GM, int QM = QBM>
__global__ void __launch_bounds__(2 * QM, QM == QBM ? 2 : 1) qmm_kernel(const QmmParams p) {
  static_assert(BN == 128 || BN == 160 || BN == 256, "W tile rows");
  static_assert(QM == QBM || (QM == 2 * QBM && EPI != QMM_QKV_ROPE), "x tile rows");
  constexpr int NWV = QM / 32;  // waves: 2 per 64 x rows
  static_assert(EPI != QMM_SWIGLU || BN % 64 == 0, "SwiGLU pairs gate and up rows per wave");
  constexpr int NJ = BN / 32;                // 16-row W tiles per wave
  constexpr int WR = (BN + QM - 1) / QM;     // W rows staged per thread (the second only below BN)
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);  // [2][QM][RS], swizzled
  uint16_t* ws = xs + 2 * QM * RS;                   // [NWB][BN][RS], swizzled
  constexpr int NWB = qmm_wbufs(QM);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;  // wave sub-tile: x rows 64 wm, W rows BN/2 wn
  const int li = lane & 15, q = lane >> 4;
  const int M = p.M, K = p.K, G = K / 64;
  int N = p.N;
  // output columns per workgroup: BN, or BN / 2 gate / up pairs for SwiGLU
  constexpr int CN = EPI == QMM_SWIGLU ? BN / 2 : BN;
  // Tile of this workgroup.  Row-major (column tiles fastest): the ~768
  // resident workgroups cover a few row tiles and every column tile, so
  // each x row tile and W tile is reused from L2 while resident.  With
  // vocabulary-sized N the resident set is less than one row of tiles and
  // every W tile would come from HBM once per row tile; there workgroups
  // are grouped by XCD instead (the hardware sends workgroup b to XCD
  // b % 8, each XCD with its own L2): XCD k takes one contiguous range of
  // a column-major tile order, so a W tile is fetched into one L2 and
  // reused there by every row tile.
  int mt, nt;
  {
    const int T = gridDim.x;
    if (p.xcd) {
      const int q8 = T >> 3, r8 = T & 7;
      const int k = blockIdx.x & 7, i = blockIdx.x >> 3;
      const int lin = k < r8 ? k * (q8 + 1) + i : r8 * (q8 + 1) + (k - r8) * q8 + i;
      if (p.xcd == 2) {
        const int ntiles = T / p.mtiles;
        mt = lin / ntiles;
        nt = lin - mt * ntiles;
      } else {
        mt = lin % p.mtiles;
        nt = lin / p.mtiles;
      }
    } else {
      const int ntiles = T / p.mtiles;
      mt = blockIdx.x / ntiles;
      nt = blockIdx.x % ntiles;
    }
  }
  const int m0 = mt * QM;
  int n0 = nt * CN;
  const int gb = blockIdx.z * p.gps, ge = min(G, gb + p.gps);
  // the segment holding this workgroup's columns (uniform)
  const uint32_t* pw = p.w;
  const uint16_t *ps = p.s, *pb = p.b;
  const uint32_t* psb = p.sb;
  uint16_t* py = p.y;
  int si = 0;
  if constexpr (EPI == QMM_STORE || EPI == QMM_QKV_ROPE) {
    if (p.nseg > 1) {
      si = (n0 >= p.seg_n0[1]) + (p.nseg > 2 && n0 >= p.seg_n0[2]);
      pw = p.seg_w[si];
      ps = p.seg_s[si];
      pb = p.seg_b[si];
      psb = p.seg_sb[si];
      py = p.seg_y[si];
      n0 -= p.seg_n0[si];
      N = p.seg_n0[si + 1] - p.seg_n0[si];
    }
  }

  // ---- global -> LDS / registers for one group (rows clamped: their
  // results are never stored) ----
  // x straight into LDS (global_load_lds_dwordx4: lane l's 16 bytes land
  // at the instruction's LDS base + 16 l): wave w's instruction i fills
  // tile rows 8 (NWV i + w) .. + 7, lane l row l / 8 and physical chunk
  // l % 8, so it loads logical chunk (l % 8) ^ (row & 7), the swz layout
  const uint16_t* xd[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int row = 8 * (NWV * i + wave) + (lane >> 3), lc = (lane & 7) ^ (row & 7);
    xd[i] = p.x + static_cast<int64_t>(min(m0 + row, M - 1)) * K + lc * 8;
  }
  auto issue_x = [&](int g, uint16_t* xb) {
#pragma unroll
    for (int i = 0; i < 4; i++)
      __builtin_amdgcn_global_load_lds(xd[i] + g * 64, xb + 512 * (NWV * i + wave), 16, 0, 0);
  };
  // W rows wr (and wr + QM with BN above QM) of the tile, half wh of the
  // group; with 512 threads the rows past BN stage nothing
  const int wr = tid >> 1, wh = tid & 1;
  const bool row0 = QM < BN || wr < BN;  // (uniform per wave: BN is a multiple of 32)
  // SwiGLU: each wave's BN / 2 W rows are BN / 4 gate rows and the up rows
  // of the same output columns, so a lane holds both products of its
  // outputs (gate in tiles j < NJ / 2, up in j + NJ / 2)
  // (group-major: W row wrow of group g at (g N + wrow) 8 words, its s|b
  // at g N + wrow, so the tile's rows of one group are consecutive)
  auto wsrc = [&](int row, const uint32_t*& w_, const uint16_t*& s_, const uint16_t*& b_, const uint32_t*& sb_) {
    const int r = row % (BN / 2), col = (row / (BN / 2)) * (BN / 4) + r % (BN / 4);
    const bool up_row = EPI == QMM_SWIGLU && r >= BN / 4;
    const int64_t wrow = min(n0 + (EPI == QMM_SWIGLU ? col : row), N - 1);
    if constexpr (GM) {
      w_ = (up_row ? p.w2 : pw) + wrow * 8 + wh * 4;
      sb_ = (up_row ? p.sb2 : psb) + wrow;
    } else {
      w_ = (up_row ? p.w2 : pw) + wrow * (K / 8) + wh * 4;
      s_ = (up_row ? p.s2 : ps) + wrow * G;
      b_ = (up_row ? p.b2 : pb) + wrow * G;
    }
  };
  const uint32_t *wp0, *wp1 = nullptr;
  const uint16_t *sp0 = nullptr, *bp0 = nullptr, *sp1 = nullptr, *bp1 = nullptr;
  const uint32_t *sbp0 = nullptr, *sbp1 = nullptr;
  wsrc(min(wr, BN - 1), wp0, sp0, bp0, sbp0);
  // (BN 160: the second row exists for wr < 32, i.e. wave 0; uniform per wave)
  const bool row1 = WR == 2 && wr + QM < BN;
  if (row1) wsrc(wr + QM, wp1, sp1, bp1, sbp1);
  // One group's W operands in registers: one or two 16-byte row halves and
  // their scales and biases -- one word s | b << 16 per row in the
  // group-major layout, two 16-bit loads in MLX's.  Raw loaded words only:
  // the split into s and b happens at the store, so no wait for a load
  // comes before its data is needed.  Plain members passed by value, so a
  // set stays in registers.
  struct QStage {
    uint4 w0, w1;
    uint32_t sb0, sb1;
    uint16_t s0, b0, s1, b1;
  };
  auto load = [&](int g) {
    QStage r;
    if (!row0) return r;
    if constexpr (GM) {
      const int64_t go = static_cast<int64_t>(g) * N;
      r.w0 = *reinterpret_cast<const uint4*>(wp0 + go * 8);
      r.sb0 = sbp0[go];
      if (row1) {
        r.w1 = *reinterpret_cast<const uint4*>(wp1 + go * 8);
        r.sb1 = sbp1[go];
      }
    } else {
      r.w0 = *reinterpret_cast<const uint4*>(wp0 + g * 8);
      r.s0 = sp0[g];
      r.b0 = bp0[g];
      if (row1) {
        r.w1 = *reinterpret_cast<const uint4*>(wp1 + g * 8);
        r.s1 = sp1[g];
        r.b1 = bp1[g];
      }
    }
    return r;
  };
  // ---- registers -> LDS: W dequantized to bf16 ----
  auto store = [&](const QStage r, uint16_t* wt) {
    // sv, bv: the row's scale and bias as floats
    auto put_row = [&](int row, const uint4 wq, float sv, float bv) {
      auto put_word = [&](int chunk, uint32_t word) {
        // nibble k of the word is value k: even k in the low nibble of byte
        // k/2, odd k in the high nibble
        uint32_t lo = word & 0x0f0f0f0fu, hi = (word >> 4) & 0x0f0f0f0fu;
        // opaque, so each byte converts with one v_cvt_f32_ubyte<n> instead of
        // a bit-field extract and a convert
        asm volatile("" : "+v"(lo), "+v"(hi));
        uint4 o;
        o.x = pk_bf16(fmaf(sv, static_cast<float>(lo & 0xffu), bv), fmaf(sv, static_cast<float>(hi & 0xffu), bv));
        o.y = pk_bf16(fmaf(sv, static_cast<float>((lo >> 8) & 0xffu), bv),
                      fmaf(sv, static_cast<float>((hi >> 8) & 0xffu), bv));
        o.z = pk_bf16(fmaf(sv, static_cast<float>((lo >> 16) & 0xffu), bv),
                      fmaf(sv, static_cast<float>((hi >> 16) & 0xffu), bv));
        o.w = pk_bf16(fmaf(sv, static_cast<float>(lo >> 24), bv), fmaf(sv, static_cast<float>(hi >> 24), bv));
        *reinterpret_cast<uint4*>(wt + swz(row, chunk)) = o;
      };
      put_word(wh * 4, wq.x);
      put_word(wh * 4 + 1, wq.y);
      put_word(wh * 4 + 2, wq.z);
      put_word(wh * 4 + 3, wq.w);
    };
    if (!row0) return;
    if constexpr (GM) {
      put_row(wr, r.w0, __uint_as_float(r.sb0 << 16), __uint_as_float(r.sb0 & 0xffff0000u));
      if (row1) put_row(wr + QM, r.w1, __uint_as_float(r.sb1 << 16), __uint_as_float(r.sb1 & 0xffff0000u));
    } else {
      put_row(wr, r.w0, bf2f(r.s0), bf2f(r.b0));
      if (row1) put_row(wr + QM, r.w1, bf2f(r.s1), bf2f(r.b1));
    }
  };

  f32x4_t acc[4][NJ];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < NJ; j++) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // ---- the products of one group from LDS ----
  auto compute = [&](const uint16_t* xt, const uint16_t* wt) {
    bf16x8_t af[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int t = 0; t < 2; t++)
        af[i][t] = *reinterpret_cast<const bf16x8_t*>(xt + swz(wm * 64 + i * 16 + li, t * 4 + q));
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      const int c = wn * (BN / 2) + j * 16 + li;
      const bf16x8_t b0 = *reinterpret_cast<const bf16x8_t*>(wt + swz(c, q));
      const bf16x8_t b1 = *reinterpret_cast<const bf16x8_t*>(wt + swz(c, 4 + q));
#pragma unroll
      for (int i = 0; i < 4; i++) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i][0], b0, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i][1], b1, acc[i][j], 0, 0, 0);
      }
    }
  };

  // x of group g + 1 goes straight into the other x tile while group g's
  // products run; W and s|b come through registers, dequantized into the one
  // W tile once every read of the last group's is done.  (Against x staged
  // through registers and two W register sets for 128-row tiles, Qwen3-4B
  // 4096-token prefill: q | k | v 139.5 -> 136.8 us, o / down 174.9 ->
  // 171.4, gate | up 423.0 -> 418.6.)
  // With two W tiles (256-row x tiles) group g + 1's W goes into the tile
  // group g - 1 used, whose reads all ended before the last barrier, so a
  // wave dequantizes while the others' products run and one barrier per
  // group remains.
  issue_x(gb, xs);
  QStage sa = load(gb);
  store(sa, ws);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // x of group gb is in LDS
  __syncthreads();
  for (int g = gb; g < ge; g++) {
    const int cur = (g - gb) & 1;
    const bool more = g + 1 < ge;
    if (more) {
      issue_x(g + 1, xs + (cur ^ 1) * QM * RS);
      sa = load(g + 1);
    }
    compute(xs + cur * QM * RS, ws + (NWB == 2 ? cur * BN * RS : 0));
    if (!more) break;
    if constexpr (NWB == 1) __syncthreads();  // every read of this group's W tile (and x tile) is done
    store(sa, ws + (NWB == 2 ? (cur ^ 1) * BN * RS : 0));
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // x of group g + 1 is in LDS
    __syncthreads();
  }

  // ---- epilogue: lane holds W row 16 j + li, x rows 4 q + r of each tile ----
  if constexpr (EPI == QMM_QKV_ROPE) {
    // The tile is one head (128 columns of the q, k or v segment) of 128
    // tokens.  Its bf16 outputs -- the values the store epilogue writes --
    // go to LDS, then each wave takes 32 tokens and does for each what
    // qk_norm_rope_kv_kernel does for that (token, head): QK-norm and RoPE
    // with the same lane function and the same (cos, sin) (qwen3.rs:392-413),
    // q into q_out [Hq, M, 128], k and v into the caches at row offset + t
    // (qwen3.rs:431-489).
    static_assert(BN == 128, "one head per tile");
    constexpr int TS = 128 + 8;  // LDS row stride (elements)
    uint16_t* tl = xs;           // [QBM][TS]: 34 KB over the x and W tiles (48 KB)
    __syncthreads();             // every wave's last products have read them
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int r = 0; r < 4; r++)
          tl[(wm * 64 + i * 16 + 4 * q + r) * TS + wn * 64 + j * 16 + li] = f2bf(acc[i][j][r]);
    __syncthreads();
    const QkvRopeOut& o = p.rope;
    const int head = n0 / 128;
    const int offset = o.offset_dev ? *o.offset_dev : o.offset;
    const uint16_t* nw = si == 0 ? o.q_norm : o.k_norm;
    const float wa = si < 2 ? bf2f(nw[lane]) : 0.0f, wb = si < 2 ? bf2f(nw[lane + 64]) : 0.0f;
    // every (cos, sin) of the wave's tokens requested before the first is
    // used (the stores below may alias the table as far as the compiler
    // knows, so a load inside the loop would wait behind them)
    constexpr int TW = QBM / 4;  // tokens per wave
    float2 csv[TW];
#pragma unroll
    for (int tt = 0; tt < TW; tt++) {
      const int m = min(m0 + wave * TW + tt, M - 1);
      csv[tt] = si < 2 ? o.cs[static_cast<int64_t>(m) * 64 + lane] : make_float2(0.0f, 0.0f);
    }
#pragma unroll
    for (int tt = 0; tt < TW; tt++) {
      const int t = wave * TW + tt, m = m0 + t;
      if (m >= M) break;  // uniform per wave
      const uint16_t a = tl[t * TS + lane], b = tl[t * TS + lane + 64];
      if (si == 2) {
        uint16_t* dst = o.v_cache + (static_cast<int64_t>(head) * o.cap + offset + m) * 128;
        dst[lane] = a;
        dst[lane + 64] = b;
      } else {
        const float2 cs = csv[tt];
        uint16_t o1, o2;
        qk_norm_rope_lane_cs(bf2f(a), bf2f(b), wa, wb, cs.x, cs.y, o.eps, o1, o2);
        uint16_t* dst = si == 0 ? o.q_out + (static_cast<int64_t>(head) * M + m) * 128
                                : o.k_cache + (static_cast<int64_t>(head) * o.cap + offset + m) * 128;
        dst[lane] = o1;
        dst[lane + 64] = o2;
      }
    }
    return;
  }
  if constexpr (EPI == QMM_SWIGLU) {
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < NJ / 2; j++) {
        const int n = n0 + wn * (BN / 4) + j * 16 + li;
        if (n >= N) continue;
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int m = m0 + wm * 64 + i * 16 + 4 * q + r;
          if (m >= M) continue;
          // silu(gate) * up, each MLX op rounding to bf16 (kernels.rs:73-74)
          const float g = round_bf(acc[i][j][r]);
          const float u = round_bf(acc[i][j + NJ / 2][r]);
          const float sg = round_bf(1.0f / (1.0f + expf(-g)));
          py[static_cast<int64_t>(m) * N + n] = f2bf(round_bf(g * sg) * u);
        }
      }
    return;
  }
  if constexpr (EPI == QMM_RESIDUAL) {
    if (!p.part) {
      // y may be res itself (the in-place residual add), so the compiler
      // keeps each residual load behind the previous output store and the
      // epilogue would wait out one memory round trip per output; each
      // thread reads and writes only its own outputs, so the residuals of
      // a 16-row slice are loaded first, then its outputs stored
#pragma unroll
      for (int i = 0; i < 4; i++) {
        uint16_t rv[NJ][4];
#pragma unroll
        for (int j = 0; j < NJ; j++) {
          const int n = n0 + wn * (BN / 2) + j * 16 + li;
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const int m = m0 + wm * 64 + i * 16 + 4 * q + r;
            rv[j][r] = (n < N && m < M) ? p.res[static_cast<int64_t>(m) * N + n] : 0;
          }
        }
#pragma unroll
        for (int j = 0; j < NJ; j++) {
          const int n = n0 + wn * (BN / 2) + j * 16 + li;
          if (n >= N) continue;
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const int m = m0 + wm * 64 + i * 16 + 4 * q + r;
            if (m >= M) continue;
            py[static_cast<int64_t>(m) * N + n] = f2bf(bf2f(rv[j][r]) + round_bf(acc[i][j][r]));
          }
        }
      }
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      const int n = n0 + wn * (BN / 2) + j * 16 + li;
      if (n >= N) continue;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = m0 + wm * 64 + i * 16 + 4 * q + r;
        if (m >= M) continue;
        const int64_t o = static_cast<int64_t>(m) * N + n;
        if (p.part) {
          p.part[static_cast<int64_t>(blockIdx.z) * M * N + o] = acc[i][j][r];
        } else {
          py[o] = f2bf(acc[i][j][r]);
        }
      }
    }
}

// y = bf16(sum over splits of the fp32 partials) (or res + that, rounded
// as the residual epilogue), 4 outputs per thread
// vec (mn % 4 == 0, part 16-byte and y / res 8-byte aligned): each split's
// four partials in one 16-byte load and the four residuals in one 8-byte
// load ahead of the one 8-byte store (y may be res), summed in the same
// order as the element loop.
__global__ void __launch_bounds__(256) qmm_reduce_kernel(const float* part, const uint16_t* res, uint16_t* y,
                                                         int64_t mn, int splits, int vec) {
  const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i0 >= mn) return;
  if (vec) {
    float t[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s = 0; s < splits; s++) {
      const float4 v = *reinterpret_cast<const float4*>(part + s * mn + i0);
      t[0] += v.x;
      t[1] += v.y;
      t[2] += v.z;
      t[3] += v.w;
    }
    uint16_t o[4];
    if (res) {
      const uint2 r2 = *reinterpret_cast<const uint2*>(res + i0);
      const uint16_t r[4] = {static_cast<uint16_t>(r2.x & 0xffffu), static_cast<uint16_t>(r2.x >> 16),
                             static_cast<uint16_t>(r2.y & 0xffffu), static_cast<uint16_t>(r2.y >> 16)};
#pragma unroll
      for (int e = 0; e < 4; e++) o[e] = f2bf(bf2f(r[e]) + round_bf(t[e]));
    } else {
#pragma unroll
      for (int e = 0; e < 4; e++) o[e] = f2bf(t[e]);
    }
    *reinterpret_cast<uint2*>(y + i0) = make_uint2(o[0] | (static_cast<uint32_t>(o[1]) << 16),
                                                   o[2] | (static_cast<uint32_t>(o[3]) << 16));
    return;
  }
  for (int64_t i = i0; i < min(i0 + 4, mn); i++) {
    float t = 0.0f;
    for (int s = 0; s < splits; s++) t += part[s * mn + i];
    y[i] = res ? f2bf(bf2f(res[i]) + round_bf(t)) : f2bf(t);
  }
}

// Split-K partials (GEMM and matrix-core GEMV) for callers that bring no
// workspace: one device buffer per (device, stream), grown on demand.
// Growing allocates and synchronizes, so a call captured into a graph must
// find the buffer big enough (an earlier uncaptured call of the shape on
// that stream sized it).  Work on one stream runs in order, so its launches
// may share a buffer; work on different streams never shares one.
struct PartBuf {
  float* p = nullptr;
  size_t floats = 0;
};
std::mutex g_part_mu;
std::map<std::pair<int, hipStream_t>, PartBuf> g_parts;

}  // namespace

int stream_scratch(size_t floats, hipStream_t stream, float** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(BMX_E_ARG, "scratch: no current HIP device");
  std::lock_guard<std::mutex> lock(g_part_mu);
  PartBuf& b = g_parts[{dev, stream}];
  if (floats > b.floats) {
    if (b.p) {
      // earlier launches on this stream may still read the old buffer
      if (hipStreamSynchronize(stream) != hipSuccess) return set_error(BMX_E_ALLOC, "scratch: stream sync failed");
      (void)hipFree(b.p);
    }
    b.p = nullptr;
    b.floats = 0;
    if (hipMalloc(&b.p, floats * sizeof(float)) != hipSuccess)
      return set_error(BMX_E_ALLOC, "scratch: no memory for %zu split-K partials", floats);
    b.floats = floats;
  }
  *out = b.p;
  return BMX_OK;
}

namespace {
thread_local int g_no_alloc_depth = 0;
}

NoAllocScope::NoAllocScope() { g_no_alloc_depth++; }
NoAllocScope::~NoAllocScope() { g_no_alloc_depth--; }

int split_scratch(size_t need, float* ws, size_t ws_floats, hipStream_t stream, float** out) {
  if (ws) {
    if (ws_floats < need)
      return set_error(BMX_E_ARG, "workspace of %zu bytes is too small: this shape needs %zu",
                       ws_floats * sizeof(float), need * sizeof(float));
    *out = ws;
    return BMX_OK;
  }
  if (g_no_alloc_depth > 0)
    return set_error(BMX_E_ARG, "this shape needs a workspace of %zu bytes", need * sizeof(float));
  return stream_scratch(need, stream, out);
}

namespace {

// K splits of an M x N x K product: split while the tiles leave most of the
// device idle (splits of at least 8 groups, a multiple of 8 groups each).
// Two refinements measured on the sweep shapes: a grid of 1-1.5 workgroups
// per CU (257-384 tiles) with a long K runs faster in two halves of K
// (M = 2048, N 2560, K 9728: 192 -> 170 us; at K 4096 equal, at K 2560
// slower), and a split small enough to allow 8-group splits
// takes them (M = 128, N 4096, K 2560: 3 splits 28.7 us, 5 splits 23.8 us);
// splits that spill the grid into more rounds measured slower everywhere.
void qmm_split(int M, int N, int K, int* splits_out, int* gps_out, int cols_per_tile = QBN) {
  const int G = K / 64;
  const int tiles = ((N + cols_per_tile - 1) / cols_per_tile) * ((M + QBM - 1) / QBM);
  int splits = 1;
  while (tiles * splits * 2 <= 512 && G / (splits * 2) >= 8) splits *= 2;
  if (splits == 1 && tiles > 256 && tiles <= 384 && G >= 128) splits = 2;
  if (splits > 1 && G / 8 > splits && G / 8 <= 8 && tiles * (G / 8) <= 512) splits = G / 8;
  int gps = (G + splits - 1) / splits;
  if (splits > 1) gps = (gps + 7) / 8 * 8;
  *splits_out = (G + gps - 1) / gps;
  *gps_out = gps;
}

}  // namespace

size_t qmm_need_floats(QmmEpilogue epi, int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 64) return 0;
  int splits, gps;
  qmm_split(M, N, K, &splits, &gps, epi == QMM_SWIGLU ? QBN / 2 : QBN);
  return splits > 1 ? static_cast<size_t>(splits) * M * N : 0;
}

size_t qmm_workspace_floats(int max_M, int N, int K) {
  size_t need = 0;
  // the split count depends on M only through the row-tile count
  for (int t = 1; t <= (max_M + QBM - 1) / QBM; t++) {
    const int M = std::min(t * QBM, max_M);
    int splits, gps;
    qmm_split(M, N, K, &splits, &gps);
    if (splits > 1) need = std::max(need, static_cast<size_t>(splits) * M * N);
  }
  return need;
}

namespace {

template <int EPI, int BN, int QM = QBM>
const void* qmm_kernel_for(bool gm) {
  return gm ? reinterpret_cast<const void*>(qmm_kernel<EPI, BN, true, QM>)
            : reinterpret_cast<const void*>(qmm_kernel<EPI, BN, false, QM>);
}
template <int EPI, int BN>
const void* qmm_kernel_rows(bool gm, int qm) {
  return qm > QBM ? qmm_kernel_for<EPI, BN, 2 * QBM>(gm) : qmm_kernel_for<EPI, BN>(gm);
}

// The GEMM with an epilogue over MLX-layout (sb == nullptr) or group-major
// weights (w, w2 and sb, sb2 in the layout of QmmParams)
int qmm_epi_impl(QmmEpilogue epi, const uint16_t* x, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                 const uint32_t* sb, const uint32_t* w2, const uint16_t* s2, const uint16_t* b2, const uint32_t* sb2,
                 const uint16_t* res, uint16_t* y, int M, int N, int K, float* ws, size_t ws_floats,
                 hipStream_t stream) {
  const bool gm = sb != nullptr;
  if (M <= 0) return BMX_OK;
  if (K % 64 || N <= 0) return set_error(BMX_E_SHAPE, "qmm: N=%d K=%d", N, K);
  if (!aligned(x, 16) || !aligned(w, 16) || (epi == QMM_SWIGLU && !aligned(w2, 16)))
    return set_error(BMX_E_ALIGN, "qmm: x and W must be 16-byte aligned");
  if ((M + QBM - 1) / QBM > 65535 || static_cast<int64_t>((M + QBM - 1) / QBM) * ((N + QBN / 2 - 1) / (QBN / 2)) > INT32_MAX)
    return set_error(BMX_E_SHAPE, "qmm: M=%d N=%d too large", M, N);
  // output columns per workgroup: 128 or 256 (64 or 128 gate / up pairs for
  // SwiGLU)
  const int wide_cols = epi == QMM_SWIGLU ? QBN : 2 * QBN;
  const bool wide = qmm_wide(M, (N + wide_cols - 1) / wide_cols);
  const int bn = wide ? 256 : epi != QMM_SWIGLU && qmm_tile160(M, N) ? 160 : 128;
  const int cols = epi == QMM_SWIGLU ? bn / 2 : bn;
  int splits = 1, gps = K / 64;
  if (bn == 128) qmm_split(M, N, K, &splits, &gps, cols);
  // SwiGLU needs both products of an output in one workgroup: no K split
  if (epi == QMM_SWIGLU && splits > 1) return kNoFit;
  // 256-row x tiles on 8 waves (one workgroup per CU) from M = 2048 on:
  // for 160- and 256-column tiles, and for 128-column tiles where their grid
  // fills its last round of 256 CUs to 90% or more.  Public entry point,
  // MLX layout, against 128-row tiles: 4096 x 12288 x 4096 464 -> 410 us,
  // 4096 x 4096 x 12288 549 -> 474 us, 2048 x 151936 x 4096 3080 -> 2689
  // us; but 2048 x 9728 x 2560 (608 tiles of 256 rows: 79% of the last
  // round) 132 -> 152 us.
  const int64_t t256 = static_cast<int64_t>((M + 2 * QBM - 1) / (2 * QBM)) * ((N + cols - 1) / cols);
  const bool fills = t256 * 10 >= (t256 + 255) / 256 * 256 * 9;
  const int qm = splits == 1 && M >= 2048 && (bn != 128 || fills) ? 2 * QBM : QBM;
  const int mtiles = (M + qm - 1) / qm, ntiles = (N + cols - 1) / cols;
  // Tile order.  Vocabulary-sized N: grouped by XCD in column-major order
  // (151936 x 4096 at M = 2048 runs 1.5x faster; the model's projections
  // ran 4-9% slower so).  The residual GEMMs (o, down: K 4096 / 9728, so a
  // large x) grouped by XCD in row-major order, so each XCD's L2 takes the x
  // rows of its own row tiles and every column tile's W instead of every x
  // row tile and its own W: 207.2 -> 201.3 us per call averaged over o and
  // down in the Qwen3-4B 4096-token prefill (q | k | v and gate | up measured
  // equal or slower that way).
  const int xcd = ntiles > 512 ? 1 : epi == QMM_RESIDUAL ? 2 : 0;
  QmmParams p{x, w, s, b, w2, s2, b2, res, y, nullptr, M, N, K, gps, mtiles, xcd};
  p.sb = sb;
  p.sb2 = sb2;
  if (splits > 1) {
    if (int rc = split_scratch(static_cast<size_t>(splits) * M * N, ws, ws_floats, stream, &p.part)) return rc;
  }
  const dim3 grid(static_cast<unsigned>(mtiles) * ntiles, 1, splits);
  auto launch = [&](const void* kern, int bn) {
    if (int rc = allow_lds_ptr(kern, qmm_lds(bn, qm))) return rc;
    void* args[] = {&p};
    if (int rc = check_hip(hipLaunchKernel(kern, grid, dim3(2 * qm), args, qmm_lds(bn, qm), stream), "qmm launch"))
      return rc;
    return check_launch("qmm");
  };
  const void* kern = bn == 256 ? (epi == QMM_SWIGLU     ? qmm_kernel_rows<QMM_SWIGLU, 256>(gm, qm)
                                  : epi == QMM_RESIDUAL ? qmm_kernel_rows<QMM_RESIDUAL, 256>(gm, qm)
                                                        : qmm_kernel_rows<QMM_STORE, 256>(gm, qm))
                     : bn == 160 ? (epi == QMM_RESIDUAL ? qmm_kernel_rows<QMM_RESIDUAL, 160>(gm, qm)
                                                        : qmm_kernel_rows<QMM_STORE, 160>(gm, qm))
                                 : (epi == QMM_SWIGLU     ? qmm_kernel_rows<QMM_SWIGLU, 128>(gm, qm)
                                    : epi == QMM_RESIDUAL ? qmm_kernel_rows<QMM_RESIDUAL, 128>(gm, qm)
                                                          : qmm_kernel_rows<QMM_STORE, 128>(gm, qm));
  const int rc = launch(kern, bn);
  if (rc) return rc;
  if (splits > 1) {
    const int64_t mn = static_cast<int64_t>(M) * N;
    const uint16_t* r = epi == QMM_RESIDUAL ? res : nullptr;
    const int vec = mn % 4 == 0 && aligned(p.part, 16) && aligned(y, 8) && (r == nullptr || aligned(r, 8));
    hipLaunchKernelGGL(qmm_reduce_kernel, dim3(static_cast<unsigned>((mn + 1023) / 1024)), dim3(256), 0, stream,
                       p.part, r, y, mn, splits, vec);
    return check_launch("qmm_reduce");
  }
  return BMX_OK;
}

// q | k | v (up to 3 column segments) in one launch where every segment is
// whole tiles and K is not split; else kNoFit (gm) or a launch per segment
int qmm_segments_impl(const uint16_t* x, int nseg, const uint32_t* const* w, const uint16_t* const* s,
                      const uint16_t* const* b, const uint32_t* const* sb, uint16_t* const* y, const int* n, int M,
                      int K, float* ws, size_t ws_floats, hipStream_t stream) {
  const bool gm = sb != nullptr;
  if (M <= 0) return BMX_OK;
  if (nseg < 1 || nseg > 3) return set_error(BMX_E_ARG, "qmm: %d segments", nseg);
  int ntot = 0;
  bool one = K % 64 == 0 && aligned(x, 16);
  for (int i = 0; i < nseg; i++) {
    one = one && n[i] > 0 && n[i] % QBN == 0 && aligned(w[i], 16);
    ntot += n[i];
  }
  // 256-column tiles when every segment is whole ones and the grid is large
  bool wide = one && qmm_wide(M, ntot / (2 * QBN));
  for (int i = 0; i < nseg; i++) wide = wide && n[i] % (2 * QBN) == 0;
  int splits = 2, gps = 0;
  if (wide) {
    splits = 1;
    gps = K / 64;
  } else if (one) {
    qmm_split(M, ntot, K, &splits, &gps, QBN);
  }
  // one launch when every segment is whole tiles and K is not split (the
  // reduction writes one y); else a launch per segment
  if (!one || splits > 1 || (M + QBM - 1) / QBM > 65535) {
    if (gm) return kNoFit;
    for (int i = 0; i < nseg; i++)
      if (int rc = launch_qmm(x, w[i], s[i], b[i], y[i], M, n[i], K, ws, ws_floats, stream)) return rc;
    return BMX_OK;
  }
  const int bn = wide ? 2 * QBN : QBN;
  const int mtiles = (M + QBM - 1) / QBM, ntiles = ntot / bn;
  QmmParams p{x, w[0], s[0], b[0], nullptr, nullptr, nullptr, nullptr, y[0], nullptr, M, ntot, K, gps, mtiles, 0};
  p.nseg = nseg;
  int c = 0;
  for (int i = 0; i < nseg; i++) {
    p.seg_n0[i] = c;
    p.seg_w[i] = w[i];
    p.seg_s[i] = s[i];
    p.seg_b[i] = b[i];
    p.seg_sb[i] = gm ? sb[i] : nullptr;
    p.seg_y[i] = y[i];
    c += n[i];
  }
  for (int i = nseg; i < 4; i++) p.seg_n0[i] = c;
  const void* kern = wide ? qmm_kernel_for<QMM_STORE, 256>(gm) : qmm_kernel_for<QMM_STORE, 128>(gm);
  if (int rc = allow_lds_ptr(kern, qmm_lds(bn))) return rc;
  void* args[] = {&p};
  if (int rc = check_hip(hipLaunchKernel(kern, dim3(static_cast<unsigned>(mtiles) * ntiles, 1, 1), dim3(QT), args,
                                         qmm_lds(bn), stream),
                         "qmm launch"))
    return rc;
  return check_launch("qmm");
}

}  // namespace

int launch_qmm_epi(QmmEpilogue epi, const uint16_t* x, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                   const uint32_t* w2, const uint16_t* s2, const uint16_t* b2, const uint16_t* res, uint16_t* y, int M,
                   int N, int K, float* ws, size_t ws_floats, hipStream_t stream) {
  return qmm_epi_impl(epi, x, w, s, b, nullptr, w2, s2, b2, nullptr, res, y, M, N, K, ws, ws_floats, stream);
}

int launch_qmm_epi_gm(QmmEpilogue epi, const uint16_t* x, const uint32_t* w, const uint32_t* sb, const uint32_t* w2,
                      const uint32_t* sb2, const uint16_t* res, uint16_t* y, int M, int N, int K, float* ws,
                      size_t ws_floats, hipStream_t stream) {
  if (!sb || (epi == QMM_SWIGLU && !sb2)) return set_error(BMX_E_ARG, "qmm: group-major s|b missing");
  return qmm_epi_impl(epi, x, w, nullptr, nullptr, sb, w2, nullptr, nullptr, sb2, res, y, M, N, K, ws, ws_floats,
                      stream);
}

int launch_qmm_segments(const uint16_t* x, int nseg, const uint32_t* const* w, const uint16_t* const* s,
                        const uint16_t* const* b, uint16_t* const* y, const int* n, int M, int K, float* ws,
                        size_t ws_floats, hipStream_t stream) {
  return qmm_segments_impl(x, nseg, w, s, b, nullptr, y, n, M, K, ws, ws_floats, stream);
}

int launch_qmm_segments_gm(const uint16_t* x, int nseg, const uint32_t* const* w, const uint32_t* const* sb,
                           uint16_t* const* y, const int* n, int M, int K, float* ws, size_t ws_floats,
                           hipStream_t stream) {
  const uint16_t* none[3] = {nullptr, nullptr, nullptr};
  return qmm_segments_impl(x, nseg, w, none, none, sb, y, n, M, K, ws, ws_floats, stream);
}

int launch_qmm_qkv_rope_gm(const uint16_t* x, const uint32_t* const* w, const uint32_t* const* sb, const int* n,
                           int M, int K, const QkvRopeOut& out, hipStream_t stream) {
  if (M <= 0) return BMX_OK;
  if (!out.offset_dev && (out.offset < 0 || out.offset + M > out.cap))
    return set_error(BMX_E_KV_CAPACITY, "KV cache exhausted: requested %d positions, max %d", out.offset + M, out.cap);
  if (K % 64 || !aligned(x, 16)) return kNoFit;
  int ntot = 0;
  for (int i = 0; i < 3; i++) {
    if (n[i] <= 0 || n[i] % QBN || !aligned(w[i], 16) || !sb[i]) return kNoFit;
    ntot += n[i];
  }
  // the tiling the store form takes: whole 128-column tiles, K not split
  if (qmm_wide(M, ntot / (2 * QBN))) return kNoFit;
  int splits = 1, gps = 0;
  qmm_split(M, ntot, K, &splits, &gps, QBN);
  if (splits > 1 || (M + QBM - 1) / QBM > 65535) return kNoFit;
  const int mtiles = (M + QBM - 1) / QBM, ntiles = ntot / QBN;
  QmmParams p{x, w[0], nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, M, ntot, K, gps,
              mtiles, 0};
  p.nseg = 3;
  int c = 0;
  for (int i = 0; i < 3; i++) {
    p.seg_n0[i] = c;
    p.seg_w[i] = w[i];
    p.seg_sb[i] = sb[i];
    c += n[i];
  }
  p.seg_n0[3] = c;
  p.rope = out;
  const void* kern = reinterpret_cast<const void*>(qmm_kernel<QMM_QKV_ROPE, QBN, true>);
  if (int rc = allow_lds_ptr(kern, qmm_lds(QBN))) return rc;
  void* args[] = {&p};
  if (int rc = check_hip(hipLaunchKernel(kern, dim3(static_cast<unsigned>(mtiles) * ntiles, 1, 1), dim3(QT), args,
                                         qmm_lds(QBN), stream),
                         "qmm launch"))
    return rc;
  return check_launch("qmm_qkv_rope");
}

// The group-major copy of an MLX-layout weight: one thread per (group g,
// row n), i = g N + n, so consecutive threads write consecutive 32-byte rows
__global__ void __launch_bounds__(256) qmm_repack_kernel(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                                                         uint32_t* wt, uint32_t* sbt, int N, int G) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(G) * N) return;
  const int g = static_cast<int>(i / N), n = static_cast<int>(i - static_cast<int64_t>(g) * N);
  const int64_t src = static_cast<int64_t>(n) * G + g;
  const uint4* ws = reinterpret_cast<const uint4*>(w + src * 8);
  uint4* wd = reinterpret_cast<uint4*>(wt + i * 8);
  wd[0] = ws[0];
  wd[1] = ws[1];
  sbt[i] = static_cast<uint32_t>(s[src]) | (static_cast<uint32_t>(b[src]) << 16);
}

int launch_qmm_repack(const uint32_t* w, const uint16_t* s, const uint16_t* b, int N, int K, uint32_t* wt,
                      uint32_t* sbt, hipStream_t stream) {
  if (N <= 0 || K <= 0 || K % 64) return set_error(BMX_E_SHAPE, "qmm repack: N=%d K=%d", N, K);
  if (!aligned(w, 16) || !aligned(wt, 16)) return set_error(BMX_E_ALIGN, "qmm repack: W must be 16-byte aligned");
  const int64_t n = static_cast<int64_t>(K / 64) * N;
  hipLaunchKernelGGL(qmm_repack_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream, w, s, b,
                     wt, sbt, N, K / 64);
  return check_launch("qmm_repack");
}

int launch_qmm(const uint16_t* x, const uint32_t* w, const uint16_t* s, const uint16_t* b, uint16_t* y, int M, int N,
               int K, float* ws, size_t ws_floats, hipStream_t stream) {
  return launch_qmm_epi(QMM_STORE, x, w, s, b, nullptr, nullptr, nullptr, nullptr, y, M, N, K, ws, ws_floats, stream);
}

}  // namespace bmx
