// qmvx host side: shape selection for the matrix-core GEMV of 1..8 rows of x
// (kernels in qmvx_kernel.h, one translation unit per x-row tile), and the
// reduction of the K-split mode.
//
// Row-count invariance.  Every choice that shapes a row's arithmetic -- K
// chunks, K slices per tile, group pairs per wave, the K split -- is made
// from the matrix shape alone (planned for the largest x-row tile, 8), and
// a row of x always sits in the same row of the MFMA A operand, so a row's
// output bits do not depend on how many rows share the launch: a speculative
// verify row equals the single-token decode of the same position.
#include <stdlib.h>

#include <algorithm>

#include "qmvx_kernel.h"

namespace bmx {

using namespace qmvx;

namespace {

// Workgroups of the split kernel the device holds at once, as planned for
// (one per CU); the chunk count aims at about this many tile-sets per
// staged x chunk.
constexpr int kSplitSlots = 256;
constexpr int kSplitTileSetsPerChunk = 4;
// shapes that split: K of at least 8192 and at least 2^25 weights (measured
// at 5 rows of x: 5120 x 8192 and 5120 x 25600 gain, 2560 x 9728 loses)
constexpr int kSplitMinK = 8192;
constexpr int64_t kSplitMinWeights = 1ll << 25;

// K split over workgroups (qmvx_kernel.h): tile-sets of one 16-row tile
// with 8 K-slices per workgroup; chunks of KC groups (a multiple of 8, 16 to
// kMaxChunkKC), as many as keep each workgroup's x chunk small next to the
// weights it streams.  False when the shape gives fewer than two chunks.
bool split_shape(int total_tiles, int G, Shape* sh) {
  int nkc = std::max(2, (kSplitTileSetsPerChunk * kSplitSlots + total_tiles - 1) / total_tiles);
  int KC = ((G + nkc - 1) / nkc + 7) / 8 * 8;
  KC = std::min(kMaxChunkKC, std::max(16, KC));
  nkc = (G + KC - 1) / KC;
  if (nkc < 2) return false;
  sh->SK = kWaves;
  sh->TB = 1;
  sh->KC = KC;
  sh->nkc = nkc;
  sh->npc = (KC / 2 + kWaves - 1) / kWaves;
  sh->nts = total_tiles;
  return true;
}

size_t shape_lds(int mt, int nh, const Shape& sh) {
  const int RW = 16 * sh.TB;
  return static_cast<size_t>(mt) * (sh.KC * 8 + 1) * 16 + static_cast<size_t>(sh.KC) * 16 * 4 +
         2ull * nh * RW * sb_stride(sh.KC) * 4 + static_cast<size_t>(kWaves) * nh * 4 * 64 * 4 +
         static_cast<size_t>(kWaves + 1) * mt * 4;
}

// y (STORE) or x + y (RESIDUAL) from the fp32 partials of the split kernel,
// part[chunk][m][tile-set row], added in chunk order; one output per thread.
__global__ void __launch_bounds__(256) qmvx_reduce_kernel(const QmvParams p, const int nkc, const int ntr,
                                                          const int residual) {
  const int e = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
  if (e >= p.m * ntr) return;
  const int m = e / ntr, tr = e - m * ntr;
  const int ts = tr >> 4;  // 16-row tile-sets
  int sg = 0;
  if (p.nseg > 1 && ts >= p.seg[1].blk0) sg = 1;
  if (p.nseg > 2 && ts >= p.seg[2].blk0) sg = 2;
  const int row = tr - p.seg[sg].blk0 * 16;
  if (row >= p.seg[sg].rows) return;
  float acc = 0.0f;
  for (int c = 0; c < nkc; c++) acc += p.part[(static_cast<int64_t>(c) * p.m + m) * ntr + tr];
  if (residual) {
    // x = x + o_proj(attn) in bf16 (qwen3.rs:520-521, 541)
    const int64_t o = static_cast<int64_t>(m) * p.N + row;
    p.seg[0].y[o] = f2bf(bf2f(p.res[o]) + round_bf(acc));
  } else {
    p.seg[sg].y[static_cast<int64_t>(m) * p.seg[sg].rows + row] = f2bf(acc);
  }
}

int launch_mt_any(int mt, int mode, QmvEpilogue epi, const QmvParams& p, const Shape& sh, size_t lds,
                  hipStream_t stream) {
  switch (mt) {
    case 1: return launch_m1(mode, epi, p, sh, lds, stream);
    case 2: return launch_m2(mode, epi, p, sh, lds, stream);
    case 4: return launch_m4(mode, epi, p, sh, lds, stream);
    case 5: return launch_m5(mode, epi, p, sh, lds, stream);
    default: return launch_m8(mode, epi, p, sh, lds, stream);
  }
}

// x-row tile every shape decision is planned for
constexpr int kPlanRows = 8;
// the matrix-core GEMV takes matrices with N and K both at least this
constexpr int kMfmaMinDim = 5120;

}  // namespace

bool qmv_mfma_family(int N, int K) { return N >= kMfmaMinDim && K >= kMfmaMinDim && K % 512 == 0; }

size_t qmvx_workspace_floats(int M, int N, int K) {
  if (!qmv_mfma_family(N, K) || K < kSplitMinK || static_cast<int64_t>(N) * K < kSplitMinWeights) return 0;
  Shape sh{};
  if (!split_shape((N + 15) / 16, K / 64, &sh)) return 0;
  return static_cast<size_t>(sh.nkc) * M * sh.nts * 16;
}

int try_launch_qmvx(QmvParams p, QmvEpilogue epi, hipStream_t stream) {
  if (p.m < 1 || p.m > 8 || p.amax) return kNoFit;
  if (p.K % 512 || !p.sb_vec) return kNoFit;  // s|b in 16-byte units of 8 groups
  const int mt = p.m <= 1 ? 1 : p.m <= 2 ? 2 : p.m <= 4 ? 4 : p.m <= 5 ? 5 : 8;
  const int G = p.K / 64;
  const int nh = epi == QMV_SWIGLU ? 2 : 1;

  // ---- K split over workgroups: no fused norm, no SwiGLU, long rows of a
  // large matrix -- below that the x restaging it saves costs less than its
  // reduction launch ----
  if (epi != QMV_SWIGLU && !p.norm_w && p.K >= kSplitMinK &&
      static_cast<int64_t>(p.N) * p.K >= kSplitMinWeights) {
    int tiles = 0;
    for (int i = 0; i < p.nseg; i++) {
      p.seg[i].blk0 = tiles;  // segments start on tile-set boundaries
      tiles += (p.seg[i].rows + 15) / 16;
    }
    Shape sh{};
    if (split_shape(tiles, G, &sh)) {
      const size_t lds = shape_lds(mt, 1, sh);
      const size_t need = static_cast<size_t>(sh.nkc) * p.m * sh.nts * 16;
      if (int rc = split_scratch(need, p.part, p.part_floats, stream, &p.part)) return rc;
      if (int rc = launch_mt_any(mt, kSplit, epi, p, sh, lds, stream)) return rc;
      const int ntr = sh.nts * 16;
      hipLaunchKernelGGL(qmvx_reduce_kernel, dim3((p.m * ntr + 255) / 256), dim3(256), 0, stream, p, sh.nkc, ntr,
                         epi == QMV_RESIDUAL ? 1 : 0);
      return check_launch("qmvx_reduce");
    }
  }

  // chunks of K: one when the x of kPlanRows rows fits the staging
  // registers (kXU units per thread) and spans at most kMaxKC groups; else
  // chunks of at most kMaxChunkKC groups (the next chunk's x is in flight
  // during a step)
  int nkc = 1;
  if (kPlanRows * G * 8 > kXU * kThreads || G > kMaxKC)
    nkc = std::max((kPlanRows * G * 8 + kXU * kThreads - 1) / (kXU * kThreads), (G + kMaxChunkKC - 1) / kMaxChunkKC);
  const int KC = ((G + nkc - 1) / nkc + 7) / 8 * 8;
  nkc = (G + KC - 1) / KC;
  if (nkc > 1 && (p.norm_w || epi == QMV_SWIGLU)) return kNoFit;
  auto tile_sets = [&](int tb) {
    if (epi == QMV_SWIGLU) return (p.N + 16 * tb - 1) / (16 * tb);
    int n = 0;
    for (int i = 0; i < p.nseg; i++) n += (p.seg[i].rows + 16 * tb - 1) / (16 * tb);
    return n;
  };
  // K slices per tile (a power of two): the fewest that keep a wave at or
  // under 16 group pairs per step (8 with two matrices or several chunks:
  // registers), then more while tile-sets are few
  const int np_max = (nh == 2 || nkc > 1) ? 8 : 16;
  int SK = 1;
  while (SK < kWaves && (KC / 2 + SK - 1) / SK > np_max) SK *= 2;
  while (SK < kWaves && tile_sets(kWaves / SK) < 512) SK *= 2;
  Shape sh{};
  sh.SK = SK;
  sh.TB = kWaves / SK;
  sh.KC = KC;
  sh.nkc = nkc;
  sh.npc = (KC / 2 + SK - 1) / SK;
  if (sh.npc > np_max) return kNoFit;
  const int RW = 16 * sh.TB;
  if (nh * RW * (KC / 8) > kThreads) return kNoFit;  // one s|b unit pair per thread
  // tile-sets; segments start on tile-set boundaries
  if (epi == QMV_SWIGLU) {
    sh.nts = tile_sets(sh.TB);
    for (int i = 0; i < p.nseg; i++) p.seg[i].blk0 = 0;
  } else {
    sh.nts = 0;
    for (int i = 0; i < p.nseg; i++) {
      p.seg[i].blk0 = sh.nts;
      sh.nts += (p.seg[i].rows + RW - 1) / RW;
    }
  }
  // (the fit is judged at the planned tile, so it never depends on M)
  if (shape_lds(kPlanRows, nh, sh) > 160 * 1024) return kNoFit;
  return launch_mt_any(mt, nkc > 1 ? kChunked : kOneChunk, epi, p, sh, shape_lds(mt, nh, sh), stream);
}

}  // namespace bmx
