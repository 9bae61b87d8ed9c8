// qmvx host side: shape selection for the MFMA GEMV of 2..8 rows of x
// (kernels in qmvx_kernel.h, one translation unit per x-row tile).
#include <algorithm>

#include "qmvx_kernel.h"

namespace bmx {

using namespace qmvx;

int try_launch_qmvx(QmvParams p, QmvEpilogue epi, hipStream_t stream) {
  if (p.m < 2 || p.m > 8 || p.amax) return -1;
  if (p.K % 512 || !p.sb_vec) return -1;  // s|b in 16-byte units of 8 groups
  const int mt = p.m <= 2 ? 2 : p.m <= 4 ? 4 : p.m <= 5 ? 5 : 8;
  const int G = p.K / 64;
  const int nh = epi == QMV_SWIGLU ? 2 : 1;
  // chunks of K: one when x fits the staging registers (kXU units per
  // thread) and spans at most kMaxKC groups; else chunks of at most
  // kMaxChunkKC groups (the next chunk's x is in flight during a step)
  int nkc = 1;
  if (mt * G * 8 > kXU * kThreads || G > kMaxKC)
    nkc = std::max((mt * G * 8 + kXU * kThreads - 1) / (kXU * kThreads), (G + kMaxChunkKC - 1) / kMaxChunkKC);
  const int KC = ((G + nkc - 1) / nkc + 7) / 8 * 8;
  nkc = (G + KC - 1) / KC;
  if (nkc > 1 && (p.norm_w || epi == QMV_SWIGLU)) return -1;
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
  if (sh.npc > np_max) return -1;
  const int RW = 16 * sh.TB;
  if (nh * 2 * RW * (KC / 8) > kSBU * kThreads) return -1;
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
  const size_t lds = static_cast<size_t>(mt) * (KC * 8 + 1) * 16 + static_cast<size_t>(KC) * 16 * 4 +
                     2ull * nh * RW * KC * 2 + static_cast<size_t>(kWaves) * nh * 4 * 64 * 4 +
                     static_cast<size_t>(kWaves + 1) * mt * 4;
  if (lds > 160 * 1024) return -1;
  switch (mt) {
    case 2: return launch_m2(nkc > 1, epi, p, sh, lds, stream);
    case 4: return launch_m4(nkc > 1, epi, p, sh, lds, stream);
    case 5: return launch_m5(nkc > 1, epi, p, sh, lds, stream);
    default: return launch_m8(nkc > 1, epi, p, sh, lds, stream);
  }
}

}  // namespace bmx
