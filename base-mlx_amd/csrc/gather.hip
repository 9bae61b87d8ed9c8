// gather_qmm: routed (MoE expert) 4-bit affine quantized matmul, gfx950.
//
// Semantics restated: mlx_ext::gather_qmm(x, w, scales, biases,
// lhs_indices, rhs_indices, transpose = true, 64, 4, sorted_indices)
// (crates/base-mlx-core/src/mlx_ext.rs:66-117), as QSwitchLinear::forward
// calls it for the experts of SwitchGlu with lhs_indices = None (crates/
// base-mlx-core/src/model/granite.rs:74-88, 181-201): W, s, b stack E
// experts ([E, N, K/8] u32, [E, N, K/64] bf16), and route r -- one (token,
// top-k slot) pair of the index array -- computes
//   y[r] = x[lhs(r)] . W[rhs(r)]^T               ([M, K] x [K, N] -> [M, N])
// with quantized_matmul's group decomposition, fp32 accumulation and a bf16
// result.  lhs(r) = lhs_indices[r] when given, else r / x_bcast: MLX's
// broadcast of x over the top-k axis (top_k for the gate/up projection,
// whose x [T, 1, 1, K] every slot of a token shares; 1 for the down
// projection, which has one input row block per route).  rhs(r) =
// rhs_indices[r] when given, else r.  sorted_indices only tells MLX the
// routes come grouped by expert; results do not depend on it.
//
// Work decomposition: a workgroup of 4 waves owns RB consecutive output
// rows of one route (grid = row tiles x routes); the expert id is read on
// the device, so a captured graph replays with new routes.  The route's x
// rows are staged once in LDS, pair-permuted with per-chunk sums (as the
// GEMV of qmv.hip stages them); each output row is served by S lanes that
// stride over its 64-wide groups (32 bytes of W, one s and one b per group
// and lane), with every W load of a lane issued before the staging.
#include <algorithm>

#include "bmx_device.h"

namespace bmx {
namespace {

constexpr int kGThreads = 256;
constexpr int kGChunk = 80;   // LDS bytes per 32 x values: 64 data + 16 pad
constexpr int kGMaxNG = 8;    // groups per lane
constexpr int kGMaxM = 8;     // rows of x per route

struct GatherParams {
  const uint16_t* x;    // route r: rows [M, K] at x + lhs(r) * x_rstride
  const uint32_t* w;    // [E, N, K/8]
  const uint16_t* s;    // [E, N, K/64]
  const uint16_t* b;    // [E, N, K/64]
  const uint32_t* lhs;  // [R] x block of each route, or null: r / x_bcast
  const uint32_t* rhs;  // [R] expert of each route, or null: r
  uint16_t* y;          // route r: rows [M, N] at y + r * y_rstride
  int64_t x_rstride, y_rstride;
  int x_bcast, nxb, E, M, N, K;  // nxb: x blocks
  int S;                // lanes per output row (power of two, 1..64)
};

template <int MT>
__global__ void __launch_bounds__(kGThreads) gather_qmv_kernel(const GatherParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int K = p.K, G = K / 64, C = K / 32, W8 = K / 8;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lshift = __builtin_ctz(p.S);
  const int slot = lane >> lshift, sl = lane & (p.S - 1);
  const int slots = 64 >> lshift;
  const int rb = 4 * slots;
  const int route = blockIdx.y;
  // out-of-range expert and x block ids are clamped (a valid address for
  // every route)
  const int64_t e = min(p.rhs ? p.rhs[route] : static_cast<uint32_t>(route), static_cast<uint32_t>(p.E - 1));
  const int64_t xb = p.lhs ? min(p.lhs[route], static_cast<uint32_t>(p.nxb - 1)) : route / p.x_bcast;
  const uint16_t* xr = p.x + xb * p.x_rstride;
  const int row = blockIdx.x * rb + wave * slots + slot;
  const int64_t rr = min(row, p.N - 1);
  const uint32_t* wrow = p.w + (e * p.N + rr) * (K / 8);
  const uint16_t* srow = p.s + (e * p.N + rr) * G;
  const uint16_t* brow = p.b + (e * p.N + rr) * G;
  unsigned char* xs = smem;                                           // [MT][C] x kGChunk
  float* sxs = reinterpret_cast<float*>(smem + MT * C * kGChunk);     // [MT][C]

  // ---- W, s, b of this lane's groups g = sl + u * S (clamped, unconditional) ----
  uint4 w0[kGMaxNG], w1[kGMaxNG];
  uint16_t sv[kGMaxNG], bv[kGMaxNG];
#pragma unroll
  for (int u = 0; u < kGMaxNG; u++) {
    const int g = min(sl + (u << lshift), G - 1);
    w0[u] = *reinterpret_cast<const uint4*>(wrow + g * 8);
    w1[u] = *reinterpret_cast<const uint4*>(wrow + g * 8 + 4);
    sv[u] = srow[g];
    bv[u] = brow[g];
  }
  __builtin_amdgcn_sched_barrier(0);
  // ---- x rows into LDS: pair-permuted 16-byte units, per-chunk sums ----
  // (a chunk of 32 values is 4 consecutive units = 4 consecutive lanes)
  const int units = p.M * W8;
  for (int base = 0; base < MT * W8; base += kGThreads) {
    const int idx = base + static_cast<int>(threadIdx.x);
    const bool act = idx < units;
    const int m = act ? idx / W8 : 0;
    const int j = act ? idx - m * W8 : 0;
    uint4 d = make_uint4(0, 0, 0, 0);
    if (act) d = *reinterpret_cast<const uint4*>(xr + static_cast<int64_t>(m) * K + j * 8);
    const uint32_t dv[4] = {d.x, d.y, d.z, d.w};
    float part = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; q++) part += bf2f(dv[q] & 0xffffu) + bf2f(dv[q] >> 16);
    part += dpp_f32<0xB1>(part);
    part += dpp_f32<0x4E>(part);
    if (act) {
      *reinterpret_cast<uint4*>(xs + (m * C + (j >> 2)) * kGChunk + (j & 3) * 16) = permute_pairs(d);
      if ((j & 3) == 0) sxs[m * C + (j >> 2)] = part;
    }
  }
  __syncthreads();
  // ---- dot products: y[m] += s * D + (b - 128 s) * Sx per group ----
  const NibbleK nk = nibble_consts();
  float acc[MT];
#pragma unroll
  for (int m = 0; m < MT; m++) acc[m] = 0.0f;
#pragma unroll
  for (int u = 0; u < kGMaxNG; u++) {
    const int g = sl + (u << lshift);
    if (g < G) {
      const float s = bf2f(sv[u]);
      const float bb = bf2f(bv[u]) - 128.0f * s;
#pragma unroll
      for (int m = 0; m < MT; m++) {
        if (m >= p.M) break;
        const uint4* xp0 = reinterpret_cast<const uint4*>(xs + (m * C + 2 * g) * kGChunk);
        const uint4* xp1 = reinterpret_cast<const uint4*>(xs + (m * C + 2 * g + 1) * kGChunk);
        float d0 = 0.0f, d1 = 0.0f;
        d0 = word_dot(w0[u].x, xp0[0], d0, nk);
        d1 = word_dot(w0[u].y, xp0[1], d1, nk);
        d0 = word_dot(w0[u].z, xp0[2], d0, nk);
        d1 = word_dot(w0[u].w, xp0[3], d1, nk);
        d0 = word_dot(w1[u].x, xp1[0], d0, nk);
        d1 = word_dot(w1[u].y, xp1[1], d1, nk);
        d0 = word_dot(w1[u].z, xp1[2], d0, nk);
        d1 = word_dot(w1[u].w, xp1[3], d1, nk);
        const float sx = sxs[m * C + 2 * g] + sxs[m * C + 2 * g + 1];
        acc[m] += s * (d0 + d1);
        acc[m] += bb * sx;
      }
    }
  }
  // ---- reduce the S lanes of each row, store ----
#pragma unroll
  for (int m = 0; m < MT; m++) acc[m] = wave_sum_xor(acc[m], p.S);
  if (sl == 0 && row < p.N) {
    uint16_t* yr = p.y + static_cast<int64_t>(route) * p.y_rstride + row;
#pragma unroll
    for (int m = 0; m < MT; m++) {
      if (m >= p.M) break;
      yr[static_cast<int64_t>(m) * p.N] = f2bf(acc[m]);
    }
  }
}

}  // namespace

int launch_gather_qmm(const uint16_t* x, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                      const uint32_t* lhs, const uint32_t* rhs, uint16_t* y, int R, int x_bcast, int nxb,
                      int64_t x_rstride, int64_t y_rstride, int E, int M, int N, int K, hipStream_t stream) {
  if (R == 0) return BMX_OK;
  if (R < 0 || R > 65535 || E <= 0 || M <= 0 || N <= 0 || K <= 0 || x_bcast <= 0 || nxb <= 0)
    return set_error(BMX_E_SHAPE, "gather_qmm: bad sizes R=%d E=%d M=%d N=%d K=%d x_bcast=%d x blocks=%d", R, E, M,
                     N, K, x_bcast, nxb);
  if (K % 64) return set_error(BMX_E_SHAPE, "gather_qmm: K=%d not a multiple of the group size 64", K);
  if (M > kGMaxM) return set_error(BMX_E_UNSUPPORTED, "gather_qmm: M=%d rows per route (at most %d)", M, kGMaxM);
  const int G = K / 64;
  // lanes per row: the fewest (a power of two) that keep a lane at or under
  // kGMaxNG groups, then more while the grid is under 512 workgroups and
  // every lane keeps a group
  int S = 1;
  while (S < 64 && (G + S - 1) / S > kGMaxNG) S *= 2;
  if ((G + S - 1) / S > kGMaxNG)
    return set_error(BMX_E_UNSUPPORTED, "gather_qmm: K=%d above %d", K, 64 * 64 * kGMaxNG);
  auto tiles = [&](int s) { return static_cast<int64_t>((N + 4 * (64 / s) - 1) / (4 * (64 / s))) * R; };
  while (S < 64 && 2 * S <= G && tiles(S) < 512) S *= 2;
  const int mt = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
  const size_t lds = static_cast<size_t>(mt) * (K / 32) * (kGChunk + 4);
  if (lds > 160 * 1024) return set_error(BMX_E_UNSUPPORTED, "gather_qmm: M*K=%d too large", M * K);
  const int rb = 4 * (64 / S);
  GatherParams p{x, w, s, b, lhs, rhs, y, x_rstride, y_rstride, x_bcast, nxb, E, M, N, K, S};
  const dim3 grid((N + rb - 1) / rb, R);
  const void* kern = mt == 1   ? reinterpret_cast<const void*>(gather_qmv_kernel<1>)
                     : mt == 2 ? reinterpret_cast<const void*>(gather_qmv_kernel<2>)
                     : mt == 4 ? reinterpret_cast<const void*>(gather_qmv_kernel<4>)
                               : reinterpret_cast<const void*>(gather_qmv_kernel<8>);
  if (lds > 64 * 1024)
    if (int rc = allow_lds_ptr(kern, lds)) return rc;
  switch (mt) {
    case 1: hipLaunchKernelGGL(gather_qmv_kernel<1>, grid, dim3(kGThreads), lds, stream, p); break;
    case 2: hipLaunchKernelGGL(gather_qmv_kernel<2>, grid, dim3(kGThreads), lds, stream, p); break;
    case 4: hipLaunchKernelGGL(gather_qmv_kernel<4>, grid, dim3(kGThreads), lds, stream, p); break;
    default: hipLaunchKernelGGL(gather_qmv_kernel<8>, grid, dim3(kGThreads), lds, stream, p);
  }
  return check_launch("gather_qmm");
}

}  // namespace bmx

using namespace bmx;

extern "C" int bmx_gather_qmm(const bmx_bf16* x, const uint32_t* w, const bmx_bf16* scales, const bmx_bf16* biases,
                              const uint32_t* rhs_indices, bmx_bf16* out, int n_routes, int x_bcast, int n_experts,
                              int M, int N, int K, int group_size, int bits, void* stream) {
  if (!x || !w || !scales || !biases || !out || (!rhs_indices && n_routes > 0))
    return set_error(BMX_E_ARG, "gather_qmm: null pointer");
  if (bits != 4 || group_size != 64)
    return set_error(BMX_E_UNSUPPORTED, "gather_qmm: only bits=4, group_size=64 (got %d, %d)", bits, group_size);
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 15)
    return set_error(BMX_E_ALIGN, "gather_qmm: x and w must be 16-byte aligned");
  const int nxb = x_bcast > 0 ? (n_routes + x_bcast - 1) / x_bcast : 0;  // x blocks the routes read
  return launch_gather_qmm(x, w, scales, biases, nullptr, rhs_indices, out, n_routes, x_bcast, nxb,
                           static_cast<int64_t>(M) * K, static_cast<int64_t>(M) * N, n_experts, M, N, K,
                           as_stream(stream));
}

extern "C" int bmx_gather_qmm_indexed(const bmx_bf16* x, const uint32_t* w, const bmx_bf16* scales,
                                      const bmx_bf16* biases, const uint32_t* lhs_indices,
                                      const uint32_t* rhs_indices, bmx_bf16* out, int n_routes, int n_x_blocks,
                                      int n_experts, int M, int N, int K, int transpose, int group_size, int bits,
                                      int sorted_indices, void* stream) {
  (void)sorted_indices;  // a grouping hint in MLX; the results do not depend on it
  if (!x || !w || !scales || !biases || !out) return set_error(BMX_E_ARG, "gather_qmm: null pointer");
  if (!transpose) return set_error(BMX_E_UNSUPPORTED, "gather_qmm: transpose=false is not supported");
  if (bits != 4 || group_size != 64)
    return set_error(BMX_E_UNSUPPORTED, "gather_qmm: only bits=4, group_size=64 (got %d, %d)", bits, group_size);
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 15)
    return set_error(BMX_E_ALIGN, "gather_qmm: x and w must be 16-byte aligned");
  if (n_x_blocks <= 0 || n_routes < 0) return set_error(BMX_E_SHAPE, "gather_qmm: %d x blocks", n_x_blocks);
  // without lhs_indices the x blocks broadcast evenly over the routes
  if (!lhs_indices && n_routes % n_x_blocks)
    return set_error(BMX_E_SHAPE, "gather_qmm: %d routes over %d x blocks without lhs_indices", n_routes, n_x_blocks);
  // without rhs_indices route r uses expert r
  if (!rhs_indices && n_routes != n_experts)
    return set_error(BMX_E_SHAPE, "gather_qmm: %d routes and %d experts without rhs_indices", n_routes, n_experts);
  const int x_bcast = lhs_indices || n_routes == 0 ? 1 : n_routes / n_x_blocks;
  return launch_gather_qmm(x, w, scales, biases, lhs_indices, rhs_indices, out, n_routes, x_bcast, n_x_blocks,
                           static_cast<int64_t>(M) * K, static_cast<int64_t>(M) * N, n_experts, M, N, K,
                           as_stream(stream));
}
