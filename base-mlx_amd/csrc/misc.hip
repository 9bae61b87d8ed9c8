// Greedy argmax and the elementwise ops of a Qwen3 block (gfx950).
//
// Semantics restated:
//   argmax / argmax_axis over the last axis (engine.rs:195-202,
//     speculative.rs:168-173, 289-293): index of the largest value, the
//     first such index on ties, as uint32;
//   mlp_block activation silu(g) * up (model/kernels.rs:73-74): each MLX op
//     rounds to bf16 -- sigmoid, g * sigmoid, then * up;
//   residual add `&x + &y` in bf16 (qwen3.rs:521, 541).
#include <math.h>

#include "bmx_device.h"

namespace bmx {
namespace {

constexpr int kArgThreads = 1024;

__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi) {
  return v > bv || (v == bv && i < bi);
}

// (value, index) reduction across a workgroup of kArgThreads; the result is
// valid in thread 0.
__device__ __forceinline__ void block_best(float& bv, uint32_t& bi) {
  __shared__ float sv[kArgThreads / 64];
  __shared__ uint32_t si[kArgThreads / 64];
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const uint32_t oi = __shfl_xor(bi, off, 64);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kArgThreads / 64; w++)
      if (better(sv[w], si[w], bv, bi)) {
        bv = sv[w];
        bi = si[w];
      }
  }
}

// Row 0's token handed to the next decode step (see DecodeChain): the step's
// token and position advance in device memory, and the token goes to the
// next slot of the host ring as one system-scope store (straight to host
// memory, visible to the polling host without a copy or a stream sync).
__device__ __forceinline__ void chain_publish(const DecodeChain& ch, uint32_t tok) {
  int* io = ch.io;
  io[0] = static_cast<int>(tok);
  io[1] += 1;
  const unsigned k = static_cast<unsigned>(io[3]);
  io[3] = static_cast<int>(k + 1);
  __hip_atomic_store(ch.ring + (k & ch.mask), tok, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// one workgroup per row; rows of a multiple of 8 values at 16-byte
// alignment are read 8 values per load, 8 loads in flight per thread
__global__ void __launch_bounds__(kArgThreads)
    argmax_kernel(const uint16_t* __restrict__ x, int64_t n, uint32_t* __restrict__ out, const DecodeChain ch) {
  const uint16_t* xr = x + static_cast<int64_t>(blockIdx.x) * n;
  float bv = -INFINITY;
  uint32_t bi = 0xffffffffu;
  if (n % 8 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0) {
    const uint4* xv = reinterpret_cast<const uint4*>(xr);
    const int64_t nv = n / 8;
    constexpr int B = 8;
    for (int64_t j0 = threadIdx.x; j0 < nv; j0 += static_cast<int64_t>(kArgThreads) * B) {
      uint4 d[B];
#pragma unroll
      for (int u = 0; u < B; u++) {
        const int64_t j = j0 + static_cast<int64_t>(u) * kArgThreads;
        d[u] = j < nv ? xv[j] : make_uint4(0xff80ff80u, 0xff80ff80u, 0xff80ff80u, 0xff80ff80u);  // -inf
      }
#pragma unroll
      for (int u = 0; u < B; u++) {
        const uint32_t w[4] = {d[u].x, d[u].y, d[u].z, d[u].w};
        const uint32_t base = static_cast<uint32_t>((j0 + static_cast<int64_t>(u) * kArgThreads) * 8);
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const float v = bf2f((w[e >> 1] >> (16 * (e & 1))) & 0xffffu);
          if (better(v, base + e, bv, bi)) {
            bv = v;
            bi = base + e;
          }
        }
      }
    }
  } else {
    for (int64_t i = threadIdx.x; i < n; i += kArgThreads) {
      const float v = bf2f(xr[i]);
      if (better(v, static_cast<uint32_t>(i), bv, bi)) {
        bv = v;
        bi = static_cast<uint32_t>(i);
      }
    }
  }
  block_best(bv, bi);
  // all -inf / NaN rows: index 0
  if (threadIdx.x == 0) {
    const uint32_t tok = bi == 0xffffffffu ? 0u : bi;
    out[blockIdx.x] = tok;
    if (ch.io != nullptr && blockIdx.x == 0) chain_publish(ch, tok);
  }
}

// one workgroup per row over the per-workgroup partials (value bits, index)
// of the GEMV epilogue
__global__ void __launch_bounds__(kArgThreads)
    argmax_partials_kernel(const uint2* __restrict__ part, int nblk, uint32_t* __restrict__ out,
                           const DecodeChain ch) {
  const uint2* pr = part + static_cast<int64_t>(blockIdx.x) * nblk;
  float bv = -INFINITY;
  uint32_t bi = 0xffffffffu;
  constexpr int B = 8;
  for (int j0 = threadIdx.x; j0 < nblk; j0 += kArgThreads * B) {
    uint2 d[B];
#pragma unroll
    for (int u = 0; u < B; u++) {
      const int j = j0 + u * kArgThreads;
      d[u] = j < nblk ? pr[j] : make_uint2(0xff800000u, 0xffffffffu);
    }
#pragma unroll
    for (int u = 0; u < B; u++) {
      const float v = __uint_as_float(d[u].x);
      if (better(v, d[u].y, bv, bi)) {
        bv = v;
        bi = d[u].y;
      }
    }
  }
  block_best(bv, bi);
  if (threadIdx.x == 0) {
    const uint32_t tok = bi == 0xffffffffu ? 0u : bi;
    out[blockIdx.x] = tok;
    if (ch.io != nullptr && blockIdx.x == 0) chain_publish(ch, tok);
  }
}

__global__ void __launch_bounds__(256)
    silu_mul_kernel(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u, uint16_t* __restrict__ y,
                    int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const float gv = bf2f(g[i]);
  const float sg = round_bf(1.0f / (1.0f + expf(-gv)));
  const float a = round_bf(gv * sg);
  y[i] = f2bf(a * bf2f(u[i]));
}

__global__ void __launch_bounds__(256)
    add_kernel(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b, uint16_t* y, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) y[i] = f2bf(bf2f(a[i]) + bf2f(b[i]));
}

// dst[i] = src[i] (token ids u32 -> i32 for the embedding gather)
__global__ void tokens_to_ids_kernel(const uint32_t* __restrict__ src, int32_t* __restrict__ dst, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = static_cast<int32_t>(src[i]);
}

}  // namespace

int launch_argmax(const uint16_t* x, int64_t rows, int64_t n, uint32_t* out, hipStream_t stream,
                  const DecodeChain* chain) {
  if (rows <= 0) return BMX_OK;
  if (n <= 0 || n > UINT32_MAX) return set_error(BMX_E_SHAPE, "argmax: n=%lld", (long long)n);
  if (rows > INT32_MAX) return set_error(BMX_E_SHAPE, "argmax: rows=%lld", (long long)rows);
  if (chain && (rows != 1 || !chain->io || !chain->ring)) return set_error(BMX_E_ARG, "argmax: chained hand-off of %lld rows", (long long)rows);
  const DecodeChain ch = chain ? *chain : DecodeChain{};
  hipLaunchKernelGGL(argmax_kernel, dim3(static_cast<unsigned>(rows)), dim3(kArgThreads), 0, stream, x, n, out, ch);
  return check_launch("argmax");
}

int launch_argmax_partials(const uint2* part, int rows, int nblk, uint32_t* out, hipStream_t stream,
                           const DecodeChain* chain) {
  if (rows <= 0) return BMX_OK;
  if (nblk <= 0) return set_error(BMX_E_SHAPE, "argmax partials: %d per row", nblk);
  if (chain && (rows != 1 || !chain->io || !chain->ring)) return set_error(BMX_E_ARG, "argmax: chained hand-off of %d rows", rows);
  const DecodeChain ch = chain ? *chain : DecodeChain{};
  hipLaunchKernelGGL(argmax_partials_kernel, dim3(rows), dim3(kArgThreads), 0, stream, part, nblk, out, ch);
  return check_launch("argmax_partials");
}

int launch_silu_mul(const uint16_t* g, const uint16_t* u, uint16_t* y, int64_t n, hipStream_t stream) {
  if (n <= 0) return BMX_OK;
  hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream, g, u, y, n);
  return check_launch("silu_mul");
}

int launch_add(const uint16_t* a, const uint16_t* b, uint16_t* y, int64_t n, hipStream_t stream) {
  if (n <= 0) return BMX_OK;
  hipLaunchKernelGGL(add_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream, a, b, y, n);
  return check_launch("add");
}

int launch_tokens_to_ids(const uint32_t* src, int32_t* dst, int n, hipStream_t stream) {
  if (n <= 0) return BMX_OK;
  hipLaunchKernelGGL(tokens_to_ids_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, src, dst, n);
  return check_launch("tokens_to_ids");
}

}  // namespace bmx

using namespace bmx;

extern "C" int bmx_argmax_rows(const bmx_bf16* x, int64_t rows, int64_t n, uint32_t* out, void* stream) {
  if (!x || !out) return set_error(BMX_E_ARG, "argmax: null pointer");
  return launch_argmax(x, rows, n, out, as_stream(stream));
}

extern "C" int bmx_silu_mul(const bmx_bf16* gate, const bmx_bf16* up, bmx_bf16* y, int64_t n, void* stream) {
  if (!gate || !up || !y) return set_error(BMX_E_ARG, "silu_mul: null pointer");
  return launch_silu_mul(gate, up, y, n, as_stream(stream));
}

extern "C" int bmx_add(const bmx_bf16* a, const bmx_bf16* b, bmx_bf16* y, int64_t n, void* stream) {
  if (!a || !b || !y) return set_error(BMX_E_ARG, "add: null pointer");
  return launch_add(a, b, y, n, as_stream(stream));
}
