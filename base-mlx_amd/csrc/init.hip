// Seeded random initialisation on device, bit-identical to the CPU
// generator used to check it: approx-normal deviates (centred sum of four
// 16-bit uniforms of a splitmix64 counter hash, scaled by c) and the MLX
// affine 4-bit gs64 quantizer (s = (max-min)/15, q = rne((w-min)/s) clipped
// to [0,15], b = min).  Every float operation is written with an explicit
// _rn intrinsic so no contraction can change a bit.
#include "bmx_device.h"

namespace bmx {
namespace {

__device__ __forceinline__ float normal_at(uint64_t mseed, uint64_t idx, float c) {
  return __fmul_rn(static_cast<float>(irwin4(rand64_mixed(mseed, idx))), c);
}

// One thread quantizes one 64-wide group.  The affine formula is evaluated
// exactly on the integer deviates t (element = t * c):
//   q = round_half_even(15 (t - tmin) / (tmax - tmin)),
//   s = bf16(float((tmax - tmin) * c * (1/15))) in double, b = bf16(tmin * c).
__global__ void __launch_bounds__(256)
    init_qlinear_kernel(uint64_t mseed, int64_t N, int64_t K, float c, uint32_t* __restrict__ w,
                        uint16_t* __restrict__ s, uint16_t* __restrict__ b) {
  const int64_t G = K / 64;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= N * G) return;
  const int64_t n = gid / G, g = gid - n * G;
  const uint64_t base = static_cast<uint64_t>(n * K + g * 64);
  int32_t t[64];
#pragma unroll
  for (int i = 0; i < 64; i++) t[i] = irwin4(rand64_mixed(mseed, base + i));
  int32_t hi = t[0], lo = t[0];
#pragma unroll
  for (int i = 1; i < 64; i++) {
    hi = t[i] > hi ? t[i] : hi;
    lo = t[i] < lo ? t[i] : lo;
  }
  const int32_t den = hi - lo;
  uint32_t words[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    uint32_t wd = 0;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      int32_t q = 0;
      if (den > 0) {
        const int32_t num = 15 * (t[j * 8 + e] - lo);
        q = num / den;
        const int32_t r = num - q * den;
        if (2 * r > den || (2 * r == den && (q & 1))) q++;
      }
      wd |= static_cast<uint32_t>(q) << (4 * e);
    }
    words[j] = wd;
  }
  const double sd = den > 0 ? __dmul_rn(__dmul_rn(static_cast<double>(den), static_cast<double>(c)), 1.0 / 15.0)
                            : 1e-7;
  uint4* wp = reinterpret_cast<uint4*>(w + n * (K / 8) + g * 8);
  wp[0] = make_uint4(words[0], words[1], words[2], words[3]);
  wp[1] = make_uint4(words[4], words[5], words[6], words[7]);
  s[n * G + g] = f2bf_int(static_cast<float>(sd));  // double -> float -> bf16, two roundings
  b[n * G + g] = f2bf(__fmul_rn(static_cast<float>(lo), c));
}

__global__ void __launch_bounds__(256)
    fill_normal_bf16_kernel(uint64_t mseed, int64_t n, float c, uint16_t* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = f2bf(normal_at(mseed, static_cast<uint64_t>(i), c));
}

// KV positions [0, seq_len) of every (layer, k|v, head) row get approx
// N(0,1) values at counter (row * cap + t) * hd + d.
__global__ void __launch_bounds__(256)
    fill_kv_kernel(uint16_t* __restrict__ data, int64_t rows, int cap, int hd, int seq_len, uint64_t mseed, float c) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t per_row = static_cast<int64_t>(seq_len) * hd;
  if (i >= rows * per_row) return;
  const int64_t r = i / per_row, rem = i - r * per_row;
  const int64_t idx = r * cap * hd + rem;
  data[idx] = f2bf(normal_at(mseed, static_cast<uint64_t>(idx), c));
}

}  // namespace

uint64_t host_mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

int launch_init_qlinear(uint64_t seed, int64_t N, int64_t K, float c, uint32_t* w, uint16_t* s, uint16_t* b,
                        hipStream_t stream) {
  if (N <= 0 || K <= 0 || K % 64) return set_error(BMX_E_SHAPE, "init_qlinear: N=%lld K=%lld", (long long)N, (long long)K);
  if (!aligned(w, 16)) return set_error(BMX_E_ALIGN, "init_qlinear: W not 16-byte aligned");
  const int64_t groups = N * (K / 64);
  hipLaunchKernelGGL(init_qlinear_kernel, dim3(static_cast<unsigned>((groups + 255) / 256)), dim3(256), 0, stream,
                     host_mix64(seed), N, K, c, w, s, b);
  return check_launch("init_qlinear");
}

int launch_fill_kv_synthetic(uint16_t* data, int64_t rows, int cap, int hd, int seq_len, uint64_t seed, float c,
                             hipStream_t stream) {
  const int64_t n = rows * seq_len * hd;
  if (n <= 0) return BMX_OK;
  hipLaunchKernelGGL(fill_kv_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream, data, rows,
                     cap, hd, seq_len, host_mix64(seed), c);
  return check_launch("fill_kv");
}

}  // namespace bmx

using namespace bmx;

extern "C" int bmx_init_qlinear(uint64_t seed, int64_t N, int64_t K, float c, uint32_t* w,
                                bmx_bf16* scales, bmx_bf16* biases, void* stream) {
  if (!w || !scales || !biases) return set_error(BMX_E_ARG, "init_qlinear: null pointer");
  return launch_init_qlinear(seed, N, K, c, w, scales, biases, as_stream(stream));
}

extern "C" int bmx_fill_normal_bf16(uint64_t seed, int64_t n, float c, bmx_bf16* out, void* stream) {
  if (!out) return set_error(BMX_E_ARG, "fill_normal_bf16: null pointer");
  if (n <= 0) return BMX_OK;
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(fill_normal_bf16_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     as_stream(stream), host_mix64(seed), n, c, out);
  return check_launch("fill_normal_bf16");
}
