// Dequantization of MLX affine 4-bit gs64 weights:
//   out[n,k] = bf16(s[n,k/64] * q[n,k] + b[n,k/64])
// (s*q is exact in fp32, so the only rounding is the final bf16 one.)
// Semantics restated: mlx_rs::ops::dequantize as used by QEmbedding::lookup
// (crates/base-mlx-core/src/model/qwen3.rs:67-76).
#include "bmx_device.h"

namespace bmx {
namespace {

// One thread expands one packed word (8 values) into one 16-byte store.
__device__ __forceinline__ uint4 dequant_word(uint32_t wd, float s, float b) {
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float lo = s * static_cast<float>((wd >> (8 * i)) & 0xfu) + b;
    const float hi = s * static_cast<float>((wd >> (8 * i + 4)) & 0xfu) + b;
    o[i] = static_cast<uint32_t>(f2bf(lo)) | (static_cast<uint32_t>(f2bf(hi)) << 16);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

__global__ void __launch_bounds__(256)
    dequant_kernel(const uint32_t* __restrict__ w, const uint16_t* __restrict__ s,
                   const uint16_t* __restrict__ b, uint16_t* __restrict__ out, int64_t N, int64_t K) {
  const int64_t words = N * (K / 8);
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= words) return;
  const int64_t n = i / (K / 8), kw = i - n * (K / 8);
  const int64_t g = n * (K / 64) + kw / 8;
  *reinterpret_cast<uint4*>(out + i * 8) = dequant_word(w[i], bf2f(s[g]), bf2f(b[g]));
}

__global__ void __launch_bounds__(256)
    dequant_gather_kernel(const int32_t* __restrict__ ids, int64_t rows, const uint32_t* __restrict__ w,
                          const uint16_t* __restrict__ s, const uint16_t* __restrict__ b,
                          uint16_t* __restrict__ out, int64_t K) {
  const int64_t m = blockIdx.y;
  const int64_t kw = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (kw >= K / 8) return;
  const int32_t id = ids[m];
  uint4 v = make_uint4(0, 0, 0, 0);
  if (id >= 0 && id < rows) {
    const int64_t g = static_cast<int64_t>(id) * (K / 64) + kw / 8;
    v = dequant_word(w[static_cast<int64_t>(id) * (K / 8) + kw], bf2f(s[g]), bf2f(b[g]));
  }
  *reinterpret_cast<uint4*>(out + m * K + kw * 8) = v;
}

}  // namespace

int launch_dequant_gather(const int32_t* ids, int64_t M, int64_t rows, const uint32_t* w, const uint16_t* s,
                          const uint16_t* b, uint16_t* out, int64_t K, hipStream_t stream) {
  if (M <= 0) return BMX_OK;
  if (M > 65535) return set_error(BMX_E_SHAPE, "dequant_gather: M=%lld > 65535", (long long)M);
  if (!aligned(out, 16)) return set_error(BMX_E_ALIGN, "dequant_gather: out not 16-byte aligned");
  const int64_t words = K / 8;
  hipLaunchKernelGGL(dequant_gather_kernel, dim3(static_cast<unsigned>((words + 255) / 256), static_cast<unsigned>(M)),
                     dim3(256), 0, stream, ids, rows, w, s, b, out, K);
  return check_launch("dequant_gather");
}

}  // namespace bmx

using namespace bmx;

static int check_format(const char* what, int64_t K, int group_size, int bits) {
  if (bits != 4 || group_size != 64)
    return set_error(BMX_E_UNSUPPORTED, "%s: only bits=4, group_size=64 (got %d, %d)", what, bits, group_size);
  if (K <= 0 || K % 64) return set_error(BMX_E_SHAPE, "%s: K=%lld not a positive multiple of 64", what, (long long)K);
  return BMX_OK;
}

extern "C" int bmx_dequantize_affine(const uint32_t* w, const bmx_bf16* scales, const bmx_bf16* biases,
                                     bmx_bf16* out, int64_t N, int64_t K, int group_size, int bits,
                                     void* stream) {
  if (int rc = check_format("dequantize", K, group_size, bits)) return rc;
  if (!w || !scales || !biases || !out) return set_error(BMX_E_ARG, "dequantize: null pointer");
  if (N <= 0) return BMX_OK;
  if (!aligned(out, 16)) return set_error(BMX_E_ALIGN, "dequantize: out not 16-byte aligned");
  const int64_t words = N * (K / 8);
  hipLaunchKernelGGL(dequant_kernel, dim3(static_cast<unsigned>((words + 255) / 256)), dim3(256), 0,
                     as_stream(stream), w, scales, biases, out, N, K);
  return check_launch("dequantize");
}

extern "C" int bmx_dequant_gather(const int32_t* ids, int64_t M, int64_t rows, const uint32_t* w,
                                  const bmx_bf16* scales, const bmx_bf16* biases, bmx_bf16* out, int64_t K,
                                  int group_size, int bits, void* stream) {
  if (int rc = check_format("dequant_gather", K, group_size, bits)) return rc;
  if (!ids || !w || !scales || !biases || !out) return set_error(BMX_E_ARG, "dequant_gather: null pointer");
  return launch_dequant_gather(ids, M, rows, w, scales, biases, out, K, as_stream(stream));
}
