// RMSNorm, RoPE, the fused QK-norm + RoPE + KV-cache write of a Qwen3
// attention block, and the in-place slice update of the KV cache (gfx950).
//
// Semantics restated (MLX upstream ops called by the reference):
//   fast::rms_norm (crates/base-mlx-core/src/model/qwen3.rs:44-55):
//     y = w * bf16(x * rsqrt(mean(x^2) + eps)), fp32 internally
//   fast::rope(x, dims=D, traditional=false, base=theta, scale=1, offset)
//     (qwen3.rs:407-413): rotate-half; for i < D/2,
//     angle = (offset + t) * theta^(-i/(D/2)),
//     y_i = x_i cos - x_{i+D/2} sin,  y_{i+D/2} = x_i sin + x_{i+D/2} cos
//   mlx_ext::slice_update (crates/base-mlx-core/src/mlx_ext.rs:21-64):
//     numpy src[start:stop:strides] = update, in place.
// The inverse-frequency table theta^(-i/(D/2)) is evaluated on the host in
// double, rounded to float, and passed by value in the kernel arguments, so
// kernels are graph-capturable and use exactly the CPU's table.
#include <math.h>
#include <string.h>

#include "bmx_device.h"

namespace bmx {

RopeTable make_rope_table(int D, float theta) {
  RopeTable t;
  memset(&t, 0, sizeof(t));
  const int half = D / 2;
  for (int i = 0; i < half && i < 128; i++) t.inv_freq[i] = static_cast<float>(pow(static_cast<double>(theta), -static_cast<double>(i) / half));
  return t;
}

namespace {

// one wave per row; dim % 8 == 0
__global__ void __launch_bounds__(256)
    rms_norm_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, uint16_t* __restrict__ y,
                    int64_t rows, int dim, float eps) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const uint16_t* xr = x + r * dim;
  if (dim <= 4096) {
    // the row (at most 8 chunks of 8 per lane) and the weight in registers:
    // x read once, every load in flight together; the same operations in
    // the same order as the loops below
    uint4 d[8], wn[8];
#pragma unroll
    for (int c = 0; c < 8; c++) {
      const int k = lane * 8 + 512 * c;
      if (k < dim) {
        d[c] = *reinterpret_cast<const uint4*>(xr + k);
        wn[c] = *reinterpret_cast<const uint4*>(w + k);
      }
    }
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; c++) {
      if (lane * 8 + 512 * c >= dim) break;
      const uint32_t v[4] = {d[c].x, d[c].y, d[c].z, d[c].w};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float lo = bf2f(v[i] & 0xffffu), hi = bf2f(v[i] >> 16);
        ss += lo * lo + hi * hi;
      }
    }
    ss = wave_sum_xor(ss, 64);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(dim) + eps);
#pragma unroll
    for (int c = 0; c < 8; c++) {
      const int k = lane * 8 + 512 * c;
      if (k >= dim) break;
      const uint32_t v[4] = {d[c].x, d[c].y, d[c].z, d[c].w}, wv[4] = {wn[c].x, wn[c].y, wn[c].z, wn[c].w};
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float lo = bf2f(wv[i] & 0xffffu) * round_bf(bf2f(v[i] & 0xffffu) * inv);
        const float hi = bf2f(wv[i] >> 16) * round_bf(bf2f(v[i] >> 16) * inv);
        o[i] = static_cast<uint32_t>(f2bf(lo)) | (static_cast<uint32_t>(f2bf(hi)) << 16);
      }
      *reinterpret_cast<uint4*>(y + r * dim + k) = make_uint4(o[0], o[1], o[2], o[3]);
    }
    return;
  }
  float ss = 0.0f;
  for (int k = lane * 8; k < dim; k += 512) {
    const uint4 d = *reinterpret_cast<const uint4*>(xr + k);
    const uint32_t v[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float lo = bf2f(v[i] & 0xffffu), hi = bf2f(v[i] >> 16);
      ss += lo * lo + hi * hi;
    }
  }
  ss = wave_sum_xor(ss, 64);
  const float inv = 1.0f / sqrtf(ss / static_cast<float>(dim) + eps);
  for (int k = lane * 8; k < dim; k += 512) {
    const uint4 d = *reinterpret_cast<const uint4*>(xr + k);
    const uint4 wn = *reinterpret_cast<const uint4*>(w + k);
    const uint32_t v[4] = {d.x, d.y, d.z, d.w}, wv[4] = {wn.x, wn.y, wn.z, wn.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float lo = bf2f(wv[i] & 0xffffu) * round_bf(bf2f(v[i] & 0xffffu) * inv);
      const float hi = bf2f(wv[i] >> 16) * round_bf(bf2f(v[i] >> 16) * inv);
      o[i] = static_cast<uint32_t>(f2bf(lo)) | (static_cast<uint32_t>(f2bf(hi)) << 16);
    }
    *reinterpret_cast<uint4*>(y + r * dim + k) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

__device__ __forceinline__ void rope_pair(float a, float b, float ang, float& o1, float& o2) {
  const float c = cosf(ang), s = sinf(ang);
  o1 = a * c - b * s;
  o2 = a * s + b * c;
}

// x, y: [H, T, D] with D = 2 * half, half <= 64 * PL; one wave per (h, t)
__global__ void __launch_bounds__(256)
    rope_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y, int64_t HT, int T, int D,
                int64_t offset, RopeTable tab) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= HT) return;
  const int t = static_cast<int>(row % T);
  const int half = D / 2;
  const float pos = static_cast<float>(offset + t);
  const uint16_t* xr = x + row * D;
  uint16_t* yr = y + row * D;
  for (int i = lane; i < half; i += 64) {
    float o1, o2;
    rope_pair(bf2f(xr[i]), bf2f(xr[i + half]), pos * tab.inv_freq[i], o1, o2);
    yr[i] = f2bf(o1);
    yr[i + half] = f2bf(o2);
  }
}

// Fused per-head RMSNorm (QK-norm, qwen3.rs:392-399), RoPE at positions
// offset + t (qwen3.rs:407-413), KV write at [offset, offset + M)
// (qwen3.rs:431-489), head_dim 128.  One wave per (token, group of up to
// kQkHeads q heads or kv heads): the rotation's cos / sin depend on the
// token and the lane only and are computed once per wave; every head's rows
// are loaded before any arithmetic.  Lane i holds the rotate-half pair
// (i, i + 64) of each head (the lane function the decode attention's
// prologue uses too, so both write the same bits).
constexpr int kQkHeads = 8;
struct QkvRopeParams {
  const uint16_t* q;  // [M, Hq*128] (qkv projection output rows)
  const uint16_t* k;  // [M, Hkv*128]
  const uint16_t* v;  // [M, Hkv*128]
  const uint16_t* q_norm;
  const uint16_t* k_norm;
  uint16_t* q_out;    // [Hq, M, 128]
  uint16_t* k_cache;  // [Hkv, cap, 128] of this layer
  uint16_t* v_cache;  // [Hkv, cap, 128]
  const int* offset_dev;  // if set, the offset is read here (graph replay)
  int offset;
  int M, Hq, Hkv, cap;
  float eps;
  RopeTable tab;
};

__global__ void __launch_bounds__(256) qk_norm_rope_kv_kernel(const QkvRopeParams p) {
  const int wid = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int qg = (p.Hq + kQkHeads - 1) / kQkHeads, kg = (p.Hkv + kQkHeads - 1) / kQkHeads;
  if (wid >= p.M * (qg + kg)) return;
  const int t = wid / (qg + kg);
  const int g = wid - t * (qg + kg);
  const bool is_q = g < qg;
  const int h0 = (is_q ? g : g - qg) * kQkHeads;
  const int nh = min(kQkHeads, (is_q ? p.Hq : p.Hkv) - h0);
  const int offset = p.offset_dev ? *p.offset_dev : p.offset;
  const uint16_t* src = is_q ? p.q + (static_cast<int64_t>(t) * p.Hq + h0) * 128
                             : p.k + (static_cast<int64_t>(t) * p.Hkv + h0) * 128;
  const uint16_t* nw = is_q ? p.q_norm : p.k_norm;
  uint16_t a[kQkHeads], b[kQkHeads];
#pragma unroll
  for (int i = 0; i < kQkHeads; i++) {
    const int hi = min(i, nh - 1);
    a[i] = src[hi * 128 + lane];
    b[i] = src[hi * 128 + lane + 64];
  }
  const float wa = bf2f(nw[lane]), wb = bf2f(nw[lane + 64]);
  float c, s;
  rope_cs(p.tab.inv_freq[lane], static_cast<float>(offset + t), c, s);
  if (is_q) {
#pragma unroll
    for (int i = 0; i < kQkHeads; i++) {
      if (i >= nh) break;
      uint16_t o1, o2;
      qk_norm_rope_lane_cs(bf2f(a[i]), bf2f(b[i]), wa, wb, c, s, p.eps, o1, o2);
      uint16_t* dst = p.q_out + (static_cast<int64_t>(h0 + i) * p.M + t) * 128;
      dst[lane] = o1;
      dst[lane + 64] = o2;
    }
  } else {
    const uint16_t* vs = p.v + (static_cast<int64_t>(t) * p.Hkv + h0) * 128;
    uint16_t va[kQkHeads], vb[kQkHeads];
#pragma unroll
    for (int i = 0; i < kQkHeads; i++) {
      const int hi = min(i, nh - 1);
      va[i] = vs[hi * 128 + lane];
      vb[i] = vs[hi * 128 + lane + 64];
    }
#pragma unroll
    for (int i = 0; i < kQkHeads; i++) {
      if (i >= nh) break;
      uint16_t o1, o2;
      qk_norm_rope_lane_cs(bf2f(a[i]), bf2f(b[i]), wa, wb, c, s, p.eps, o1, o2);
      const int64_t slot = (static_cast<int64_t>(h0 + i) * p.cap + offset + t) * 128;
      p.k_cache[slot + lane] = o1;
      p.k_cache[slot + lane + 64] = o2;
      p.v_cache[slot + lane] = va[i];
      p.v_cache[slot + lane + 64] = vb[i];
    }
  }
}

struct SliceParams {
  int ndim;
  int64_t ext[8];     // extent of the update along each axis
  int64_t start[8];
  int64_t step[8];    // stride of the slice along each axis
  int64_t sstride[8]; // element stride of src along each axis
  int64_t total;
};

__global__ void __launch_bounds__(256)
    slice_update_kernel(uint16_t* __restrict__ src, const uint16_t* __restrict__ upd, SliceParams sp) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= sp.total) return;
  int64_t rem = i, off = 0;
  for (int d = sp.ndim - 1; d >= 0; d--) {
    const int64_t c = rem % sp.ext[d];
    rem /= sp.ext[d];
    off += (sp.start[d] + c * sp.step[d]) * sp.sstride[d];
  }
  src[off] = upd[i];
}

}  // namespace

int launch_qk_norm_rope_kv(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* q_norm,
                           const uint16_t* k_norm, uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache,
                           int M, int Hq, int Hkv, int D, int cap, int offset, const int* offset_dev, float eps,
                           const RopeTable& tab, hipStream_t stream) {
  if (D != 128) return set_error(BMX_E_UNSUPPORTED, "qk_norm_rope_kv: head_dim must be 128 (got %d)", D);
  if (M <= 0 || Hq <= 0 || Hkv <= 0) return set_error(BMX_E_SHAPE, "qk_norm_rope_kv: bad shape");
  if (!offset_dev && (offset < 0 || offset + M > cap))
    return set_error(BMX_E_KV_CAPACITY, "KV cache exhausted: requested %d positions, max %d", offset + M, cap);
  QkvRopeParams p{q, k, v, q_norm, k_norm, q_out, k_cache, v_cache, offset_dev, offset, M, Hq, Hkv, cap, eps, tab};
  const int waves = M * ((Hq + kQkHeads - 1) / kQkHeads + (Hkv + kQkHeads - 1) / kQkHeads);
  hipLaunchKernelGGL(qk_norm_rope_kv_kernel, dim3((waves + 3) / 4), dim3(256), 0, stream, p);
  return check_launch("qk_norm_rope_kv");
}

namespace {

__global__ void __launch_bounds__(256) rope_cs_kernel(float2* cs, int M, int offset, const int* offset_dev,
                                                      const RopeTable tab) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= static_cast<int64_t>(M) * 64) return;
  const int t = static_cast<int>(e >> 6), i = static_cast<int>(e & 63);
  const int off = offset_dev ? *offset_dev : offset;
  float c, s;
  rope_cs(tab.inv_freq[i], static_cast<float>(off + t), c, s);  // as qk_norm_rope_kv_kernel
  cs[e] = make_float2(c, s);
}

}  // namespace

int launch_rope_cs(float2* cs, int M, int offset, const int* offset_dev, const RopeTable& tab, hipStream_t stream) {
  if (M <= 0) return BMX_OK;
  hipLaunchKernelGGL(rope_cs_kernel, dim3(static_cast<unsigned>((static_cast<int64_t>(M) * 64 + 255) / 256)),
                     dim3(256), 0, stream, cs, M, offset, offset_dev, tab);
  return check_launch("rope_cs");
}

int launch_rms_norm(const uint16_t* x, const uint16_t* w, uint16_t* y, int64_t rows, int dim, float eps,
                    hipStream_t stream) {
  if (rows <= 0) return BMX_OK;
  if (dim <= 0 || dim % 8) return set_error(BMX_E_SHAPE, "rms_norm: dim=%d not a positive multiple of 8", dim);
  if (!aligned(x, 16) || !aligned(w, 16) || !aligned(y, 16))
    return set_error(BMX_E_ALIGN, "rms_norm: pointers must be 16-byte aligned");
  hipLaunchKernelGGL(rms_norm_kernel, dim3(static_cast<unsigned>((rows + 3) / 4)), dim3(256), 0, stream, x, w, y,
                     rows, dim, eps);
  return check_launch("rms_norm");
}

}  // namespace bmx

using namespace bmx;

extern "C" int bmx_rms_norm(const bmx_bf16* x, const bmx_bf16* w, bmx_bf16* y, int64_t rows, int64_t dim, float eps,
                            void* stream) {
  if (!x || !w || !y) return set_error(BMX_E_ARG, "rms_norm: null pointer");
  if (dim > INT32_MAX) return set_error(BMX_E_SHAPE, "rms_norm: dim too large");
  return launch_rms_norm(x, w, y, rows, static_cast<int>(dim), eps, as_stream(stream));
}

extern "C" int bmx_rope(const bmx_bf16* x, bmx_bf16* y, int64_t H, int64_t T, int64_t D, float theta, int64_t offset,
                        void* stream) {
  if (!x || !y) return set_error(BMX_E_ARG, "rope: null pointer");
  if (H <= 0 || T <= 0) return BMX_OK;
  if (D <= 0 || D % 2 || D > 256) return set_error(BMX_E_SHAPE, "rope: dims=%lld must be even and <= 256", (long long)D);
  const RopeTable tab = make_rope_table(static_cast<int>(D), theta);
  const int64_t HT = H * T;
  hipLaunchKernelGGL(rope_kernel, dim3(static_cast<unsigned>((HT + 3) / 4)), dim3(256), 0, as_stream(stream), x, y,
                     HT, static_cast<int>(T), static_cast<int>(D), offset, tab);
  return check_launch("rope");
}

extern "C" int bmx_slice_update(bmx_bf16* src, int ndim, const int64_t* shape, const bmx_bf16* update,
                                const int64_t* start, const int64_t* stop, const int64_t* strides, void* stream) {
  if (!src || !shape || !update || !start || !stop || !strides) return set_error(BMX_E_ARG, "slice_update: null pointer");
  if (ndim <= 0 || ndim > 8) return set_error(BMX_E_ARG, "slice_update: ndim=%d outside 1..8", ndim);
  SliceParams sp{};
  sp.ndim = ndim;
  sp.total = 1;
  for (int d = 0; d < ndim; d++) {
    if (strides[d] <= 0 || start[d] < 0 || stop[d] > shape[d] || shape[d] <= 0)
      return set_error(BMX_E_SHAPE, "slice_update: axis %d slice [%lld:%lld:%lld] outside shape %lld", d,
                       (long long)start[d], (long long)stop[d], (long long)strides[d], (long long)shape[d]);
    sp.ext[d] = stop[d] > start[d] ? (stop[d] - start[d] + strides[d] - 1) / strides[d] : 0;
    sp.start[d] = start[d];
    sp.step[d] = strides[d];
    sp.total *= sp.ext[d];
  }
  sp.sstride[ndim - 1] = 1;
  for (int d = ndim - 2; d >= 0; d--) sp.sstride[d] = sp.sstride[d + 1] * shape[d + 1];
  if (sp.total == 0) return BMX_OK;
  hipLaunchKernelGGL(slice_update_kernel, dim3(static_cast<unsigned>((sp.total + 255) / 256)), dim3(256), 0,
                     as_stream(stream), src, update, sp);
  return check_launch("slice_update");
}

extern "C" int bmx_qk_norm_rope_kv(const bmx_bf16* q, const bmx_bf16* k, const bmx_bf16* v, const bmx_bf16* q_norm,
                                   const bmx_bf16* k_norm, bmx_bf16* q_out, bmx_bf16* k_cache, bmx_bf16* v_cache,
                                   int M, int n_heads, int n_kv_heads, int head_dim, int capacity, int offset,
                                   float eps, float theta, void* stream) {
  if (!q || !k || !v || !q_norm || !k_norm || !q_out || !k_cache || !v_cache)
    return set_error(BMX_E_ARG, "qk_norm_rope_kv: null pointer");
  return launch_qk_norm_rope_kv(q, k, v, q_norm, k_norm, q_out, k_cache, v_cache, M, n_heads, n_kv_heads, head_dim,
                                capacity, offset, nullptr, eps, make_rope_table(head_dim, theta), as_stream(stream));
}
