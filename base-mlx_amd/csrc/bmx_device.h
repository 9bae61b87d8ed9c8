// Device-side helpers shared by the bmx HIP kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bmx_internal.h"

namespace bmx {

// bf16 is carried as raw uint16_t bits everywhere.
__device__ __forceinline__ float bf2f(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
// f32 -> bf16, round to nearest even; NaN stays a (quiet) NaN.  One
// v_cvt_pk_bf16_f32 (gfx950), and conversions of neighbouring values pair up.
__device__ __forceinline__ uint16_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }
// The same rounding in integer arithmetic, for a float that must first exist
// as a float: the compiler folds double -> float -> bf16 conversions into one
// (single-rounding) conversion, which differs in rare ties.
__device__ __forceinline__ uint16_t f2bf_int(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

// acc + a.lo*b.lo + a.hi*b.hi with bf16 operands and an fp32 accumulator
// (v_dot2c_f32_bf16).  bf16 x bf16 products are exact in fp32.
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), acc, false);
}

template <typename T>
__device__ __forceinline__ T wave_sum_xor(T v, int width) {
  for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// The nibble-pair mask 0x000F000F and the bf16 magic 0x43004300 held in
// registers the compiler cannot fold back into literals: a gfx9 VOP3
// instruction takes no literal operand, so with literals each pair would
// unpack as an and plus an or; with both in VGPRs it is one v_and_or_b32.
// A kernel makes them once and passes them to word_dot.
struct NibbleK {
  uint32_t mask, magic;
};
__device__ __forceinline__ NibbleK nibble_consts() {
  NibbleK k{0x000f000fu, 0x43004300u};
  asm volatile("" : "+v"(k.mask), "+v"(k.magic));
  return k;
}

// Dot of one packed word (8 nibbles q_0..q_7) with its pair-permuted x
// (permute_pairs: (x_e, x_{e+4}) per word), +128 bias on every q:
// (w >> 4j & 0x000F000F) | 0x43004300 is the bf16 pair (128 + q_j, 128 +
// q_{j+4}), fed straight to v_dot2c_f32_bf16.
__device__ __forceinline__ float word_dot(uint32_t w, uint4 xp, float acc, const NibbleK& k) {
  acc = dot2_bf16((w & k.mask) | k.magic, xp.x, acc);
  acc = dot2_bf16(((w >> 4) & k.mask) | k.magic, xp.y, acc);
  acc = dot2_bf16(((w >> 8) & k.mask) | k.magic, xp.z, acc);
  acc = dot2_bf16(((w >> 12) & k.mask) | k.magic, xp.w, acc);
  return acc;
}

// ---- Per-row arithmetic of the GEMV kernels (qmv.hip) --------------------
// Every GEMV kernel of 1..8 rows of x (single-phase, persistent, phased)
// computes each row with exactly these operations, in this order, written
// with explicit fused multiply-adds so that no kernel's code generation can
// contract them differently.  With the same lanes per weight row (a
// function of N and K only) and the same chunk -> lane assignment (chunk c
// to lane c mod S, in increasing c), a row's output is therefore the same
// bits whatever the number of rows of x in the launch: a speculative-verify
// row equals the single-token decode of that position.

// Sum of squares of 8 bf16 values (one 16-byte unit of x), added to ss.
__device__ __forceinline__ float gemv_ss_unit(uint4 d, float ss) {
  const uint32_t v[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const float lo = bf2f(v[q] & 0xffffu), hi = bf2f(v[q] >> 16);
    ss = __builtin_fmaf(lo, lo, ss);
    ss = __builtin_fmaf(hi, hi, ss);
  }
  return ss;
}
// 1 / rms from the four waves' sums of squares (fast::rms_norm,
// crates/base-mlx-core/src/model/qwen3.rs:50-55)
__device__ __forceinline__ float gemv_norm_inv(float r0, float r1, float r2, float r3, int K, float eps) {
  return 1.0f / sqrtf((((r0 + r1) + r2) + r3) / static_cast<float>(K) + eps);
}
// h = w * bf16(x * inv), 8 values, bf16 result
__device__ __forceinline__ uint4 gemv_norm_unit(uint4 d, uint4 wn, float inv) {
  uint32_t dv[4] = {d.x, d.y, d.z, d.w};
  const uint32_t wq[4] = {wn.x, wn.y, wn.z, wn.w};
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const float lo = bf2f(wq[q] & 0xffffu) * round_bf(bf2f(dv[q] & 0xffffu) * inv);
    const float hi = bf2f(wq[q] >> 16) * round_bf(bf2f(dv[q] >> 16) * inv);
    dv[q] = static_cast<uint32_t>(f2bf(lo)) | (static_cast<uint32_t>(f2bf(hi)) << 16);
  }
  return make_uint4(dv[0], dv[1], dv[2], dv[3]);
}
// Sum of 8 bf16 values (a quarter of a chunk's x sum), in a fixed order
__device__ __forceinline__ float gemv_unit_sum(uint4 d) {
  const uint32_t dv[4] = {d.x, d.y, d.z, d.w};
  float part = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; q++) part += bf2f(dv[q] & 0xffffu) + bf2f(dv[q] >> 16);
  return part;
}
// s and b - 128 s of a group from its interleaved (s | b << 16) word
__device__ __forceinline__ void gemv_sb(uint32_t sb, float& sv, float& bb) {
  sv = bf2f(sb & 0xffffu);
  bb = __builtin_fmaf(-128.0f, sv, bf2f(sb >> 16));
}
// One 16-byte chunk (32 nibbles, half a group) of one weight row against
// the pair-permuted x chunk (x0..x3) with chunk sum sx:
//   acc += s * D + (b - 128 s) * sx,   D = sum (128 + q) x  (two dot2 chains)
__device__ __forceinline__ float gemv_chunk(uint4 w, uint4 x0, uint4 x1, uint4 x2, uint4 x3, float sv, float bb,
                                            float sx, float acc, const NibbleK& nk) {
  float d0 = 0.0f, d1 = 0.0f;
  d0 = word_dot(w.x, x0, d0, nk);
  d1 = word_dot(w.y, x1, d1, nk);
  d0 = word_dot(w.z, x2, d0, nk);
  d1 = word_dot(w.w, x3, d1, nk);
  acc = __builtin_fmaf(sv, d0 + d1, acc);
  return __builtin_fmaf(bb, sx, acc);
}

// DPP lane moves within 16-lane rows (gfx9 dpp_ctrl encodings):
// quad_perm [1,0,3,2] = 0xB1 (lane ^ 1), quad_perm [2,3,0,1] = 0x4E
// (lane ^ 2), row_ror:4 = 0x124 and row_ror:8 = 0x128 (rotations by 4 and 8
// inside the row; the reductions below do not depend on the direction).
// Every source lane lies inside its row, so no lane reads a disabled or
// out-of-row source.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// max / sum over each 16-lane row; every lane of the row gets the result
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x124>(v));
  return fmaxf(v, dpp_f32<0x128>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f32<0xB1>(v);
  v += dpp_f32<0x4E>(v);
  v += dpp_f32<0x124>(v);
  return v + dpp_f32<0x128>(v);
}

// Sum over groups of S consecutive lanes (S = 8, 16, 32 or 64); every lane
// of a group gets the group's sum.  Inside 16-lane rows with DPP: quad_perm
// [1,0,3,2] (0xB1), quad_perm [2,3,0,1] (0x4E), row_half_mirror (0x141:
// lane i <-> 7 - i within 8), row_mirror (0x140: lane i <-> 15 - i).
// v + (v of lane ^ 16) and v + (v of lane ^ 32) through the gfx950 lane
// swaps (v_permlane16_swap: odd 16-lane rows of one operand against even
// rows of the other; v_permlane32_swap: the two 32-lane halves), one VALU
// step each instead of a round trip through the LDS crossbar.  With both
// operands v, the two results hold the pair's values in a fixed order, and
// since a + b == b + a exactly, every lane gets the bits of the shuffle form.
__device__ __forceinline__ float add_xor16(float v) {
  const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
__device__ __forceinline__ float add_xor32(float v) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
__device__ __forceinline__ float max_xor16(float v) {
  const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float max_xor32(float v) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float lanes_sum(float v, int S) {
  v += dpp_f32<0xB1>(v);
  v += dpp_f32<0x4E>(v);
  v += dpp_f32<0x141>(v);
  if (S >= 16) v += dpp_f32<0x140>(v);
  if (S >= 32) v = add_xor16(v);
  if (S >= 64) v = add_xor32(v);
  return v;
}

// Per-head RMSNorm (fp32 inside, bf16 result) followed by rotate-half RoPE
// at angle pos * freq, for one head row of 128 held by a whole wave: lane
// holds dims lane and lane + 64 (values a, b and norm weights wa, wb on
// entry; the rotated bf16 pair on return).  QK-norm and rope of
// Qwen3::forward_internal (crates/base-mlx-core/src/model/qwen3.rs:392-413).
// Every kernel that norms and rotates q or k calls this, so they agree bit
// for bit.
// the same with the rotation's cos / sin given (they depend on the position
// and lane only, so a wave over several heads of one token computes them once)
__device__ __forceinline__ void qk_norm_rope_lane_cs(float a, float b, float wa, float wb, float c, float s,
                                                     float eps, uint16_t& o1, uint16_t& o2) {
  // the fused multiply-adds are written out, so every place this function
  // is inlined rounds the same way
  // the row's sum of squares: a symmetric butterfly (DPP inside 16-lane
  // rows, lane swaps across them), every lane the same bits
  const float ss = lanes_sum(__builtin_fmaf(a, a, __fmul_rn(b, b)), 64);
  const float inv = 1.0f / sqrtf(ss / 128.0f + eps);
  const float na = bf2f(f2bf(wa * round_bf(a * inv)));
  const float nb = bf2f(f2bf(wb * round_bf(b * inv)));
  o1 = f2bf(__builtin_fmaf(na, c, -__fmul_rn(nb, s)));
  o2 = f2bf(__builtin_fmaf(nb, c, __fmul_rn(na, s)));
}
__device__ __forceinline__ void rope_cs(float freq, float pos, float& c, float& s) {
  const float ang = pos * freq;
  c = cosf(ang);
  s = sinf(ang);
}
__device__ __forceinline__ void qk_norm_rope_lane(float a, float b, float wa, float wb, float freq, float pos,
                                                  float eps, uint16_t& o1, uint16_t& o2) {
  float c, s;
  rope_cs(freq, pos, c, s);
  qk_norm_rope_lane_cs(a, b, wa, wb, c, s, eps, o1, o2);
}

// floor(a / b) for 0 <= a < 2^20 and b >= 1, from rcp_b = 1.0f / b (correctly
// rounded): (a + 0.5) / b lies at least 0.5 / b from an integer, while the
// product's relative error is below 2^-22, i.e. below (a + 0.5) / b * 2^-22
// < 0.5 / b whenever a + 0.5 < 2^21.
__device__ __forceinline__ int udiv_small(int a, float rcp_b) {
  return static_cast<int>((static_cast<float>(a) + 0.5f) * rcp_b);
}

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

// Same counter-based generator as the oracle (splitmix64 finalizer).
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__device__ __forceinline__ uint64_t rand64_mixed(uint64_t mixed_seed, uint64_t idx) {
  return mix64(mixed_seed + (idx + 1u) * 0x9E3779B97F4A7C15ull);
}
__device__ __forceinline__ int32_t irwin4(uint64_t r) {
  return static_cast<int32_t>((r & 0xffffu) + ((r >> 16) & 0xffffu) +
                              ((r >> 32) & 0xffffu) + ((r >> 48) & 0xffffu)) -
         131070;
}

}  // namespace bmx
